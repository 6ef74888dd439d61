/*
 * oracle.c — CPU restatement of the reference's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product (elffuss-engine_amd/) never calls it. It shares no code with the
 * product: every function below is restated from the reference's JavaScript
 * and WGSL, cited by file:line under /root/reference/js.
 *
 * Floating point: compiled with -ffp-contract=off so that each f32 product
 * and sum rounds as the reference's separate WGSL operations do.
 *
 * Parity status of each part (how it is pinned is in tests/test_oracle.py):
 *   half/aF16 conversions  pinned (numpy float16, exhaustive f16 -> f32)
 *   dequant, 6 types       pinned (field-level block encoders, cpu.js:62-77
 *                          second statement for Q6_K/Q8_0, grid invariants)
 *   Q8_0 quantizer         pinned (known answers of Math.round, numpy float16)
 *   repack / buffer math   pinned (known answers of repack.js:225-229, round trip)
 *   f64 GEMV, fp16 GEMM    pinned (numpy matmul of the dequantized matrix)
 *   top-k                  pinned (numpy lexsort, hand-made ties, -0 == +0)
 *   CPU path (Q8 activations + integer dot)  pinned to its stated model:
 *                          block fields (|q| <= 127, a +-127 per nonzero block,
 *                          half-step error, s = d * sum q, zero blocks), ties
 *                          away from zero, lossless blocks = f64 within the f32
 *                          combine bound, bits independent of threads and
 *                          chunks. The model itself (the 40-byte block as f32
 *                          d, f32 s, 32 int8; roundf) is the reference's
 *                          compiled WASM, whose C source is not shipped and
 *                          which cannot run here: that literal code stays
 *                          parity unpinned (cpu.js:24-27,350-381).
 */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_Q8_0 8
#define OR_Q2_K 10
#define OR_Q4_K 12
#define OR_Q6_K 14
#define OR_IQ2_XXS 16
#define OR_Q8_0R 264

/* ---- f16 ---------------------------------------------------------------- */

/* deF16 (cpu.js:39-44): sign, exponent, mantissa evaluated in double. */
double or_def16(uint32_t bits) {
  double s = (bits & 0x8000u) ? -1.0 : 1.0;
  int e = (int)((bits >> 10) & 0x1Fu);
  int m = (int)(bits & 0x3FFu);
  if (e == 0) return s * m * ldexp(1.0, -24);
  if (e == 31) return m ? NAN : s * INFINITY;
  return s * (1.0 + m / 1024.0) * ldexp(1.0, e - 15);
}

/* unpack2x16float(...)[0] as used by load_scale (kernels.wgsl.js:85-87): the
 * f16 value as f32 (exact). */
static float hf(const uint8_t *p) { return (float)or_def16((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

/* aF16 (cpu.js:84-99): the double goes through a Float32Array, then to f16
 * with round-to-nearest-even, written after the reference's own steps. */
uint32_t or_af16(double v) {
  float f = (float)v;
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t s = (x >> 16) & 0x8000u, e = (x >> 23) & 0xFFu, m = x & 0x7FFFFFu;
  if (e == 0xFFu) return s | 0x7C00u | (m ? 0x200u : 0u);
  int ee = (int)e - 127 + 15;
  if (ee >= 0x1F) return s | 0x7C00u;
  if (ee <= 0) {
    if (ee < -10) return s;
    uint32_t mm = (m | 0x800000u) >> (1 - ee);
    return s | ((mm + 0x1000u + ((mm >> 13) & 1u) - 1u) >> 13);
  }
  uint32_t r = s | ((uint32_t)ee << 10) | (m >> 13);
  uint32_t resto = m & 0x1FFFu;
  if (resto > 0x1000u || (resto == 0x1000u && (r & 1u))) r++;
  return r;
}

/* ---- geometry (gguf.js:51-64) ------------------------------------------- */
int or_geometry(int type, uint32_t *elems, uint32_t *bytes) {
  switch (type) {
    case OR_Q8_0: case OR_Q8_0R: *elems = 32; *bytes = 34; return 0;
    case OR_Q2_K: *elems = 256; *bytes = 84; return 0;
    case OR_Q4_K: *elems = 256; *bytes = 144; return 0;
    case OR_Q6_K: *elems = 256; *bytes = 210; return 0;
    case OR_IQ2_XXS: *elems = 256; *bytes = 66; return 0;
    default: return -1;
  }
}

/* ---- IQ2_XXS grid (quant-tables.js:34-36,40-105) ------------------------
 * The grid values are loaded by the caller (the test passes the table it
 * checks); byte j of entry e = byte (j&3) of word 2e + (j>>2). */
static uint32_t g_grid[512];
static int g_grid_set = 0;
void or_set_grid(const uint32_t *words512) {
  memcpy(g_grid, words512, sizeof g_grid);
  g_grid_set = 1;
}

/* ---- dequantization: the reference's DECODERS ---------------------------- */

static uint32_t rd32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Q8_0 (kernels.wgsl.js:154-169): f32(int8 q) * d. */
static void deq_q8_0(const uint8_t *b, float *o) {
  float d = hf(b);
  for (int i = 0; i < 32; ++i) o[i] = (float)(int8_t)b[2 + i] * d;
}

/* Q2_K (kernels.wgsl.js:194-222). */
static void deq_q2_k(const uint8_t *b, float *o) {
  float d = hf(b + 80), dmin = hf(b + 82);
  for (int n = 0; n < 2; ++n) {
    const uint8_t *q = b + 16 + 32 * n;
    for (int j = 0; j < 4; ++j) {
      int shift = 2 * j;
      uint32_t sca = b[n * 8 + j * 2], scb = b[n * 8 + j * 2 + 1];
      float dl1 = d * (float)(sca & 0xF), ml1 = dmin * (float)(sca >> 4);
      float dl2 = d * (float)(scb & 0xF), ml2 = dmin * (float)(scb >> 4);
      int obase = n * 128 + j * 32;
      for (int i = 0; i < 16; ++i) {
        o[obase + i] = dl1 * (float)((q[i] >> shift) & 3) - ml1;
        o[obase + 16 + i] = dl2 * (float)((q[16 + i] >> shift) & 3) - ml2;
      }
    }
  }
}

/* SCALE_MIN_K4 (kernels.wgsl.js:94-104). */
static void scale_min_k4(const uint8_t *s, int j, uint32_t *sc, uint32_t *m) {
  if (j < 4) {
    *sc = s[j] & 63u;
    *m = s[j + 4] & 63u;
  } else {
    *sc = (s[j + 4] & 0xFu) | ((uint32_t)(s[j - 4] >> 6) << 4);
    *m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
  }
}

/* Q4_K (kernels.wgsl.js:227-250). */
static void deq_q4_k(const uint8_t *b, float *o) {
  float d = hf(b), dmin = hf(b + 2);
  for (int j = 0; j < 4; ++j) {
    uint32_t sc1, m1, sc2, m2;
    scale_min_k4(b + 4, 2 * j, &sc1, &m1);
    scale_min_k4(b + 4, 2 * j + 1, &sc2, &m2);
    float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
    float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
    const uint8_t *q = b + 16 + 32 * j;
    for (int l = 0; l < 32; ++l) {
      o[64 * j + l] = d1 * (float)(q[l] & 0xF) - mm1;
      o[64 * j + 32 + l] = d2 * (float)(q[l] >> 4) - mm2;
    }
  }
}

/* Q6_K (kernels.wgsl.js:269-330). */
static void deq_q6_k(const uint8_t *b, float *o) {
  float d = hf(b + 208);
  for (int n = 0; n < 2; ++n) {
    const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
    const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
    for (int l = 0; l < 32; ++l) {
      int is = l >> 4;
      float d1 = d * (float)sc[is], d2 = d * (float)sc[is + 2];
      float d3 = d * (float)sc[is + 4], d4 = d * (float)sc[is + 6];
      uint32_t h = qh[l];
      int q1 = (int)((ql[l] & 0xF) | ((h & 3) << 4)) - 32;
      int q2 = (int)((ql[32 + l] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
      int q3 = (int)((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
      int q4 = (int)((ql[32 + l] >> 4) | (((h >> 6) & 3) << 4)) - 32;
      o[128 * n + l] = d1 * (float)q1;
      o[128 * n + 32 + l] = d2 * (float)q2;
      o[128 * n + 64 + l] = d3 * (float)q3;
      o[128 * n + 96 + l] = d4 * (float)q4;
    }
  }
}

/* IQ2_XXS (kernels.wgsl.js:368-396), sign byte = 7 stored bits + even parity. */
static void deq_iq2_xxs(const uint8_t *b, float *o) {
  float d = hf(b);
  for (int ib = 0; ib < 8; ++ib) {
    uint32_t a0 = rd32(b + 2 + 8 * ib), a1 = rd32(b + 6 + 8 * ib);
    float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
    for (int l = 0; l < 4; ++l) {
      uint32_t gi = (a0 >> (8 * l)) & 0xFF;
      uint32_t bits = (a1 >> (7 * l)) & 127;
      uint32_t par = 0;
      for (uint32_t t = bits; t; t >>= 1) par ^= t & 1u;
      uint32_t signs = bits | (par << 7);
      uint32_t g0 = g_grid[gi * 2], g1 = g_grid[gi * 2 + 1];
      for (int j = 0; j < 8; ++j) {
        uint32_t gw = j >= 4 ? g1 : g0;
        float gv = (float)((gw >> ((j & 3) * 8)) & 0xFF);
        float sg = (signs & (1u << j)) ? -1.0f : 1.0f;
        o[ib * 32 + l * 8 + j] = db * gv * sg;
      }
    }
  }
}

/* Q8_0R (kernels.wgsl.js:852-865 with bq_escala/bq_palabra, kernels.bloques.wgsl.js:188-196):
 * quants of block i at bytes [32i, 32i+32), scale at byte 32N + 2i. */
static void deq_q8_0r(const uint8_t *buf, uint32_t n_tensor, uint64_t i, float *o) {
  float d = hf(buf + 32ull * n_tensor + 2 * i);
  const uint8_t *q = buf + 32 * i;
  for (int j = 0; j < 32; ++j) o[j] = (float)(int8_t)q[j] * d;
}

/* Dequantize blocks [0, n_blocks). n_tensor is only read for Q8_0R (the N of
 * the whole tensor, which locates its scale region). */
int or_dequant(int type, const uint8_t *w, uint64_t n_blocks, uint32_t n_tensor, float *out) {
  uint32_t E, B;
  if (or_geometry(type, &E, &B)) return -1;
  if (type == OR_IQ2_XXS && !g_grid_set) return -2;
  for (uint64_t i = 0; i < n_blocks; ++i) {
    float *o = out + i * E;
    const uint8_t *b = w + i * B;
    switch (type) {
      case OR_Q8_0: deq_q8_0(b, o); break;
      case OR_Q8_0R: deq_q8_0r(w, n_tensor, i, o); break;
      case OR_Q2_K: deq_q2_k(b, o); break;
      case OR_Q4_K: deq_q4_k(b, o); break;
      case OR_Q6_K: deq_q6_k(b, o); break;
      case OR_IQ2_XXS: deq_iq2_xxs(b, o); break;
    }
  }
  return 0;
}

/* filaAF32 (cpu.js:45-80), the reference's second, JS-side statement of the
 * Q8_0 and Q6_K decoders: each product rounded to f32 (Math.fround). */
int or_dequant_cpujs(int type, const uint8_t *w, uint64_t n_blocks, float *out) {
  for (uint64_t b = 0; b < n_blocks; ++b) {
    if (type == OR_Q8_0) {
      const uint8_t *p = w + b * 34;
      float d = (float)or_def16((uint32_t)p[0] | ((uint32_t)p[1] << 8));
      for (int i = 0; i < 32; ++i) out[b * 32 + i] = (float)((double)(int8_t)p[2 + i] * (double)d);
    } else if (type == OR_Q6_K) {
      const uint8_t *p = w + b * 210;
      float d = (float)or_def16((uint32_t)p[208] | ((uint32_t)p[209] << 8));
      for (int n = 0; n < 2; ++n) {
        const uint8_t *ql = p + n * 64, *qh = p + 128 + n * 32;
        const int8_t *sc = (const int8_t *)(p + 192 + n * 8);
        float *ob = out + b * 256 + n * 128;
        for (int l = 0; l < 32; ++l) {
          int is = l >> 4;
          uint32_t lo0 = ql[l], lo32 = ql[32 + l], h = qh[l];
          ob[l] = (float)((double)(float)((double)d * sc[is]) * (double)((int)((lo0 & 0xf) | ((h & 3) << 4)) - 32));
          ob[32 + l] = (float)((double)(float)((double)d * sc[is + 2]) * (double)((int)((lo32 & 0xf) | (((h >> 2) & 3) << 4)) - 32));
          ob[64 + l] = (float)((double)(float)((double)d * sc[is + 4]) * (double)((int)((lo0 >> 4) | (((h >> 4) & 3) << 4)) - 32));
          ob[96 + l] = (float)((double)(float)((double)d * sc[is + 6]) * (double)((int)((lo32 >> 4) | (((h >> 6) & 3) << 4)) - 32));
        }
      }
    } else {
      return -1;
    }
  }
  return 0;
}

/* ---- matmul oracles ----------------------------------------------------- */

/* y[t][r] = sum_k w[r][k] x[t][k] in double over the exactly dequantized f32
 * weights and the f32 activations (the contract of quant.matmul, ops.js:827-829;
 * output layout y[(base_t + t) * rows + row], kernels.wgsl.js:1160-1185). */
int or_gemv_f64(int type, const uint8_t *w, uint32_t n_tensor, uint32_t rows, uint32_t k, const float *x,
                uint32_t tokens, double *y) {
  uint32_t E, B;
  if (or_geometry(type, &E, &B) || k % E) return -1;
  uint32_t bpr = k / E;
  float *row = (float *)malloc(sizeof(float) * k);
  float *tmp = (float *)malloc(sizeof(float) * E);
  if (!row || !tmp) { free(row); free(tmp); return -3; }
  for (uint32_t r = 0; r < rows; ++r) {
    for (uint32_t b = 0; b < bpr; ++b) {
      uint64_t bi = (uint64_t)r * bpr + b;
      if (type == OR_Q8_0R) deq_q8_0r(w, n_tensor, bi, tmp);
      else or_dequant(type, w + bi * B, 1, 0, tmp);
      memcpy(row + (uint64_t)b * E, tmp, sizeof(float) * E);
    }
    for (uint32_t t = 0; t < tokens; ++t) {
      double s = 0.0;
      const float *xt = x + (uint64_t)t * k;
      for (uint32_t i = 0; i < k; ++i) s += (double)row[i] * (double)xt[i];
      y[(uint64_t)t * rows + r] = s;
    }
  }
  free(row);
  free(tmp);
  return 0;
}

/* RNE binary32 -> binary16 -> value, as WGSL f16() conversion does
 * (kernels.drift.wgsl.js:88,104: vec4<f16>(v)). */
static double to_f16_value(float f) { return or_def16(or_af16((double)f)); }

/* The reference's fp16 GEMM rounding points (DRIFT, kernels.drift.wgsl.js:65-142;
 * GEMM2 exacto is bit-identical to it, kernels.gemm2.wgsl.js:12-23): x and the
 * dequantized w rounded to f16, products accumulated; here in double. */
int or_gemm_f16(int type, const uint8_t *w, uint32_t n_tensor, uint32_t rows, uint32_t k, const float *x,
                uint32_t tokens, double *y) {
  uint32_t E, B;
  if (or_geometry(type, &E, &B) || k % E) return -1;
  uint32_t bpr = k / E;
  double *row = (double *)malloc(sizeof(double) * k);
  double *xh = (double *)malloc(sizeof(double) * (uint64_t)k * tokens);
  float *tmp = (float *)malloc(sizeof(float) * E);
  if (!row || !xh || !tmp) { free(row); free(xh); free(tmp); return -3; }
  for (uint64_t i = 0; i < (uint64_t)k * tokens; ++i) xh[i] = to_f16_value(x[i]);
  for (uint32_t r = 0; r < rows; ++r) {
    for (uint32_t b = 0; b < bpr; ++b) {
      uint64_t bi = (uint64_t)r * bpr + b;
      if (type == OR_Q8_0R) deq_q8_0r(w, n_tensor, bi, tmp);
      else or_dequant(type, w + bi * B, 1, 0, tmp);
      for (uint32_t e = 0; e < E; ++e) row[(uint64_t)b * E + e] = to_f16_value(tmp[e]);
    }
    for (uint32_t t = 0; t < tokens; ++t) {
      double s = 0.0;
      const double *xt = xh + (uint64_t)t * k;
      for (uint32_t i = 0; i < k; ++i) s += row[i] * xt[i];
      y[(uint64_t)t * rows + r] = s;
    }
  }
  free(row);
  free(xh);
  free(tmp);
  return 0;
}

/* ---- top-k --------------------------------------------------------------- */

/* clave (kernels.topk.wgsl.js:75-82): -0 counts as +0, positives get the sign
 * bit, negatives are inverted; u32 order = f32 order. */
uint32_t or_topk_key(uint32_t bits) {
  uint32_t b = bits == 0x80000000u ? 0u : bits;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static const uint32_t *g_sort_bits;
static int cmp_rank(const void *a, const void *b) {
  uint32_t i = *(const uint32_t *)a, j = *(const uint32_t *)b;
  uint32_t ki = or_topk_key(g_sort_bits[i]), kj = or_topk_key(g_sort_bits[j]);
  /* antes (sample.js:44): larger first; equal values: lower index first */
  if (ki != kj) return ki > kj ? -1 : 1;
  return i < j ? -1 : (i > j ? 1 : 0);
}

/* The first m of logits[0..vocab) in the (value desc, index asc) order of
 * sample.js:44-67, by a full sort. Returns the count (min(m, vocab)); sets
 * *nan when any NaN bit pattern is present (the kernel's flag 2). */
int or_topk(const uint32_t *bits, uint32_t vocab, uint32_t m, uint32_t *ids, uint32_t *out_bits, int *nan) {
  uint32_t *idx = (uint32_t *)malloc(sizeof(uint32_t) * (vocab ? vocab : 1));
  if (!idx) return -3;
  *nan = 0;
  for (uint32_t i = 0; i < vocab; ++i) {
    idx[i] = i;
    if ((bits[i] & 0x7FFFFFFFu) > 0x7F800000u) *nan = 1;
  }
  g_sort_bits = bits;
  qsort(idx, vocab, sizeof(uint32_t), cmp_rank);
  uint32_t n = m < vocab ? m : vocab;
  for (uint32_t i = 0; i < n; ++i) {
    ids[i] = idx[i];
    out_bits[i] = bits[idx[i]];
  }
  free(idx);
  return (int)n;
}

/* ---- Q8_0 quantizer (cpu.js:273-287) ------------------------------------ */

/* Math.round: nearest, ties toward +infinity. */
static double js_round(double v) {
  double f = floor(v);
  return (v - f >= 0.5) ? f + 1.0 : f;
}

int or_quantize_q8_0(const float *x, uint64_t n, uint8_t *out) {
  if (n % 32) return -1;
  for (uint64_t b = 0; b < n / 32; ++b) {
    double a = 0;
    for (int i = 0; i < 32; ++i) a = fmax(a, fabs((double)x[b * 32 + i]));
    double d = a / 127, id = d != 0.0 ? 1 / d : 0;
    uint8_t *o = out + b * 34;
    uint32_t h = or_af16(d);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; ++i) {
      double r = js_round((double)x[b * 32 + i] * id);
      o[2 + i] = (uint8_t)(int8_t)(int32_t)r; /* DataView.setInt8: value modulo 256 */
    }
  }
  return 0;
}

/* ---- Q8_0R repack (repack.js:103-219, kernels.bloques.wgsl.js:19-35) ----- */

uint64_t or_bytes_reordered(uint32_t n) { return ((uint64_t)34 * n + 3) / 4 * 4; }   /* bytesReordenado */
uint64_t or_bytes_buffer_r(uint32_t n) { return ((uint64_t)34 * n + 15) / 16 * 16; } /* bytesBufferR */
uint32_t or_blocks_from_buffer(uint64_t bytes) { return (uint32_t)((2 * (bytes / 4)) / 17); } /* bloquesDeBuffer */

/* reordena (repack.js:187-199) by its byte-wise path (repack.js:165-172):
 * quants of block i to [32i, 32i+32), the scale to bytes 32N+2i, 32N+2i+1;
 * the rest of dst zeroed. dst must hold or_bytes_reordered(n) bytes. */
int or_repack(const uint8_t *src, uint32_t n, uint8_t *dst, uint64_t dst_bytes) {
  uint64_t W = 32ull * n;
  if (dst_bytes < or_bytes_reordered(n)) return -1;
  for (uint64_t i = 0; i < n; ++i) {
    uint64_t s = i * 34;
    dst[W + 2 * i] = src[s];
    dst[W + 2 * i + 1] = src[s + 1];
    for (int j = 0; j < 32; ++j) dst[32 * i + j] = src[s + 2 + j];
  }
  memset(dst + W + 2ull * n, 0, dst_bytes - (W + 2ull * n));
  return 0;
}

/* vuelveAlGGUF (repack.js:204-219). */
int or_unrepack(const uint8_t *src, uint32_t n, uint8_t *dst) {
  uint64_t W = 32ull * n;
  for (uint64_t i = 0; i < n; ++i) {
    dst[i * 34] = src[W + 2 * i];
    dst[i * 34 + 1] = src[W + 2 * i + 1];
    memcpy(dst + i * 34 + 2, src + 32 * i, 32);
  }
  return 0;
}

/* ---- CPU path (cpu.js, cpu-trabajo.js) ------------------------------------
 * parity unpinned: restated from the JavaScript side only.
 *
 * Activations are quantized once per call into 40-byte blocks per 32 values
 * (BACT = 40, cpu.js:25; e.cuantiza_filas, cpu.js:376). The layout inside the
 * 40 bytes is not visible from JS; modelled as f32 d = amax/127, f32 s = d*sum(q)
 * and 32 int8 q = round(x/d) (ggml's Q8_1 layout, which has the same size).
 * matvec_q8_0 (cpu-trabajo.js:62) then takes, per row, the integer dot of each
 * weight block with its activation block, scaled by d_w * d_a, summed in f32.
 * Rows are split into chunks claimed by a pool of threads
 * (cpu-trabajo.js:33-46, cpu.js:140-206). */

typedef struct {
  float d, s;
  int8_t q[32];
} or_act_block;

int or_cpu_quantize_acts(const float *x, uint32_t k, uint32_t tokens, or_act_block *out) {
  if (k % 32) return -1;
  for (uint64_t b = 0; b < (uint64_t)tokens * (k / 32); ++b) {
    const float *v = x + b * 32;
    float a = 0.f;
    for (int i = 0; i < 32; ++i) a = fmaxf(a, fabsf(v[i]));
    float d = a / 127.f, id = d != 0.f ? 1.f / d : 0.f;
    int sum = 0;
    for (int i = 0; i < 32; ++i) {
      int q = (int)roundf(v[i] * id);
      out[b].q[i] = (int8_t)q;
      sum += q;
    }
    out[b].d = d;
    out[b].s = d * (float)sum;
  }
  return 0;
}

static void cpu_rows_q8_0(const uint8_t *w, const or_act_block *act, float *y, uint32_t k, uint32_t rows,
                          uint32_t tokens, uint32_t r0, uint32_t r1) {
  uint32_t nb = k / 32;
  for (uint32_t t = 0; t < tokens; ++t)
    for (uint32_t r = r0; r < r1; ++r) {
      float sum = 0.f;
      const uint8_t *row = w + (uint64_t)r * nb * 34;
      const or_act_block *a = act + (uint64_t)t * nb;
      for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = row + b * 34;
        int isum = 0;
        for (int i = 0; i < 32; ++i) isum += (int)(int8_t)blk[2 + i] * (int)a[b].q[i];
        sum += (float)isum * (hf(blk) * a[b].d);
      }
      y[(uint64_t)t * rows + r] = sum;
    }
}

/* f32 dequantize-and-dot of rows [r0, r1): the baseline for the types that
 * have no CPU kernel in the reference (cpu-trabajo.js:31 lists Q8_0/Q4_0 only). */
static void cpu_rows_f32(int type, const uint8_t *w, const float *x, float *y, uint32_t k, uint32_t rows,
                         uint32_t tokens, uint32_t r0, uint32_t r1, float *scratch) {
  uint32_t E, B;
  or_geometry(type, &E, &B);
  uint32_t bpr = k / E;
  for (uint32_t r = r0; r < r1; ++r) {
    or_dequant(type, w + (uint64_t)r * bpr * B, bpr, 0, scratch);
    for (uint32_t t = 0; t < tokens; ++t) {
      const float *xt = x + (uint64_t)t * k;
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
      for (uint32_t i = 0; i < k; i += 4) {
        s0 += scratch[i] * xt[i];
        s1 += scratch[i + 1] * xt[i + 1];
        s2 += scratch[i + 2] * xt[i + 2];
        s3 += scratch[i + 3] * xt[i + 3];
      }
      y[(uint64_t)t * rows + r] = (s0 + s1) + (s2 + s3);
    }
  }
}

/* The pool: n threads claim chunks of rows from a shared counter until none
 * are left; chunk = max(4, ceil(rows / (n * 4) / 4) * 4) rows
 * (TROZOS_POR_HILO = 4, cpu.js:140,173). */
typedef struct {
  int mode; /* 0 = Q8 integer path, 1 = f32 dequant path */
  int type;
  const uint8_t *w;
  const void *act;
  float *y;
  uint32_t k, rows, tokens, per_chunk, chunks;
  atomic_uint next;
} or_job;

static void *or_worker(void *p) {
  or_job *j = (or_job *)p;
  uint32_t E = 32, B = 34;
  or_geometry(j->type, &E, &B);
  float *scratch = j->mode ? (float *)malloc(sizeof(float) * j->k) : NULL;
  for (;;) {
    uint32_t c = atomic_fetch_add(&j->next, 1u);
    if (c >= j->chunks) break;
    uint32_t r0 = c * j->per_chunk, r1 = r0 + j->per_chunk;
    if (r1 > j->rows) r1 = j->rows;
    if (j->mode == 0) cpu_rows_q8_0(j->w, (const or_act_block *)j->act, j->y, j->k, j->rows, j->tokens, r0, r1);
    else cpu_rows_f32(j->type, j->w, (const float *)j->act, j->y, j->k, j->rows, j->tokens, r0, r1, scratch);
  }
  free(scratch);
  return NULL;
}

/* Y = W X on the CPU with `threads` threads. Q8_0 goes through the
 * reference's integer path (activations quantized first, in the calling
 * thread, as cpu.js:376 does before the job); other types through the f32
 * dequantize-and-dot path. */
int or_cpu_matmul(int type, const uint8_t *w, uint32_t rows, uint32_t k, const float *x, uint32_t tokens,
                  int threads, float *y) {
  uint32_t E, B;
  if (or_geometry(type, &E, &B) || k % E || threads < 1 || type == OR_Q8_0R) return -1;
  if (type == OR_IQ2_XXS && !g_grid_set) return -2;
  or_job job;
  memset(&job, 0, sizeof job);
  or_act_block *act = NULL;
  job.mode = type == OR_Q8_0 ? 0 : 1;
  if (job.mode == 0) {
    act = (or_act_block *)malloc(sizeof(or_act_block) * (uint64_t)tokens * (k / 32));
    if (!act) return -3;
    or_cpu_quantize_acts(x, k, tokens, act);
    job.act = act;
  } else {
    job.act = x;
  }
  job.type = type;
  job.w = w;
  job.y = y;
  job.k = k;
  job.rows = rows;
  job.tokens = tokens;
  uint32_t per = (uint32_t)ceil((double)rows / (threads * 4) / 4) * 4;
  job.per_chunk = per < 4 ? 4 : per;
  job.chunks = (rows + job.per_chunk - 1) / job.per_chunk;
  atomic_init(&job.next, 0u);
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * threads);
  for (int i = 1; i < threads; ++i) pthread_create(&th[i], NULL, or_worker, &job);
  or_worker(&job); /* the coordinating thread takes chunks too (cpu.js:187) */
  for (int i = 1; i < threads; ++i) pthread_join(th[i], NULL);
  free(th);
  free(act);
  return 0;
}
