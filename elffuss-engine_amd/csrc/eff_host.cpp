// Host-side data preparation of the C ABI: type table, Q8_0R repack and its
// buffer arithmetic, the synthetic-input generator and the block quantizers.
//
// Nothing here touches the device; the HIP part lives in eff_api.hip and
// eff_kernels.hip. Functions are `extern "C"` (declared in elffuss_amd.h).
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/elffuss_amd.h"
#include "eff_formats.h"

using namespace eff;

namespace {

const uint64_t kIq2xxsGrid[256] = {
#include "iq2xxs_grid.inc"
};

// Run f(begin, end) over [0, n) split across the host's threads.
template <class F>
void parallel_for(size_t n, F f, size_t min_chunk = 1024) {
  unsigned hw = std::thread::hardware_concurrency();
  size_t nt = std::max<size_t>(1, std::min<size_t>(hw ? hw : 1, 64));
  if (n < 2 * min_chunk || nt == 1) {
    f(0, n);
    return;
  }
  nt = std::min(nt, (n + min_chunk - 1) / min_chunk);
  std::vector<std::thread> th;
  size_t step = (n + nt - 1) / nt;
  for (size_t t = 0; t < nt; ++t) {
    size_t b = t * step, e = std::min(n, b + step);
    if (b >= e) break;
    th.emplace_back([=] { f(b, e); });
  }
  for (auto &x : th) x.join();
}

inline void put_u16(uint8_t *p, uint32_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}

// JavaScript Math.round: nearest integer, ties toward +infinity.
inline double js_round(double v) {
  double r = floor(v);
  if (v - r >= 0.5) r += 1.0;
  return r;
}

// The reference's aF16 (cpu.js:84-99): the double is first stored into a
// Float32Array (round to f32), then rounded to f16, ties to even.
inline uint32_t js_af16(double v) { return float_to_half_rne((float)v); }

// Round to nearest, ties to even (the quantizers below only need a consistent
// rounding; the reference has no quantizer for these types).
inline int nint(float v) { return (int)lrintf(v); }

// ---- Q8_0: the reference quantizer (cpu.js:273-287) -----------------------
void quant_q8_0_block(const float *x, uint8_t *o) {
  double a = 0.0;
  for (int i = 0; i < 32; ++i) a = std::max(a, fabs((double)x[i]));
  double d = a / 127.0;
  double id = d != 0.0 ? 1.0 / d : 0.0;
  put_u16(o, js_af16(d));
  for (int i = 0; i < 32; ++i) {
    double r = js_round((double)x[i] * id);
    o[2 + i] = (uint8_t)(int8_t)(int)r;  // |r| <= 127 by construction
  }
}

// ---- Q4_K ------------------------------------------------------------------
// 8 sub-blocks of 32 with a 6-bit scale and a 6-bit min each; w = d*sc*q - dmin*m.
void quant_q4_k_block(const float *x, uint8_t *o) {
  float scale[8], minv[8];
  float max_scale = 0.f, max_min = 0.f;
  for (int j = 0; j < 8; ++j) {
    float mn = 0.f, mx = -INFINITY;
    for (int i = 0; i < 32; ++i) {
      mn = std::min(mn, x[32 * j + i]);
      mx = std::max(mx, x[32 * j + i]);
    }
    mx = std::max(mx, mn);
    scale[j] = (mx - mn) / 15.f;
    minv[j] = -mn;
    max_scale = std::max(max_scale, scale[j]);
    max_min = std::max(max_min, minv[j]);
  }
  uint32_t dh = float_to_half_rne(max_scale / 63.f);
  uint32_t mh = float_to_half_rne(max_min / 63.f);
  float d = half_to_float(dh), dmin = half_to_float(mh);
  int sc[8], m[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0.f ? std::min(63, std::max(0, nint(scale[j] / d))) : 0;
    m[j] = dmin > 0.f ? std::min(63, std::max(0, nint(minv[j] / dmin))) : 0;
  }
  put_u16(o, dh);
  put_u16(o + 2, mh);
  uint8_t *s = o + 4;
  for (int j = 0; j < 4; ++j) {
    s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
  }
  uint8_t q[256];
  for (int j = 0; j < 8; ++j) {
    float dl = d * (float)sc[j], ml = dmin * (float)m[j];
    for (int i = 0; i < 32; ++i) {
      int v = dl > 0.f ? nint((x[32 * j + i] + ml) / dl) : 0;
      q[32 * j + i] = (uint8_t)std::min(15, std::max(0, v));
    }
  }
  uint8_t *qs = o + 16;
  for (int j = 0; j < 4; ++j)
    for (int l = 0; l < 32; ++l) qs[32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
}

// ---- Q6_K ------------------------------------------------------------------
// 16 sub-blocks of 16 with a signed 8-bit scale; w = d*sc*(q-32), q in 0..63.
void quant_q6_k_block(const float *x, uint8_t *o) {
  float sub[16];
  float max_abs = 0.f;
  for (int j = 0; j < 16; ++j) {
    float v = 0.f;
    for (int i = 0; i < 16; ++i)
      if (fabsf(x[16 * j + i]) > fabsf(v)) v = x[16 * j + i];
    sub[j] = v / -32.f;  // the extreme value maps onto q-32 = -32
    max_abs = std::max(max_abs, fabsf(sub[j]));
  }
  uint32_t dh = float_to_half_rne(max_abs / 127.f);
  float d = half_to_float(dh);
  int8_t sc[16];
  for (int j = 0; j < 16; ++j)
    sc[j] = (int8_t)(d > 0.f ? std::min(127, std::max(-128, nint(sub[j] / d))) : 0);
  uint8_t q[256];
  for (int j = 0; j < 16; ++j) {
    float step = d * (float)sc[j];
    for (int i = 0; i < 16; ++i) {
      int v = step != 0.f ? nint(x[16 * j + i] / step) : 0;
      q[16 * j + i] = (uint8_t)(std::min(31, std::max(-32, v)) + 32);
    }
  }
  uint8_t *ql = o, *qh = o + 128;
  for (int n = 0; n < 2; ++n)
    for (int l = 0; l < 32; ++l) {
      const uint8_t *h = q + 128 * n;
      ql[64 * n + l] = (uint8_t)((h[l] & 15) | ((h[64 + l] & 15) << 4));
      ql[64 * n + 32 + l] = (uint8_t)((h[32 + l] & 15) | ((h[96 + l] & 15) << 4));
      qh[32 * n + l] = (uint8_t)((h[l] >> 4) | ((h[32 + l] >> 4) << 2) | ((h[64 + l] >> 4) << 4) |
                                 ((h[96 + l] >> 4) << 6));
    }
  memcpy(o + 192, sc, 16);
  put_u16(o + 208, dh);
}

// ---- Q2_K ------------------------------------------------------------------
// 16 sub-blocks of 16 with a 4-bit scale and a 4-bit min; w = d*sc*q - dmin*m, q in 0..3.
void quant_q2_k_block(const float *x, uint8_t *o) {
  float scale[16], minv[16];
  float max_scale = 0.f, max_min = 0.f;
  for (int j = 0; j < 16; ++j) {
    float mn = 0.f, mx = -INFINITY;
    for (int i = 0; i < 16; ++i) {
      mn = std::min(mn, x[16 * j + i]);
      mx = std::max(mx, x[16 * j + i]);
    }
    mx = std::max(mx, mn);
    scale[j] = (mx - mn) / 3.f;
    minv[j] = -mn;
    max_scale = std::max(max_scale, scale[j]);
    max_min = std::max(max_min, minv[j]);
  }
  uint32_t dh = float_to_half_rne(max_scale / 15.f);
  uint32_t mh = float_to_half_rne(max_min / 15.f);
  float d = half_to_float(dh), dmin = half_to_float(mh);
  uint8_t q[256];
  for (int j = 0; j < 16; ++j) {
    int sc = d > 0.f ? std::min(15, std::max(0, nint(scale[j] / d))) : 0;
    int m = dmin > 0.f ? std::min(15, std::max(0, nint(minv[j] / dmin))) : 0;
    o[j] = (uint8_t)(sc | (m << 4));
    float dl = d * (float)sc, ml = dmin * (float)m;
    for (int i = 0; i < 16; ++i) {
      int v = dl > 0.f ? nint((x[16 * j + i] + ml) / dl) : 0;
      q[16 * j + i] = (uint8_t)std::min(3, std::max(0, v));
    }
  }
  uint8_t *qs = o + 16;
  memset(qs, 0, 64);
  for (int n = 0; n < 2; ++n)
    for (int j = 0; j < 4; ++j)
      for (int i = 0; i < 32; ++i) qs[32 * n + i] |= (uint8_t)(q[128 * n + 32 * j + i] << (2 * j));
  put_u16(o + 80, dh);
  put_u16(o + 82, mh);
}

// ---- IQ2_XXS ---------------------------------------------------------------
// 8 groups of 32: each 8 weights take one grid entry (magnitudes from
// {8,25,43}) and 7 stored sign bits; the 8th sign is the even-parity bit.
// Group scale db = d*(0.5+ls)*0.25 with a 4-bit ls.
void quant_iq2_xxs_block(const float *x, uint8_t *o) {
  float gmax[8];
  float top = 0.f;
  for (int g = 0; g < 8; ++g) {
    float a = 0.f;
    for (int i = 0; i < 32; ++i) a = std::max(a, fabsf(x[32 * g + i]));
    gmax[g] = a / 43.f;  // the largest magnitude maps onto the largest grid value
    top = std::max(top, gmax[g]);
  }
  uint32_t dh = float_to_half_rne(top / 3.875f);  // db at ls = 15 is d * 15.5 * 0.25
  float d = half_to_float(dh);
  put_u16(o, dh);
  for (int g = 0; g < 8; ++g) {
    const float *xg = x + 32 * g;
    int ls = d > 0.f ? std::min(15, std::max(0, nint(gmax[g] / (d * 0.25f) - 0.5f))) : 0;
    float db = d * (0.5f + (float)ls) * 0.25f;
    uint32_t a0 = 0, a1 = (uint32_t)ls << 28;
    for (int l = 0; l < 4; ++l) {
      const float *v = xg + 8 * l;
      uint32_t neg = 0;
      int smallest = 0;
      for (int j = 0; j < 8; ++j) {
        if (v[j] < 0.f) neg |= 1u << j;
        if (fabsf(v[j]) < fabsf(v[smallest])) smallest = j;
      }
      if (__builtin_popcount(neg) & 1) neg ^= 1u << smallest;  // signs must have even parity
      int best = 0;
      float best_err = INFINITY;
      for (int e = 0; e < 256; ++e) {
        float err = 0.f;
        for (int j = 0; j < 8; ++j) {
          float gv = (float)((kIq2xxsGrid[e] >> (8 * j)) & 0xFF);
          float t = fabsf(v[j]) - db * gv;
          err += t * t;
        }
        if (err < best_err) {
          best_err = err;
          best = e;
        }
      }
      a0 |= (uint32_t)best << (8 * l);
      a1 |= (neg & 127u) << (7 * l);
    }
    uint8_t *p = o + 2 + 8 * g;
    memcpy(p, &a0, 4);
    memcpy(p + 4, &a1, 4);
  }
}

uint32_t mulberry32(uint32_t seed) {
  uint32_t t = seed + 0x6D2B79F5u;
  t = (t ^ (t >> 15)) * (t | 1u);
  t ^= t + (t ^ (t >> 7)) * (t | 61u);
  return t ^ (t >> 14);
}

}  // namespace

extern "C" {

int eff_type_from_name(const char *name) {
  if (!name) return EFF_E_TYPE;
  static const struct { const char *n; int t; } kNames[] = {
      {"Q8_0", EFF_TYPE_Q8_0}, {"Q2_K", EFF_TYPE_Q2_K},       {"Q4_K", EFF_TYPE_Q4_K},
      {"Q6_K", EFF_TYPE_Q6_K}, {"IQ2_XXS", EFF_TYPE_IQ2_XXS}, {"Q8_0R", EFF_TYPE_Q8_0R},
  };
  for (auto &e : kNames)
    if (strcmp(e.n, name) == 0) return e.t;
  return EFF_E_TYPE;
}

const char *eff_type_name(int type) {
  switch (type) {
    case EFF_TYPE_Q8_0: return "Q8_0";
    case EFF_TYPE_Q2_K: return "Q2_K";
    case EFF_TYPE_Q4_K: return "Q4_K";
    case EFF_TYPE_Q6_K: return "Q6_K";
    case EFF_TYPE_IQ2_XXS: return "IQ2_XXS";
    case EFF_TYPE_Q8_0R: return "Q8_0R";
    default: return nullptr;
  }
}

int eff_type_geometry(int type, uint32_t *block_elems, uint32_t *block_bytes) {
  if (!type_known(type)) return EFF_E_TYPE;
  Geometry g = geometry(type);
  if (block_elems) *block_elems = g.elems;
  if (block_bytes) *block_bytes = g.bytes;
  return EFF_OK;
}

size_t eff_bytes_reordered(int type_r, uint32_t n) {
  if (type_r != EFF_TYPE_Q8_0R) return 0;
  return ((size_t)34 * n + 3) / 4 * 4;
}

size_t eff_bytes_buffer_r(int type_r, uint32_t n) {
  if (type_r != EFF_TYPE_Q8_0R) return 0;
  return ((size_t)34 * n + 15) / 16 * 16;
}

uint32_t eff_blocks_from_buffer(int type_r, size_t bytes) {
  if (type_r != EFF_TYPE_Q8_0R) return 0;
  size_t L = bytes / 4;
  return (uint32_t)((2 * L) / 17);
}

uint32_t eff_scales_from(int type_r, uint32_t n) {
  if (type_r != EFF_TYPE_Q8_0R) return 0;
  return 8u * n;
}

int eff_repack(int type_r, const void *src, uint32_t n, void *dst, size_t dst_bytes) {
  if (type_r != EFF_TYPE_Q8_0R) return EFF_E_TYPE;
  if (!src || !dst) return EFF_E_INVALID;
  if (dst_bytes < eff_bytes_reordered(type_r, n)) return EFF_E_BOUNDS;
  const uint8_t *s = (const uint8_t *)src;
  uint8_t *q = (uint8_t *)dst;
  uint8_t *e = q + (size_t)32 * n;
  parallel_for(n, [&](size_t b, size_t end) {
    for (size_t i = b; i < end; ++i) {
      memcpy(q + 32 * i, s + 34 * i + 2, 32);
      e[2 * i] = s[34 * i];
      e[2 * i + 1] = s[34 * i + 1];
    }
  }, 1 << 16);
  size_t used = (size_t)34 * n;
  memset(q + used, 0, dst_bytes - used);
  return EFF_OK;
}

int eff_unrepack(int type_r, const void *src, size_t src_bytes, uint32_t n, void *dst) {
  if (type_r != EFF_TYPE_Q8_0R) return EFF_E_TYPE;
  if (!src || !dst) return EFF_E_INVALID;
  if (src_bytes < (size_t)34 * n) return EFF_E_BOUNDS;
  const uint8_t *q = (const uint8_t *)src;
  const uint8_t *e = q + (size_t)32 * n;
  uint8_t *o = (uint8_t *)dst;
  for (size_t i = 0; i < n; ++i) {
    o[34 * i] = e[2 * i];
    o[34 * i + 1] = e[2 * i + 1];
    memcpy(o + 34 * i + 2, q + 32 * i, 32);
  }
  return EFF_OK;
}

int eff_quantize(int type, const float *src, size_t n, void *dst, size_t dst_bytes) {
  if (!src || !dst) return EFF_E_INVALID;
  if (type == EFF_TYPE_Q8_0R || !type_known(type)) return EFF_E_TYPE;
  Geometry g = geometry(type);
  if (n % g.elems) return EFF_E_SHAPE;
  size_t nb = n / g.elems;
  if (dst_bytes < nb * g.bytes) return EFF_E_BOUNDS;
  void (*fn)(const float *, uint8_t *) = nullptr;
  switch (type) {
    case EFF_TYPE_Q8_0: fn = quant_q8_0_block; break;
    case EFF_TYPE_Q4_K: fn = quant_q4_k_block; break;
    case EFF_TYPE_Q6_K: fn = quant_q6_k_block; break;
    case EFF_TYPE_Q2_K: fn = quant_q2_k_block; break;
    case EFF_TYPE_IQ2_XXS: fn = quant_iq2_xxs_block; break;
  }
  uint8_t *o = (uint8_t *)dst;
  parallel_for(nb, [&](size_t b, size_t e) {
    for (size_t i = b; i < e; ++i) fn(src + i * g.elems, o + i * g.bytes);
  }, type == EFF_TYPE_IQ2_XXS ? 64 : 1024);
  return EFF_OK;
}

int eff_fill_normal(uint32_t seed, float sigma, float *dst, size_t n) {
  if (!dst && n) return EFF_E_INVALID;
  const double two_pi = 6.283185307179586476925286766559;
  size_t pairs = (n + 1) / 2;
  parallel_for(pairs, [&](size_t b, size_t e) {
    for (size_t p = b; p < e; ++p) {
      uint32_t c = seed + (uint32_t)(2 * p);
      double u1 = mulberry32(c) / 4294967296.0;
      double u2 = mulberry32(c + 1u) / 4294967296.0;
      double r = sqrt(-2.0 * log(1.0 - u1));
      double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
      dst[2 * p] = (float)((double)sigma * z0);
      if (2 * p + 1 < n) dst[2 * p + 1] = (float)((double)sigma * z1);
    }
  }, 1 << 14);
  return EFF_OK;
}

}  // extern "C"
