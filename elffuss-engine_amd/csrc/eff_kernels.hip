// gfx950 kernels of the quantized matrix-product path.
//
// Work unit. Every kernel walks a row of W in units of 32 weights: one Q8_0
// block, or one eighth of a 256-weight super-block. A unit is two runs of 16
// weights ("halves" A and B) at k offsets (o0, o1) inside its block, each half
// with one scale and one offset:
//     sum_i w_i x_i = sA * sum_A u_i x_i + sB * sum_B u_i x_i - mA * sum_A x_i - mB * sum_B x_i
// where u_i is a small unsigned integer taken from the block bytes. The unit
// split follows the block layout so that the bytes of a unit are contiguous:
//   Q8_0     one block; u = q + 128
//   Q4_K     16 qs bytes: low nibbles = sub-block 2j, high nibbles = 2j+1
//   Q6_K     16 ql bytes + the 16 qh bytes that complete them (two groups of 32)
//   Q2_K     16 qs bytes at two of the four bit-shifts (two sub-blocks of 16)
//   IQ2_XXS  one 32-weight group (4 grid entries, signs folded into u = ±g + 128)
// The decoders follow the reference's DECODERS (kernels.wgsl.js:154-396); the
// f32 dequantization (dequant_unit) reproduces their operation order exactly.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
#include "eff_formats.h"
#include "eff_kernels.h"

namespace eff {

__constant__ uint64_t c_iq2xxs_grid[256] = {
#include "iq2xxs_grid.inc"
};

__device__ __forceinline__ float ubyte(uint32_t w, int c) { return (float)((w >> (8 * c)) & 0xFFu); }

// ---------------------------------------------------------------------------
// Per-type raw unit data.
template <int TYPE> struct Raw;

template <> struct Raw<Q8_0> {
  uint32_t s, v[8];
};
template <> struct Raw<Q8_0R> {
  uint32_t v[8], s;
};
template <> struct Raw<Q4_K> {
  uint32_t hdr[4], qs[4], sub;
};
template <> struct Raw<Q6_K> {
  uint32_t ql[4], qh[4], sc, d, sub;
};
template <> struct Raw<Q2_K> {
  uint32_t qs[4], sc, dd, sub;
};
template <> struct Raw<IQ2_XXS> {
  uint32_t a0, a1, d;
};

template <int TYPE> constexpr uint32_t units_per_block() { return (TYPE == Q8_0 || TYPE == Q8_0R) ? 1u : 8u; }
template <int TYPE> constexpr uint32_t block_elems() { return (TYPE == Q8_0 || TYPE == Q8_0R) ? 32u : 256u; }
template <int TYPE> constexpr uint32_t block_bytes() {
  return TYPE == Q8_0 ? 34u : TYPE == Q8_0R ? 34u : TYPE == Q4_K ? 144u : TYPE == Q6_K ? 210u
       : TYPE == Q2_K ? 84u : 66u;
}

// k offsets of the two 16-weight halves of unit `sub` inside its block.
template <int TYPE>
__device__ __forceinline__ void unit_runs(uint32_t sub, uint32_t &o0, uint32_t &o1) {
  if constexpr (TYPE == Q8_0 || TYPE == Q8_0R) {
    o0 = 0; o1 = 16;
  } else if constexpr (TYPE == Q4_K) {
    // qs bytes 16*sub..: j = sub>>1, h = sub&1 -> weights 64j+16h (+32 for high nibbles)
    o0 = 64u * (sub >> 1) + 16u * (sub & 1u); o1 = o0 + 32u;
  } else if constexpr (TYPE == Q6_K) {
    // ql bytes 16*sub..: n = sub>>2, gp = (sub>>1)&1, h = sub&1
    o0 = 128u * (sub >> 2) + 32u * ((sub >> 1) & 1u) + 16u * (sub & 1u); o1 = o0 + 64u;
  } else if constexpr (TYPE == Q2_K) {
    // sub = 4n + 2jp + half: qs chunk c = 2n + half at bit shifts j = 2jp, 2jp+1;
    // consecutive pairs of units cover 64 consecutive weights
    o0 = 128u * (sub >> 2) + 64u * ((sub >> 1) & 1u) + 16u * (sub & 1u); o1 = o0 + 32u;
  } else {
    o0 = 32u * sub; o1 = o0 + 16u;
  }
}

// Loading a unit is split in two: issue_raw issues the loads and keeps the
// words as loaded; finish_raw re-assembles them (v_alignbyte of 2-byte aligned
// runs, 16-bit fields, byte pairs) into Raw. Callers that prefetch call
// finish_raw only where the unit is used, so that no instruction between the
// loads and that point waits for them.
template <int TYPE> struct RawLd {
  Raw<TYPE> r;  // Q4_K, Q2_K: the loads are the final form
};
template <> struct RawLd<Q8_0> {
  uint32_t sw, w[9], bp;
};
template <> struct RawLd<Q8_0R> {
  uint32_t v[8], sw, so;
};
template <> struct RawLd<Q6_K> {
  uint32_t ql[5], qh[5], s0, s1, dw, bp, sub;
};
template <> struct RawLd<IQ2_XXS> {
  uint32_t a[3], dw, bp;
};

// Issue the loads of unit `sub` of block `bi` (counted from the first block of `src`).
template <int TYPE>
__device__ __forceinline__ void issue_raw(RawLd<TYPE> &l, const BufSrc &src, uint32_t bi, uint32_t sub) {
  if constexpr (TYPE == Q8_0) {
    const uint32_t bp = bi * 34u, qb = (bp + 2u) & ~3u;
    l.sw = ld32(src.q, bp & ~3u);
#pragma unroll
    for (int i = 0; i < 9; ++i) l.w[i] = ld32(src.q, qb + 4u * i);
    l.bp = bp;
  } else if constexpr (TYPE == Q8_0R) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(src.q, (int)(bi * 32u), 0, 0);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(src.q, (int)(bi * 32u + 16u), 0, 0);
    l.v[0] = a.x; l.v[1] = a.y; l.v[2] = a.z; l.v[3] = a.w;
    l.v[4] = b.x; l.v[5] = b.y; l.v[6] = b.z; l.v[7] = b.w;
    l.so = bi * 2u;
    l.sw = ld32(src.s, l.so & ~3u);
  } else if constexpr (TYPE == Q4_K) {
    const uint32_t bp = bi * 144u;
    const u32x4 h = __builtin_amdgcn_raw_buffer_load_b128(src.q, (int)bp, 0, 0);
    const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(src.q, (int)(bp + 16u + 16u * sub), 0, 0);
    l.r.hdr[0] = h.x; l.r.hdr[1] = h.y; l.r.hdr[2] = h.z; l.r.hdr[3] = h.w;
    l.r.qs[0] = q.x; l.r.qs[1] = q.y; l.r.qs[2] = q.z; l.r.qs[3] = q.w;
    l.r.sub = sub;
  } else if constexpr (TYPE == Q6_K) {
    const uint32_t bp = bi * 210u;
    const uint32_t n = sub >> 2, gp = (sub >> 1) & 1u, h = sub & 1u;
    const uint32_t lo = bp + 16u * sub, ho = bp + 128u + 32u * n + 16u * h;
#pragma unroll
    for (int i = 0; i < 5; ++i) l.ql[i] = ld32(src.q, (lo & ~3u) + 4u * i);
#pragma unroll
    for (int i = 0; i < 5; ++i) l.qh[i] = ld32(src.q, (ho & ~3u) + 4u * i);
    // scales of groups gp and gp+2 at bytes 192 + 8n + 2g + h
    const uint32_t so = bp + 192u + 8u * n + 2u * gp + h;
    l.s0 = __builtin_amdgcn_raw_buffer_load_b8(src.q, (int)so, 0, 0);
    l.s1 = __builtin_amdgcn_raw_buffer_load_b8(src.q, (int)(so + 4u), 0, 0);
    l.dw = ld32(src.q, (bp + 208u) & ~3u);
    l.bp = bp;
    l.sub = sub;
  } else if constexpr (TYPE == Q2_K) {
    const uint32_t bp = bi * 84u;
    const uint32_t n = sub >> 2, jp = (sub >> 1) & 1u, c = 2u * n + (sub & 1u);
#pragma unroll
    for (int i = 0; i < 4; ++i) l.r.qs[i] = ld32(src.q, bp + 16u + 16u * c + 4u * i);
    l.r.sc = ld32(src.q, bp + 8u * n + 4u * jp);
    l.r.dd = ld32(src.q, bp + 80u);
    l.r.sub = sub;
  } else {
    const uint32_t bp = bi * 66u, ao = bp + 2u + 8u * sub;
#pragma unroll
    for (int i = 0; i < 3; ++i) l.a[i] = ld32(src.q, (ao & ~3u) + 4u * i);
    l.dw = ld32(src.q, bp & ~3u);
    l.bp = bp;
  }
}

template <int TYPE>
__device__ __forceinline__ void finish_raw(const RawLd<TYPE> &l, Raw<TYPE> &r) {
  if constexpr (TYPE == Q8_0) {
    const uint32_t sh = (l.bp + 2u) & 3u;
    r.s = (l.bp & 2u) ? (l.sw >> 16) : (l.sw & 0xFFFFu);
#pragma unroll
    for (int i = 0; i < 8; ++i) r.v[i] = __builtin_amdgcn_alignbyte(l.w[i + 1], l.w[i], sh);
  } else if constexpr (TYPE == Q8_0R) {
#pragma unroll
    for (int i = 0; i < 8; ++i) r.v[i] = l.v[i];
    r.s = (l.so & 2u) ? (l.sw >> 16) : (l.sw & 0xFFFFu);
  } else if constexpr (TYPE == Q6_K) {
    const uint32_t n = l.sub >> 2, h = l.sub & 1u;
    const uint32_t shl = (l.bp + 16u * l.sub) & 3u, shh = (l.bp + 128u + 32u * n + 16u * h) & 3u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.ql[i] = __builtin_amdgcn_alignbyte(l.ql[i + 1], l.ql[i], shl);
      r.qh[i] = __builtin_amdgcn_alignbyte(l.qh[i + 1], l.qh[i], shh);
    }
    r.sc = l.s0 | (l.s1 << 8);
    r.d = ((l.bp + 208u) & 2u) ? (l.dw >> 16) : (l.dw & 0xFFFFu);
    r.sub = l.sub;
  } else if constexpr (TYPE == IQ2_XXS) {
    // the unit's words start at block offset + 2 + 8 sub: the same alignment as + 2
    const uint32_t sh = (l.bp + 2u) & 3u;
    r.a0 = __builtin_amdgcn_alignbyte(l.a[1], l.a[0], sh);
    r.a1 = __builtin_amdgcn_alignbyte(l.a[2], l.a[1], sh);
    r.d = (l.bp & 2u) ? (l.dw >> 16) : (l.dw & 0xFFFFu);
  } else {
    r = l.r;
  }
}

template <int TYPE>
__device__ __forceinline__ void load_raw(Raw<TYPE> &r, const BufSrc &src, uint32_t bi, uint32_t sub) {
  RawLd<TYPE> l;
  issue_raw<TYPE>(l, src, bi, sub);
  finish_raw<TYPE>(l, r);
}

// 6-bit (scale, min) pair `idx` of a Q4_K block (SCALE_MIN_K4, kernels.wgsl.js:94-104).
// s1, s2, s3 are the block's scale bytes 0-3, 4-7 and 8-11 as little-endian words.
__device__ __forceinline__ void q4k_scale_min(uint32_t s1, uint32_t s2, uint32_t s3, uint32_t idx, uint32_t &sc,
                                              uint32_t &m) {
  const uint32_t sh = 8u * (idx & 3u);
  if (idx < 4) {
    sc = (s1 >> sh) & 63u;
    m = (s2 >> sh) & 63u;
  } else {
    const uint32_t a = (s3 >> sh) & 0xFFu;   // byte idx + 4
    const uint32_t b = (s1 >> sh) & 0xFFu;   // byte idx - 4
    const uint32_t c = (s2 >> sh) & 0xFFu;   // byte idx
    sc = (a & 0xFu) | ((b >> 6) << 4);
    m = (a >> 4) | ((c >> 6) << 4);
  }
}

// Unsigned values u of quad q (weights 4q..4q+3 of half A for q < 4, of half B
// for q >= 4), one per byte. `grid` is the IQ2_XXS table in LDS (u32 pairs).
template <int TYPE>
__device__ __forceinline__ uint32_t quad(const Raw<TYPE> &r, int q, const uint32_t *grid) {
  if constexpr (TYPE == Q8_0 || TYPE == Q8_0R) {
    return r.v[q] ^ 0x80808080u;  // signed byte + 128
  } else if constexpr (TYPE == Q4_K) {
    return q < 4 ? (r.qs[q] & 0x0F0F0F0Fu) : ((r.qs[q - 4] >> 4) & 0x0F0F0F0Fu);
  } else if constexpr (TYPE == Q6_K) {
    uint32_t gp = (r.sub >> 1) & 1u;
    if (q < 4) return (r.ql[q] & 0x0F0F0F0Fu) | (((r.qh[q] >> (2u * gp)) & 0x03030303u) << 4);
    return ((r.ql[q - 4] >> 4) & 0x0F0F0F0Fu) | (((r.qh[q - 4] >> (2u * gp + 4u)) & 0x03030303u) << 4);
  } else if constexpr (TYPE == Q2_K) {
    uint32_t jp = (r.sub >> 1) & 1u;
    return q < 4 ? ((r.qs[q] >> (4u * jp)) & 0x03030303u) : ((r.qs[q - 4] >> (4u * jp + 2u)) & 0x03030303u);
  } else {
    // entry l = q>>1 covers weights 8l..8l+7; this quad is its half (q&1)
    uint32_t l = (uint32_t)q >> 1;
    uint32_t gi = (r.a0 >> (8u * l)) & 0xFFu;
    uint32_t bits = (r.a1 >> (7u * l)) & 127u;
    uint32_t signs = bits | ((__builtin_popcount(bits) & 1u) << 7);  // even parity (kernels.wgsl.js:381-384)
    uint32_t g = grid[2u * gi + (q & 1)];
    uint32_t s4 = (signs >> (4u * (q & 1))) & 0xFu;
    uint32_t m = ((s4 * 0x00204081u) & 0x01010101u) * 0xFFu;  // 0xFF in each negative byte
    // +g -> g + 128 ; -g -> 128 - g, per byte, without carries between bytes
    return (g ^ (m ^ 0x80808080u)) + (m & 0x01010101u);
  }
}

// Scale and offset of the two halves: value_i = s * u_i - m.
template <int TYPE>
__device__ __forceinline__ void unit_scales(const Raw<TYPE> &r, float &sA, float &sB, float &mA, float &mB) {
  if constexpr (TYPE == Q8_0 || TYPE == Q8_0R) {
    float d = h2f(r.s);
    sA = sB = d;
    mA = mB = 128.f * d;
  } else if constexpr (TYPE == Q4_K) {
    float d = h2f(r.hdr[0] & 0xFFFFu), dmin = h2f(r.hdr[0] >> 16);
    uint32_t j = r.sub >> 1, sc, m;
    q4k_scale_min(r.hdr[1], r.hdr[2], r.hdr[3], 2u * j, sc, m);
    sA = d * (float)sc; mA = dmin * (float)m;
    q4k_scale_min(r.hdr[1], r.hdr[2], r.hdr[3], 2u * j + 1u, sc, m);
    sB = d * (float)sc; mB = dmin * (float)m;
  } else if constexpr (TYPE == Q6_K) {
    float d = h2f(r.d);
    sA = d * (float)(int8_t)(r.sc & 0xFFu);
    sB = d * (float)(int8_t)(r.sc >> 8);
    mA = 32.f * sA; mB = 32.f * sB;
  } else if constexpr (TYPE == Q2_K) {
    float d = h2f(r.dd & 0xFFFFu), dmin = h2f(r.dd >> 16);
    uint32_t half = r.sub & 1u;
    uint32_t scA = (r.sc >> (8u * half)) & 0xFFu, scB = (r.sc >> (8u * (half + 2u))) & 0xFFu;
    sA = d * (float)(scA & 0xFu); mA = dmin * (float)(scA >> 4);
    sB = d * (float)(scB & 0xFu); mB = dmin * (float)(scB >> 4);
  } else {
    float d = h2f(r.d);
    float db = d * (0.5f + (float)(r.a1 >> 28)) * 0.25f;
    sA = sB = db;
    mA = mB = 128.f * db;
  }
}

// Bit-exact f32 dequantization of one unit: out[0..15] = half A, out[16..31] =
// half B, with the reference's operation order and no FMA contraction.
template <int TYPE>
__device__ __forceinline__ void dequant_unit(const Raw<TYPE> &r, const uint32_t *grid, float *out) {
#pragma clang fp contract(off)
  if constexpr (TYPE == Q8_0 || TYPE == Q8_0R) {
    // f32(q) * d (kernels.wgsl.js:162-169, 857-865)
    float d = h2f(r.s);
#pragma unroll
    for (int i = 0; i < 32; ++i) out[i] = (float)(int8_t)((r.v[i >> 2] >> (8 * (i & 3))) & 0xFFu) * d;
  } else if constexpr (TYPE == Q4_K) {
    // d1 * q - m1 with d1 = d*sc, m1 = dmin*m (kernels.wgsl.js:233-249)
    float d = h2f(r.hdr[0] & 0xFFFFu), dmin = h2f(r.hdr[0] >> 16);
    uint32_t j = r.sub >> 1, sc, m;
    q4k_scale_min(r.hdr[1], r.hdr[2], r.hdr[3], 2u * j, sc, m);
    float d1 = d * (float)sc, m1 = dmin * (float)m;
    q4k_scale_min(r.hdr[1], r.hdr[2], r.hdr[3], 2u * j + 1u, sc, m);
    float d2 = d * (float)sc, m2 = dmin * (float)m;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t b = (r.qs[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      out[i] = d1 * (float)(b & 0xFu) - m1;
      out[16 + i] = d2 * (float)(b >> 4) - m2;
    }
  } else if constexpr (TYPE == Q6_K) {
    // (d * sc) * (q - 32) (kernels.wgsl.js:300-329)
    float d = h2f(r.d);
    float dA = d * (float)(int8_t)(r.sc & 0xFFu), dB = d * (float)(int8_t)(r.sc >> 8);
    uint32_t gp = (r.sub >> 1) & 1u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t l = (r.ql[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      uint32_t h = (r.qh[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      int qa = (int)((l & 0xFu) | (((h >> (2u * gp)) & 3u) << 4)) - 32;
      int qb = (int)((l >> 4) | (((h >> (2u * gp + 4u)) & 3u) << 4)) - 32;
      out[i] = dA * (float)qa;
      out[16 + i] = dB * (float)qb;
    }
  } else if constexpr (TYPE == Q2_K) {
    // dl * q - ml with dl = d*(sc&15), ml = dmin*(sc>>4) (kernels.wgsl.js:202-221)
    float d = h2f(r.dd & 0xFFFFu), dmin = h2f(r.dd >> 16);
    uint32_t half = r.sub & 1u, jp = (r.sub >> 1) & 1u;
    uint32_t scA = (r.sc >> (8u * half)) & 0xFFu, scB = (r.sc >> (8u * (half + 2u))) & 0xFFu;
    float dlA = d * (float)(scA & 0xFu), mlA = dmin * (float)(scA >> 4);
    float dlB = d * (float)(scB & 0xFu), mlB = dmin * (float)(scB >> 4);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t b = (r.qs[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      out[i] = dlA * (float)((b >> (4u * jp)) & 3u) - mlA;
      out[16 + i] = dlB * (float)((b >> (4u * jp + 2u)) & 3u) - mlB;
    }
  } else {
    // db * g * sign with db = d * (0.5 + ls) * 0.25 (kernels.wgsl.js:374-395)
    float d = h2f(r.d);
    float db = d * (0.5f + (float)(r.a1 >> 28)) * 0.25f;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      uint32_t gi = (r.a0 >> (8u * l)) & 0xFFu;
      uint32_t bits = (r.a1 >> (7u * l)) & 127u;
      uint32_t signs = bits | ((__builtin_popcount(bits) & 1u) << 7);
      uint32_t g0 = grid[2u * gi], g1 = grid[2u * gi + 1u];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t gw = j < 4 ? g0 : g1;
        float gv = (float)((gw >> (8 * (j & 3))) & 0xFFu);
        float sg = (signs >> j) & 1u ? -1.0f : 1.0f;
        out[8 * l + j] = db * gv * sg;
      }
    }
  }
}

template <int TYPE>
__device__ __forceinline__ void stage_grid(uint32_t *grid) {
  if constexpr (TYPE == IQ2_XXS) {
    for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) {
      uint64_t g = c_iq2xxs_grid[i];
      grid[2 * i] = (uint32_t)g;
      grid[2 * i + 1] = (uint32_t)(g >> 32);
    }
  }
}

// ---------------------------------------------------------------------------
// Dequantization (test hook): one thread per unit.
template <int TYPE>
__global__ __launch_bounds__(256) void k_dequant(WeightView wv, uint32_t n_blocks, float *__restrict__ out) {
  __shared__ uint32_t grid[TYPE == IQ2_XXS ? 512 : 1];
  stage_grid<TYPE>(grid);
  if constexpr (TYPE == IQ2_XXS) __syncthreads();
  constexpr uint32_t upb = units_per_block<TYPE>();
  const uint64_t first = (uint64_t)blockIdx.x * 256u / upb;   // first block of this workgroup
  const BufSrc src = make_src(wv, first);
  uint64_t gu = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gu >= (uint64_t)n_blocks * upb) return;
  uint64_t bi = gu / upb;
  uint32_t sub = (uint32_t)(gu % upb);
  Raw<TYPE> r;
  load_raw<TYPE>(r, src, (uint32_t)(bi - first), sub);
  float v[32];
  dequant_unit<TYPE>(r, grid, v);
  uint32_t o0, o1;
  unit_runs<TYPE>(sub, o0, o1);
  float *dst = out + bi * block_elems<TYPE>();
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    *(float4 *)(dst + o0 + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    *(float4 *)(dst + o1 + i) = make_float4(v[16 + i], v[17 + i], v[18 + i], v[19 + i]);
  }
}

// ---------------------------------------------------------------------------
// Embedding gather (quant.gather, ops.js:1104-1118; gatherShader,
// kernels.wgsl.js:1188-1221): out[t][:] = the dequantized row ids[t] of W,
// decoded a unit at a time by the same decoder as k_dequant (bit-identical to
// it). Rows are read through the buffer descriptor, so an id past the table
// reads zeros. One thread per (token, unit).
template <int TYPE>
__global__ __launch_bounds__(256) void k_gather(WeightView wv, const uint32_t *__restrict__ ids, uint32_t tokens,
                                                float *__restrict__ out) {
  __shared__ uint32_t grid[TYPE == IQ2_XXS ? 512 : 1];
  stage_grid<TYPE>(grid);
  if constexpr (TYPE == IQ2_XXS) __syncthreads();
  constexpr uint32_t upb = units_per_block<TYPE>();
  const uint32_t upr = wv.bpr * upb;  // units per row
  const uint64_t gu = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (gu >= (uint64_t)tokens * upr) return;
  const uint32_t t = (uint32_t)(gu / upr), u = (uint32_t)(gu % upr), b = u / upb, sub = u % upb;
  const BufSrc src = make_src(wv, 0);
  Raw<TYPE> r;
  load_raw<TYPE>(r, src, ids[t] * wv.bpr + b, sub);
  float v[32];
  dequant_unit<TYPE>(r, grid, v);
  uint32_t o0, o1;
  unit_runs<TYPE>(sub, o0, o1);
  float *dst = out + (uint64_t)t * wv.k + (uint64_t)b * block_elems<TYPE>();
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    *(float4 *)(dst + o0 + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    *(float4 *)(dst + o1 + i) = make_float4(v[16 + i], v[17 + i], v[18 + i], v[19 + i]);
  }
}

// Gather + the first layer's RMS norm (gatherNormaShader,
// kernels.fusion.wgsl.js:164-206): one workgroup per token writes the row to
// x and nrm = x * (1 / sqrt(sum(x^2) / dim + eps)) * wn. The row stays in LDS
// between the two phases; the squares are summed per thread over the columns
// c = tid + 256 j, then across the workgroup in a fixed order.
template <int TYPE>
__global__ __launch_bounds__(256) void k_gather_norm(WeightView wv, const uint32_t *__restrict__ ids,
                                                     const float *__restrict__ wn, float eps, float *__restrict__ x,
                                                     float *__restrict__ nrm) {
  extern __shared__ __align__(16) float row[];
  __shared__ float part[256];
  __shared__ uint32_t grid[TYPE == IQ2_XXS ? 512 : 1];
  stage_grid<TYPE>(grid);
  if constexpr (TYPE == IQ2_XXS) __syncthreads();
  constexpr uint32_t upb = units_per_block<TYPE>();
  const uint32_t t = blockIdx.x, tid = threadIdx.x, dim = wv.k, upr = wv.bpr * upb;
  const uint32_t id = ids[t];
  const BufSrc src = make_src(wv, 0);
  for (uint32_t u = tid; u < upr; u += 256u) {
    const uint32_t b = u / upb, sub = u % upb;
    Raw<TYPE> r;
    load_raw<TYPE>(r, src, id * wv.bpr + b, sub);
    float v[32];
    dequant_unit<TYPE>(r, grid, v);
    uint32_t o0, o1;
    unit_runs<TYPE>(sub, o0, o1);
    float *dl = row + b * block_elems<TYPE>();
    float *dg = x + (uint64_t)t * dim + b * block_elems<TYPE>();
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 a = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
      const float4 c = make_float4(v[16 + i], v[17 + i], v[18 + i], v[19 + i]);
      *(float4 *)(dl + o0 + i) = a;
      *(float4 *)(dl + o1 + i) = c;
      *(float4 *)(dg + o0 + i) = a;
      *(float4 *)(dg + o1 + i) = c;
    }
  }
  __syncthreads();
  float acc = 0.f;
  for (uint32_t c = tid; c < dim; c += 256u) acc = __builtin_fmaf(row[c], row[c], acc);
  part[tid] = acc;
  __syncthreads();
  for (uint32_t off = 128u; off > 0u; off >>= 1) {
    if (tid < off) part[tid] += part[tid + off];
    __syncthreads();
  }
  const float scale = 1.0f / sqrtf(part[0] / (float)dim + eps);
  float *dn = nrm + (uint64_t)t * dim;
  for (uint32_t c = tid; c < dim; c += 256u) dn[c] = row[c] * scale * wn[c];
}

// ---------------------------------------------------------------------------
// GEMV: Y[t][row] = sum_k W[row][k] X[t][k], 1..8 tokens, f32 accumulation.
//
// A workgroup is 4 waves arranged as G = 4/S row groups x S slices of k. Each
// wave owns R rows of its group and one slice of k; its lanes walk the units
// of the slice, so each x value is loaded once per R rows (from the L1/L2
// cache: x is small and read by every workgroup). The weight loads of a unit
// are issued first. Slices of one row group are added in slice order through
// LDS, so the result does not depend on scheduling.
template <int TYPE, int T, int R>
__global__ __launch_bounds__(256) void k_gemv(WeightView wv, const float *__restrict__ x,
                                              float *__restrict__ y, int S) {
  __shared__ uint32_t grid[TYPE == IQ2_XXS ? 512 : 1];
  __shared__ float red[4 * R * T];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = 4 / S, g = wave / S, sl = wave % S;
  const uint32_t rows = wv.rows, k = wv.k;
  const uint32_t trow0 = blockIdx.x * (uint32_t)(G * R);     // first row of the tile
  const uint32_t row0 = trow0 + (uint32_t)(g * R);          // first row of this wave

  if constexpr (TYPE == IQ2_XXS) {
    stage_grid<TYPE>(grid);
    __syncthreads();
  }
  const BufSrc src = make_src(wv, (uint64_t)trow0 * wv.bpr);

  uint32_t lrow[R];  // row of the tile (clamped into the matrix)
#pragma unroll
  for (int r = 0; r < R; ++r) lrow[r] = min(row0 + (uint32_t)r, rows - 1u) - trow0;

  float acc[R][T];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[r][t] = 0.f;

  constexpr uint32_t upb = units_per_block<TYPE>();
  constexpr uint32_t E = block_elems<TYPE>();
  const uint32_t units = k / 32u;
  const uint32_t ub = units / (uint32_t)S * (uint32_t)sl, ue = units / (uint32_t)S * (uint32_t)(sl + 1);

  for (uint32_t gu = ub + (uint32_t)lane; gu < ue; gu += 64u) {
    const uint32_t b = gu / upb, sub = gu % upb;
    uint32_t o0, o1;
    unit_runs<TYPE>(sub, o0, o1);
    const uint32_t k0 = b * E + o0, k1 = b * E + o1;

    Raw<TYPE> raw[R];
#pragma unroll
    for (int r = 0; r < R; ++r) load_raw<TYPE>(raw[r], src, lrow[r] * wv.bpr + b, sub);

    if constexpr (T <= 2) {
      // Scales factored out of the unit: value = s*u - m per half.
      float4 xa[T][4], xb[T][4];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          xa[t][q] = *(const float4 *)(x + (uint64_t)t * k + k0 + 4 * q);
          xb[t][q] = *(const float4 *)(x + (uint64_t)t * k + k1 + 4 * q);
        }
      float sxa[T], sxb[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        float a = 0.f, bb = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a += (xa[t][q].x + xa[t][q].y) + (xa[t][q].z + xa[t][q].w);
          bb += (xb[t][q].x + xb[t][q].y) + (xb[t][q].z + xb[t][q].w);
        }
        sxa[t] = a; sxb[t] = bb;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float ra[T], rb[T];
#pragma unroll
        for (int t = 0; t < T; ++t) ra[t] = rb[t] = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t qb = quad<TYPE>(raw[r], q, grid);
          const float f0 = ubyte(qb, 0), f1 = ubyte(qb, 1), f2 = ubyte(qb, 2), f3 = ubyte(qb, 3);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const float4 xv = q < 4 ? xa[t][q] : xb[t][q - 4];
            float &a = q < 4 ? ra[t] : rb[t];
            a = __builtin_fmaf(f0, xv.x, a);
            a = __builtin_fmaf(f1, xv.y, a);
            a = __builtin_fmaf(f2, xv.z, a);
            a = __builtin_fmaf(f3, xv.w, a);
          }
        }
        float sA, sB, mA, mB;
        unit_scales<TYPE>(raw[r], sA, sB, mA, mB);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float v = acc[r][t];
          v = __builtin_fmaf(sA, ra[t], v);
          v = __builtin_fmaf(sB, rb[t], v);
          v = __builtin_fmaf(-mA, sxa[t], v);
          acc[r][t] = __builtin_fmaf(-mB, sxb[t], v);
        }
      }
    } else {
      // Many tokens: each weight is formed once (s*u - m) and used T times.
      float sA[R], sB[R], mA[R], mB[R];
#pragma unroll
      for (int r = 0; r < R; ++r) unit_scales<TYPE>(raw[r], sA[r], sB[r], mA[r], mB[r]);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t kq = q < 4 ? k0 + 4 * q : k1 + 4 * (q - 4);
        float4 xv[T];
#pragma unroll
        for (int t = 0; t < T; ++t) xv[t] = *(const float4 *)(x + (uint64_t)t * k + kq);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t qb = quad<TYPE>(raw[r], q, grid);
          const float s = q < 4 ? sA[r] : sB[r], m = q < 4 ? mA[r] : mB[r];
          const float w0 = __builtin_fmaf(s, ubyte(qb, 0), -m), w1 = __builtin_fmaf(s, ubyte(qb, 1), -m);
          const float w2 = __builtin_fmaf(s, ubyte(qb, 2), -m), w3 = __builtin_fmaf(s, ubyte(qb, 3), -m);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            float a = acc[r][t];
            a = __builtin_fmaf(w0, xv[t].x, a);
            a = __builtin_fmaf(w1, xv[t].y, a);
            a = __builtin_fmaf(w2, xv[t].z, a);
            acc[r][t] = __builtin_fmaf(w3, xv[t].w, a);
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[r][t] = wave_sum(acc[r][t]);

  if (S == 1) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < rows)
#pragma unroll
          for (int t = 0; t < T; ++t) y[(uint64_t)t * rows + row0 + r] = acc[r][t];
    }
    return;
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) red[(wave * R + r) * T + t] = acc[r][t];
  }
  __syncthreads();
  if (tid < G * R * T) {
    const int gg = tid / (R * T), rt = tid % (R * T), r = rt / T, t = rt % T;
    float v = 0.f;
    for (int q = 0; q < S; ++q) v += red[((gg * S + q) * R + r) * T + t];
    const uint32_t row = trow0 + (uint32_t)(gg * R + r);
    if (row < rows) y[(uint64_t)t * rows + row] = v;
  }
}

// ---------------------------------------------------------------------------
// GEMM: Y[t][row] = sum_k fp16(W[row][k]) fp16(X[t][k]), fp32 accumulation.
//
// x is rounded to fp16 once by k_x_to_f16; the tile kernel (k_gemm, below)
// stages fp16 x and dequantized fp16 W through LDS for the MFMAs.
// Weights are dequantized to fp16: Q8_0/Q8_0R with packed fp16 arithmetic
// (q exact, then one rounding of q*d, i.e. fp16(d*q)), the other types as
// the bit-exact f32 value rounded to fp16.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

template <int TYPE> constexpr int gemm_bk() { return TYPE == Q6_K ? 128 : 64; }

// One thread per 8 halves of the output, laid out as [token tile][k step]
// [BM tokens][BK k]: the x slice of one tile and k step is one contiguous
// run of BM * BK halves. Tokens past `tokens` and k past `k` are zero. The
// grid's y dimension is the token tile (no division in the indexing, which
// precedes the loads).
__global__ __launch_bounds__(256) void k_x_to_f16(const float *__restrict__ x, _Float16 *__restrict__ xh,
                                                  uint32_t tokens, uint32_t k, uint32_t bm_log2, uint32_t bk_log2,
                                                  uint32_t steps) {
  const uint32_t sh = bm_log2 + bk_log2 - 3u;                 // log2 of half8 per (tile, step)
  const uint32_t ot = blockIdx.x * 256u + threadIdx.x, tile = blockIdx.y;
  if (ot >= (steps << sh)) return;
  const uint64_t o = ((uint64_t)tile * steps << sh) + ot;
  const uint32_t st = ot >> sh, in = ot & ((1u << sh) - 1u);
  const uint32_t t = in >> (bk_log2 - 3u), c = in & ((1u << (bk_log2 - 3u)) - 1u);
  const uint32_t tok = (tile << bm_log2) + t, kk = (st << bk_log2) + 8u * c;
  half8 h = {};
  if (tok < tokens && kk < k) {   // k is a multiple of 32, so all 8 values exist
    const float4 a = *(const float4 *)(x + (uint64_t)tok * k + kk);
    const float4 b = *(const float4 *)(x + (uint64_t)tok * k + kk + 4);
    h[0] = (_Float16)a.x; h[1] = (_Float16)a.y; h[2] = (_Float16)a.z; h[3] = (_Float16)a.w;
    h[4] = (_Float16)b.x; h[5] = (_Float16)b.y; h[6] = (_Float16)b.z; h[7] = (_Float16)b.w;
  }
  *(half8 *)(xh + 8 * o) = h;
}

// 32 fp16 weights of a unit: out[0..15] half A, out[16..31] half B.
template <int TYPE>
__device__ __forceinline__ void unit_f16(const Raw<TYPE> &r, const uint32_t *grid, half8 *out) {
  if constexpr (TYPE == Q8_0 || TYPE == Q8_0R) {
    // q+128 as a byte -> fp16 1024+(q+128) by placing 0x64 above it, minus
    // 1152 (exact), times d (one rounding).
    const uint32_t magic = 0x64646464u;
    const half2v d2 = {__builtin_bit_cast(_Float16, (uint16_t)r.s), __builtin_bit_cast(_Float16, (uint16_t)r.s)};
    const half2v off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      half8 h;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t u = r.v[2 * i + j] ^ 0x80808080u;
        const half2v lo = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(magic, u, 0x04010400u));
        const half2v hi = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(magic, u, 0x04030402u));
        const half2v a = (lo + off) * d2, b = (hi + off) * d2;
        h[4 * j] = a.x; h[4 * j + 1] = a.y; h[4 * j + 2] = b.x; h[4 * j + 3] = b.y;
      }
      out[i] = h;
    }
  } else {
    float v[32];
    dequant_unit<TYPE>(r, grid, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      half8 h;
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = (_Float16)v[8 * i + j];
      out[i] = h;
    }
  }
}

// Tile: BM tokens x BN rows in k steps of BK, 8 waves in two roles:
//  * 4 producer waves load the x and W bytes of step s+3 into registers (three
//    register sets: loads have three steps to arrive) and write step s+1 into
//    LDS as fp16 (W dequantized);
//  * 4 MFMA waves, CM x CN x CK, compute step s from LDS: each owns FM x FN
//    32x32x16 fragments of (BM/CM) x (BN/CN) over 1/CK of every k step (CK > 1:
//    the shares are added through LDS at the end).
// One producer and one MFMA wave share each SIMD, so dequantization and loads
// overlap the MFMAs; one barrier per step hands a stage over. Tiles are dealt
// so that the workgroups of one XCD cover a contiguous run of row tiles with
// all their token tiles: the x and W slices of a k step are shared through
// that XCD's L2.
template <int TYPE, int BM, int BN, int BK, int CM, int CN, int CK, int NS>
__global__ __launch_bounds__(512) void k_gemm(WeightView wv, const _Float16 *__restrict__ xh,
                                              float *__restrict__ y, uint32_t tokens, uint32_t row_tiles,
                                              uint32_t tok_tiles) {
  static_assert(CM * CN * CK == 4, "4 MFMA waves");
  constexpr int PT = 256;                     // producer threads
  constexpr int BKP = BK + 8;                 // padded LDS row (halves)
  constexpr int FM = BM / CM / 32, FN = BN / CN / 32, KS = BK / 16 / CK;
  static_assert(FM >= 1 && FN >= 1 && KS >= 1, "tile");
  extern __shared__ __align__(16) uint8_t gsm[];
  _Float16 *const xs0 = (_Float16 *)gsm, *const xs1 = xs0 + BM * BKP;
  _Float16 *const ws0 = xs1 + BM * BKP, *const ws1 = ws0 + BN * BKP;
  constexpr size_t kStages = (size_t)2 * (BM + BN) * BKP * 2, kRed = CK > 1 ? (size_t)BM * BN * 4 : 0;
  uint32_t *const grid = (uint32_t *)(gsm + (kStages > kRed ? kStages : kRed));
  stage_grid<TYPE>(grid);

  const uint32_t ntiles = row_tiles * tok_tiles;
  uint32_t lin = blockIdx.x;
  if (ntiles % 8 == 0) lin = (blockIdx.x % 8) * (ntiles / 8) + blockIdx.x / 8;
  const uint32_t n0 = (lin / tok_tiles) * BN, t0 = (lin % tok_tiles) * BM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool producer = wave >= 4;
  const int ptid = tid - 256;                 // producer thread index
  const uint32_t rows = wv.rows, k = wv.k;
  const int ck = wave % CK, cn = (wave / CK) % CN, cm = (wave / (CK * CN)) % CM;
  constexpr uint32_t upb = units_per_block<TYPE>();
  constexpr uint32_t E = block_elems<TYPE>();
  const BufSrc src = make_src(wv, (uint64_t)n0 * wv.bpr);
  const uint32_t steps = (k + BK - 1) / BK, last = steps - 1u;
  // fp16 x of this token tile: steps runs of BM x BK halves (zero-padded)
  const rsrc_t xsrc = make_rsrc(xh + (uint64_t)(t0 / BM) * steps * BM * BK, (uint64_t)steps * BM * BK * 2u);

  constexpr int UNITS_ALL = BN * (BK / 32);                   // weight units per step
  constexpr int UNITS = (UNITS_ALL + PT - 1) / PT;
  constexpr int XCH = BM * (BK / 8) / PT;                     // 8-half x chunks per producer thread
  static_assert(XCH * PT == BM * (BK / 8), "x chunks");
  struct Regs {
    RawLd<TYPE> raw[UNITS];
    half8 xr[XCH];
  };

  auto load_step = [&](uint32_t kb, Regs &R) {
    const uint32_t klen = min((uint32_t)BK, k - kb);
#pragma unroll
    for (int i = 0; i < UNITS; ++i) {
      const int id = ptid + PT * i;
      if (UNITS_ALL % PT != 0 && id >= UNITS_ALL) break;
      const int r = id / (BK / 32);
      const uint32_t u = (uint32_t)(id % (BK / 32));
      const uint32_t lrow = min(n0 + (uint32_t)r, rows - 1u) - n0;
      const uint32_t gu = kb / 32u + min(u, klen / 32u - 1u);
      issue_raw<TYPE>(R.raw[i], src, lrow * wv.bpr + gu / upb, gu % upb);
    }
    // contiguous: thread id takes halves 8 id .. 8 id + 7 of the step's run
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const uint32_t off = (kb / BK) * (uint32_t)(BM * BK * 2) + 16u * (uint32_t)(ptid + PT * i);
      R.xr[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(xsrc, (int)off, 0, 0));
    }
  };
  auto store_step = [&](uint32_t kb, const Regs &R, _Float16 *xs, _Float16 *ws) {
    const uint32_t klen = min((uint32_t)BK, k - kb);
#pragma unroll
    for (int i = 0; i < UNITS; ++i) {
      const int id = ptid + PT * i;
      if (UNITS_ALL % PT != 0 && id >= UNITS_ALL) break;
      const int r = id / (BK / 32);
      const uint32_t u = (uint32_t)(id % (BK / 32));
      _Float16 *d = ws + r * BKP;
      if (u >= klen / 32u) {
        const half8 z = {};
#pragma unroll
        for (int j = 0; j < 4; ++j) *(half8 *)(d + 32 * u + 8 * j) = z;
        continue;
      }
      const uint32_t gu = kb / 32u + u;
      uint32_t o0, o1;
      unit_runs<TYPE>(gu % upb, o0, o1);
      const uint32_t c0 = (gu / upb) * E + o0 - kb, c1 = (gu / upb) * E + o1 - kb;
      Raw<TYPE> raw;
      finish_raw<TYPE>(R.raw[i], raw);
      half8 h[4];
      unit_f16<TYPE>(raw, grid, h);
      *(half8 *)(d + c0) = h[0];
      *(half8 *)(d + c0 + 8) = h[1];
      *(half8 *)(d + c1) = h[2];
      *(half8 *)(d + c1 + 8) = h[3];
    }
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int id = ptid + PT * i;
      const int t = id / (BK / 8), c = id % (BK / 8);
      *(half8 *)(xs + t * BKP + 8 * c) = R.xr[i];
    }
  };

  float16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Fragments of 16-k substep ks; the next substep's are read while the
  // current one's MFMAs run (two register sets).
  auto frag = [&](const _Float16 *xa, const _Float16 *wa, int ks, half8 *a, half8 *bfr) {
    const int kq = (ck * KS + ks) * 16 + 8 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < FM; ++i) a[i] = *(const half8 *)(xa + ((cm * FM + i) * 32 + (lane & 31)) * BKP + kq);
#pragma unroll
    for (int j = 0; j < FN; ++j) bfr[j] = *(const half8 *)(wa + ((cn * FN + j) * 32 + (lane & 31)) * BKP + kq);
  };
  auto mma = [&](const _Float16 *xa, const _Float16 *wa) {
    half8 a[2][FM], bfr[2][FN];
    frag(xa, wa, 0, a[0], bfr[0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) frag(xa, wa, ks + 1, a[(ks + 1) & 1], bfr[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the MFMAs
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks & 1][i], bfr[ks & 1][j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if constexpr (TYPE == IQ2_XXS) __syncthreads();  // grid staged
  if (producer) {
    // Producer: NS register sets, loads never skipped (past the last step
    // they repeat it), so each wait covers exactly the oldest set; the loads
    // of a step go out NS - 1 steps before it is written to LDS.
    Regs R[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) load_step(min((uint32_t)j, last) * BK, R[j]);
    store_step(0, R[0], xs0, ws0);
    load_step(min((uint32_t)NS, last) * BK, R[0]);
    __syncthreads();
    for (uint32_t st = 0; st < steps; st += NS) {
#pragma unroll
      for (int j = 1; j <= NS; ++j) {
        // during step st + j - 1: step st + j goes to the other stage
        const uint32_t sj = st + (uint32_t)j;
        if (sj < steps) store_step(sj * BK, R[j % NS], (sj & 1) ? xs1 : xs0, (sj & 1) ? ws1 : ws0);
        load_step(min(sj + (uint32_t)NS, last) * BK, R[j % NS]);
        if (sj - 1u < steps) __syncthreads();
      }
    }
  } else {
    __syncthreads();
    for (uint32_t st = 0; st < steps; ++st) {
      mma((st & 1) ? xs1 : xs0, (st & 1) ? ws1 : ws0);
      __syncthreads();
    }
  }

  // k shares of the same fragments are added through LDS (the stages are free)
  if constexpr (CK > 1) {
    float *red = (float *)gsm;
    const int pair = cm * CN + cn;
    for (int q = 1; q < CK; ++q) {
      if (!producer && ck == q) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              red[(((pair * FM + i) * FN + j) * 16 + v) * 64 + lane] = acc[i][j][v];
      }
      __syncthreads();
      if (!producer && ck == 0) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] += red[(((pair * FM + i) * FN + j) * 16 + v) * 64 + lane];
      }
      __syncthreads();
    }
  }
  if (producer || ck != 0) return;

  // D[tok][row]: lane holds column (row) lane%32 and rows (tokens)
  // 8*(v/4) + 4*(lane/32) + v%4 of each 32x32 fragment.
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t row = n0 + (cn * FN + j) * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t tok = t0 + (cm * FM + i) * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < rows && tok < tokens) y[(uint64_t)tok * rows + row] = acc[i][j][v];
      }
    }
}

// ---------------------------------------------------------------------------
// Host-side launchers.

GemvPlan plan_gemv(const WeightView &wv, uint32_t tokens) {
  GemvPlan p{};
  p.rows_per_wave = 4;
  const uint32_t E = geometry(wv.type).elems;
  // Split k over the 4 waves while row tiles alone give fewer than 512
  // workgroups, keeping every slice a whole number of blocks and at least 64
  // units (one per lane).
  int S = 1;
  auto tiles = [&](int s) { uint32_t per = (uint32_t)(4 / s) * (uint32_t)p.rows_per_wave; return (wv.rows + per - 1) / per; };
  while (S < 4 && tiles(S) < 512u && wv.k % (uint32_t)(2 * S) == 0 && (wv.k / (uint32_t)(2 * S)) % E == 0 &&
         wv.k / (uint32_t)(2 * S) >= 2048u)
    S *= 2;
  p.ksplit = S;
  p.kc = wv.k / (uint32_t)S;
  p.tiles = tiles(S);
  p.grid = p.tiles;
  p.lds_bytes = 0;
  return p;
}

template <int TYPE, int T>
static hipError_t gemv_go(const WeightView &wv, const float *x, float *y, const GemvPlan &p, hipStream_t s) {
  hipLaunchKernelGGL((k_gemv<TYPE, T, 4>), dim3(p.grid), dim3(256), 0, s, wv, x, y, p.ksplit);
  return hipGetLastError();
}

template <int TYPE>
static hipError_t gemv_t(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                         hipStream_t s) {
  switch (tokens) {
    case 1: return gemv_go<TYPE, 1>(wv, x, y, p, s);
    case 2: return gemv_go<TYPE, 2>(wv, x, y, p, s);
    case 3: return gemv_go<TYPE, 3>(wv, x, y, p, s);
    case 4: return gemv_go<TYPE, 4>(wv, x, y, p, s);
    case 5: return gemv_go<TYPE, 5>(wv, x, y, p, s);
    case 6: return gemv_go<TYPE, 6>(wv, x, y, p, s);
    case 7: return gemv_go<TYPE, 7>(wv, x, y, p, s);
    case 8: return gemv_go<TYPE, 8>(wv, x, y, p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                       hipStream_t s) {
  switch (wv.type) {
    case Q8_0: return gemv_t<Q8_0>(wv, x, y, tokens, p, s);
    case Q8_0R: return gemv_t<Q8_0R>(wv, x, y, tokens, p, s);
    case Q4_K: return gemv_t<Q4_K>(wv, x, y, tokens, p, s);
    case Q6_K: return gemv_t<Q6_K>(wv, x, y, tokens, p, s);
    case Q2_K: return gemv_t<Q2_K>(wv, x, y, tokens, p, s);
    case IQ2_XXS: return gemv_t<IQ2_XXS>(wv, x, y, tokens, p, s);
    default: return hipErrorInvalidValue;
  }
}

// Register sets of the producer waves: as many as fit beside the MFMA
// waves' accumulators (both roles share one register allocation of 256).
template <int TYPE, int BM, int BN, int BK>
constexpr int gemm_sets() {
  constexpr int units = (BN * (BK / 32) + 255) / 256, xwords = 4 * (BM * (BK / 8) / 256);
  constexpr int set = xwords + units * (int)(sizeof(RawLd<TYPE>) / 4);
  constexpr int ns = 180 / set;
  return ns < 3 ? 3 : ns > 5 ? 5 : ns;
}

template <int TYPE, int BM, int BN, int BK, int CM, int CN, int CK>
static hipError_t gemm_cfg(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, hipStream_t s) {
  // two operand stages, or the fragments of the k shares at the end (BM * BN
  // floats, in the same space), whichever is larger; then the IQ2_XXS grid
  constexpr size_t stages = (size_t)2 * (BM + BN) * (BK + 8) * 2, red = CK > 1 ? (size_t)BM * BN * 4 : 0;
  constexpr size_t lds = (stages > red ? stages : red) + (TYPE == IQ2_XXS ? 2048 : 0);
  constexpr int NS = gemm_sets<TYPE, BM, BN, BK>();
  static_assert(lds <= 160 * 1024, "LDS");
  static std::atomic<uint64_t> attr{0};
  const hipError_t e = lds_limit_once((const void *)k_gemm<TYPE, BM, BN, BK, CM, CN, CK, NS>, (int)lds, attr);
  if (e != hipSuccess) return e;
  const uint32_t tok_tiles = (tokens + BM - 1) / BM, row_tiles = (wv.rows + BN - 1) / BN;
  hipLaunchKernelGGL((k_gemm<TYPE, BM, BN, BK, CM, CN, CK, NS>), dim3(row_tiles * tok_tiles), dim3(512), lds, s, wv, xh,
                     y, tokens, row_tiles, tok_tiles);
  return hipGetLastError();
}

// Tile by size: 256 x 128 tokens x rows for >= 1024 tokens (k steps of 64;
// Q6_K units need steps of 128), 128 x 128 from 256 tokens, else 128 tokens x
// 32 rows (small token counts are bound by the weight bytes; narrow tiles
// spread them over the CUs).
static bool gemm_wide(int type, uint32_t tokens) { return type != Q6_K && tokens >= 1024; }

// The configuration is chosen by `plan` (the token count of the batch the
// plan is made for) and run over `tokens` <= plan tokens: each output row
// depends only on its x row and W, summed in the configuration's order, so a
// run over fewer tokens gives the bits the same rows get in the whole batch.
template <int TYPE>
static hipError_t gemm_go(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, uint32_t plan,
                          hipStream_t s) {
  if constexpr (TYPE != Q6_K) {
    if (gemm_wide(TYPE, plan)) return gemm_cfg<TYPE, 256, 128, 64, 2, 2, 1>(wv, xh, y, tokens, s);
  }
  if (plan >= 256) return gemm_cfg<TYPE, 128, 128, 128, 2, 1, 2>(wv, xh, y, tokens, s);
  return gemm_cfg<TYPE, 128, 32, 128, 1, 1, 4>(wv, xh, y, tokens, s);
}

// Token tile and k step of the chosen configuration (log2), as the x layout needs them.
static void gemm_x_tile(int type, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg, uint32_t &bm_log2,
                        uint32_t &bk_log2) {
  if (gemm_big_applies(type, plan, k, rows)) {
    bm_log2 = gemm_big_tile_log2(plan, k, rows, cfg);
    bk_log2 = 6;
  } else if (gemm_wide(type, plan)) {
    bm_log2 = 8; bk_log2 = 6;
  } else {
    bm_log2 = 7; bk_log2 = 7;
  }
}

size_t gemm_x_bytes(int type, uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg) {
  uint32_t bm, bk;
  gemm_x_tile(type, plan, k, rows, cfg, bm, bk);
  const uint64_t tiles = (tokens + (1u << bm) - 1) >> bm, steps = (k + (1u << bk) - 1) >> bk;
  return (size_t)(tiles * steps) << (bm + bk + 1);
}

uint32_t gemm_x_layout(int type, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg) {
  uint32_t bm, bk;
  gemm_x_tile(type, plan, k, rows, cfg, bm, bk);
  return (bm << 4) | bk;
}

hipError_t launch_gemm_x(int type, const float *x, uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows,
                         uint32_t cfg, void *xh, hipStream_t s) {
  if (plan < tokens) return hipErrorInvalidValue;
  uint32_t bm, bk;
  gemm_x_tile(type, plan, k, rows, cfg, bm, bk);
  const uint32_t steps = (k + (1u << bk) - 1) >> bk, tiles = (tokens + (1u << bm) - 1) >> bm;
  const uint64_t per_tile = (uint64_t)steps << (bm + bk - 3u);   // half8 per token tile
  if (per_tile >= (1ull << 32)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_x_to_f16, dim3((uint32_t)((per_tile + 255) / 256), tiles), dim3(256), 0, s, x,
                     (_Float16 *)xh, tokens, k, bm, bk, steps);
  return hipGetLastError();
}

size_t gemm_sk_bytes(int type, uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg,
                     uint32_t ksl_opt) {
  return gemm_big_applies(type, plan, k, rows) ? gemm_big_scratch_bytes(tokens, plan, k, rows, cfg, ksl_opt) : 0;
}

hipError_t launch_gemm(const WeightView &wv, const float *x, float *y, uint32_t tokens, uint32_t plan,
                       uint32_t cfg, uint32_t ksl_opt, void *xh_scratch, void *sk_scratch, hipStream_t s) {
  const hipError_t e = launch_gemm_x(wv.type, x, tokens, plan, wv.k, wv.rows, cfg, xh_scratch, s);
  if (e != hipSuccess) return e;
  return launch_gemm_prepared(wv, (const _Float16 *)xh_scratch, y, tokens, plan, cfg, ksl_opt, sk_scratch, s);
}

hipError_t launch_gemm_prepared(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, uint32_t plan,
                                uint32_t cfg, uint32_t ksl_opt, void *sk_scratch, hipStream_t s) {
  if (plan < tokens) return hipErrorInvalidValue;
  if (gemm_big_applies(wv.type, plan, wv.k, wv.rows))
    return launch_gemm_big(wv, xh, y, tokens, plan, cfg, ksl_opt, sk_scratch, s);
  switch (wv.type) {
    case Q8_0: return gemm_go<Q8_0>(wv, xh, y, tokens, plan, s);
    case Q8_0R: return gemm_go<Q8_0R>(wv, xh, y, tokens, plan, s);
    case Q4_K: return gemm_go<Q4_K>(wv, xh, y, tokens, plan, s);
    case Q6_K: return gemm_go<Q6_K>(wv, xh, y, tokens, plan, s);
    case Q2_K: return gemm_go<Q2_K>(wv, xh, y, tokens, plan, s);
    case IQ2_XXS: return gemm_go<IQ2_XXS>(wv, xh, y, tokens, plan, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE>
static hipError_t dequant_go(const WeightView &wv, uint32_t n_blocks, float *out, hipStream_t s) {
  uint64_t units = (uint64_t)n_blocks * units_per_block<TYPE>();
  uint32_t grid = (uint32_t)((units + 255) / 256);
  hipLaunchKernelGGL((k_dequant<TYPE>), dim3(grid), dim3(256), 0, s, wv, n_blocks, out);
  return hipGetLastError();
}

// Streaming read of `bytes` bytes (the floor the GEMVs are measured against):
// workgroup b reads the contiguous chunk [b chunk, (b + 1) chunk) with 16-byte
// loads, U in flight per lane, and folds them with XOR. sink[b] is written only
// when the fold equals `magic`, so the loads stay and nothing is written in
// practice.
template <int U>
__global__ __launch_bounds__(256) void k_read_floor(const uint8_t *__restrict__ src, uint64_t bytes, uint32_t chunk,
                                                    uint32_t *__restrict__ sink, uint32_t magic) {
  const uint64_t base = (uint64_t)blockIdx.x * chunk;
  if (base >= bytes) return;
  const uint32_t n = (uint32_t)min<uint64_t>(bytes - base, chunk);
  const rsrc_t r = make_rsrc(src + base, n);
  uint32_t acc = 0;
  for (uint32_t o = threadIdx.x * 16u; o < n; o += 256u * 16u * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(o + 4096u * u), 0, 0));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == magic) sink[blockIdx.x] = acc;
}

hipError_t launch_read_floor(const uint8_t *src, uint64_t bytes, uint32_t workgroups, uint32_t unroll, uint32_t *sink,
                             hipStream_t s) {
  const uint64_t per = (bytes + workgroups - 1u) / workgroups;
  const uint64_t chunk = (per + 4095u) / 4096u * 4096u;
  if (chunk > 0x7FFFF000u) return hipErrorInvalidValue;
  const uint32_t magic = 0x9E3779B9u;
  switch (unroll) {
    case 1: hipLaunchKernelGGL(k_read_floor<1>, dim3(workgroups), dim3(256), 0, s, src, bytes, (uint32_t)chunk, sink, magic); break;
    case 2: hipLaunchKernelGGL(k_read_floor<2>, dim3(workgroups), dim3(256), 0, s, src, bytes, (uint32_t)chunk, sink, magic); break;
    case 4: hipLaunchKernelGGL(k_read_floor<4>, dim3(workgroups), dim3(256), 0, s, src, bytes, (uint32_t)chunk, sink, magic); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const WeightView &wv, uint32_t n_blocks, float *out, hipStream_t s) {
  switch (wv.type) {
    case Q8_0: return dequant_go<Q8_0>(wv, n_blocks, out, s);
    case Q8_0R: return dequant_go<Q8_0R>(wv, n_blocks, out, s);
    case Q4_K: return dequant_go<Q4_K>(wv, n_blocks, out, s);
    case Q6_K: return dequant_go<Q6_K>(wv, n_blocks, out, s);
    case Q2_K: return dequant_go<Q2_K>(wv, n_blocks, out, s);
    case IQ2_XXS: return dequant_go<IQ2_XXS>(wv, n_blocks, out, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE>
static hipError_t gather_go(const WeightView &wv, const uint32_t *ids, uint32_t tokens, float *out, hipStream_t s) {
  const uint64_t units = (uint64_t)tokens * wv.bpr * units_per_block<TYPE>();
  hipLaunchKernelGGL((k_gather<TYPE>), dim3((uint32_t)((units + 255) / 256)), dim3(256), 0, s, wv, ids, tokens, out);
  return hipGetLastError();
}

hipError_t launch_gather(const WeightView &wv, const uint32_t *ids, uint32_t tokens, float *out, hipStream_t s) {
  switch (wv.type) {
    case Q8_0: return gather_go<Q8_0>(wv, ids, tokens, out, s);
    case Q8_0R: return gather_go<Q8_0R>(wv, ids, tokens, out, s);
    case Q4_K: return gather_go<Q4_K>(wv, ids, tokens, out, s);
    case Q6_K: return gather_go<Q6_K>(wv, ids, tokens, out, s);
    case Q2_K: return gather_go<Q2_K>(wv, ids, tokens, out, s);
    case IQ2_XXS: return gather_go<IQ2_XXS>(wv, ids, tokens, out, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE>
static hipError_t gather_norm_go(const WeightView &wv, const uint32_t *ids, uint32_t tokens, const float *wn, float eps,
                                 float *x, float *nrm, hipStream_t s) {
  const size_t lds = (size_t)wv.k * 4u;
  static std::atomic<uint64_t> attr{0};
  const hipError_t e = lds_limit_once((const void *)k_gather_norm<TYPE>, (int)kGatherNormMaxDim * 4, attr);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gather_norm<TYPE>), dim3(tokens), dim3(256), lds, s, wv, ids, wn, eps, x, nrm);
  return hipGetLastError();
}

hipError_t launch_gather_norm(const WeightView &wv, const uint32_t *ids, uint32_t tokens, const float *wn, float eps,
                              float *x, float *nrm, hipStream_t s) {
  switch (wv.type) {
    case Q8_0: return gather_norm_go<Q8_0>(wv, ids, tokens, wn, eps, x, nrm, s);
    case Q8_0R: return gather_norm_go<Q8_0R>(wv, ids, tokens, wn, eps, x, nrm, s);
    case Q4_K: return gather_norm_go<Q4_K>(wv, ids, tokens, wn, eps, x, nrm, s);
    case Q6_K: return gather_norm_go<Q6_K>(wv, ids, tokens, wn, eps, x, nrm, s);
    case Q2_K: return gather_norm_go<Q2_K>(wv, ids, tokens, wn, eps, x, nrm, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace eff
