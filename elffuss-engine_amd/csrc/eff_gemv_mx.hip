// GEMV on the matrix cores: Y[t][row] = sum_k W[row][k] X[t][k] for 1..8
// tokens, with the weights kept as the signed 8-bit integers of their blocks
// and x split into three signed 8-bit digit planes.
//
// x digits. For each group of 32 consecutive x values of a token, with
// max|x| < 2^E, x is rounded to xi = round(x * 2^(21-E)) (|xi| <= 2^21) and
// written xi = d2*65536 + d1*256 + d0 with d0, d1 in [-128, 127] and
// |d2| <= 32: 22 significant bits relative to the group maximum. The group
// factor p = 2^(E-21) and the f32 sums of x over each 16 values stay beside
// the digits in LDS. A workgroup prepares the digits of the whole x once.
//
// Weights. Every type is read in tasks of 64 weights of one row, made of 4
// runs of 16 consecutive k; each run has its own scale (Q6_K, Q2_K) or two
// runs share one (Q8_0, Q4_K, IQ2_XXS). value = s * u - m with u a signed
// 8-bit integer taken from the block bytes:
//   Q8_0, Q8_0R  u = q                     s = d               m = 0
//   Q4_K         u = 4-bit q               s = d * sc          m = dmin * mn
//   Q6_K         u = ql | qh << 4 (0..63)  s = d * sc          m = 32 * d * sc
//   Q2_K         u = 2-bit q               s = d * (sc & 15)   m = dmin * (sc >> 4)
//   IQ2_XXS      u = +-grid byte           s = d*(0.5+ls)/4    m = 0
// (the block decoders of kernels.wgsl.js:154-396, in integer form).
//
// MFMA. v_mfma_i32_4x4x4_16b_i8 computes 16 independent 4x4x4 products. Lane
// l = 4b + c holds, for block b, row c of A (4 x values of digit plane c; row
// 3 is filler whose output is not used) and column c of B (4 weights of row c
// of W). Its D is then the three exact integer sums sum(u * d_i) over those
// 4 k for its own row. A wave covers 4 rows of W (c) x 16 tasks (b); the 16
// MFMAs of a task accumulate per scale group in D, and each group is folded
// into the lane's f32 sum:  acc += s * p * (D2*65536 + D1*256 + D0) - m * sum(x).
// The 16 task slots of a row are added with DPP at the end, and the k slices
// of a workgroup in a fixed order through LDS.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
#include "eff_formats.h"
#include "eff_kernels.h"
#include "eff_xdigits.h"

namespace eff {

static __constant__ uint64_t c_grid_mx[256] = {
#include "iq2xxs_grid.inc"
};

typedef int int4v __attribute__((ext_vector_type(4)));

namespace {

constexpr int kMxTables = 3072;  // IQ2_XXS grid (256 x 8 B) + sign masks (128 x 8 B), LDS bytes

__device__ __forceinline__ float ub(uint32_t w, int c) { return (float)((w >> (8 * c)) & 0xFFu); }

// ---------------------------------------------------------------------------
// Tasks: the bytes of 64 weights of one row, their int8 form (B[16], one
// dword per MFMA; MFMAs 4r..4r+3 are run r) and their scales.
//
// A wave stages, per pass, the bytes of its 4 rows that hold 16 consecutive
// tasks (RB bytes per row) into LDS with coalesced 16-byte loads, then every
// lane reads its task from there. `tbyte(ti)` is the offset of task ti's
// first byte in its row (ti a multiple of 4 starts a block), `ALIGN` the
// alignment that row and pass offsets always have, `read(p, b)` takes the
// LDS address of the pass region of the lane's row and the task slot b.
template <int TYPE> struct Task;

// LDS reads at 4-byte and at 2-byte aligned addresses.
__device__ __forceinline__ uint32_t lds32(const uint8_t *p) { return *(const uint32_t *)p; }
// (Alignment is taken off the pointer by pointer arithmetic, so that the
// compiler keeps the LDS address space and emits ds_read, not flat loads.)
__device__ __forceinline__ void lds16_a2(const uint8_t *p, uint32_t *out) {
  const uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
  const uint8_t *q = p - sh;
  uint32_t v[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) v[i] = lds32(q + 4 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sh);
}
__device__ __forceinline__ uint32_t lds16b_a2(const uint8_t *p) {
  const uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
  const uint32_t w = lds32(p - sh);
  return sh ? (w >> 16) : (w & 0xFFFFu);
}

template <> struct Task<Q8_0> {
  static constexpr int G = 2;  // scale groups (2 runs each)
  static constexpr uint32_t RUN = 16u;  // k distance between runs
  static constexpr uint32_t RB = 1088, ALIGN = 4;
  __device__ static uint32_t tbyte(uint32_t ti) { return 68u * ti; }
  uint32_t w[17];              // two blocks, 68 bytes from a 4-aligned offset
  __device__ void read(const uint8_t *p, uint32_t b) {
#pragma unroll
    for (int i = 0; i < 17; ++i) w[i] = lds32(p + 68u * b + 4u * i);
  }
  __device__ void decode(uint32_t *B, const uint32_t *) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) B[j] = __builtin_amdgcn_alignbyte(w[j + 1], w[j], 2);
#pragma unroll
    for (int j = 0; j < 8; ++j) B[8 + j] = w[9 + j];
  }
  __device__ void scales(uint32_t, float *sa, float *sb, float &fa, float &fb) const {
    sa[0] = h2f(w[0] & 0xFFFFu);
    sa[1] = h2f(w[8] >> 16);
    sb[0] = sb[1] = 0.f;
    fa = 1.f;
    fb = 0.f;
  }
  __device__ static uint32_t run_k(uint32_t ti, int r) { return 64u * ti + 16u * (uint32_t)r; }
};

// Quants and scales live in two regions; the scales (2 bytes per block) are
// staged as a second region of 64 bytes per row and pass.
template <> struct Task<Q8_0R> {
  static constexpr int G = 2;
  static constexpr uint32_t RUN = 16u;  // k distance between runs
  static constexpr uint32_t RB = 1024, ALIGN = 16, RB2 = 64, ALIGN2 = 4;
  __device__ static uint32_t tbyte(uint32_t ti) { return 64u * ti; }
  __device__ static uint32_t tbyte2(uint32_t ti) { return 4u * ti; }
  uint32_t q[16], s;
  __device__ void read(const uint8_t *p, uint32_t b) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = *(const u32x4 *)(p + 64u * b + 16u * i);
      q[4 * i] = v.x; q[4 * i + 1] = v.y; q[4 * i + 2] = v.z; q[4 * i + 3] = v.w;
    }
  }
  __device__ void read2(const uint8_t *p, uint32_t b) { s = lds32(p + 4u * b); }
  __device__ void decode(uint32_t *B, const uint32_t *) const {
#pragma unroll
    for (int j = 0; j < 16; ++j) B[j] = q[j];
  }
  __device__ void scales(uint32_t, float *sa, float *sb, float &fa, float &fb) const {
    sa[0] = h2f(s & 0xFFFFu);
    sa[1] = h2f(s >> 16);
    sb[0] = sb[1] = 0.f;
    fa = 1.f;
    fb = 0.f;
  }
  __device__ static uint32_t run_k(uint32_t ti, int r) { return 64u * ti + 16u * (uint32_t)r; }
};

// Task = sub-block pair p = ti % 4 of block ti / 4: qs bytes 32p..32p+31, low
// nibbles = sub-block 2p (runs 0, 1), high nibbles = 2p+1 (runs 2, 3).
template <> struct Task<Q4_K> {
  static constexpr int G = 2;
  static constexpr uint32_t RUN = 16u;  // k distance between runs
  static constexpr uint32_t RB = 576, ALIGN = 16;
  __device__ static uint32_t tbyte(uint32_t ti) { return 144u * (ti >> 2); }
  uint32_t h[4], qs[8];
  __device__ void read(const uint8_t *p, uint32_t b) {
    const uint8_t *blk = p + 144u * (b >> 2);
    const u32x4 a = *(const u32x4 *)blk;
    const u32x4 c = *(const u32x4 *)(blk + 16u + 32u * (b & 3u));
    const u32x4 d = *(const u32x4 *)(blk + 32u + 32u * (b & 3u));
    h[0] = a.x; h[1] = a.y; h[2] = a.z; h[3] = a.w;
    qs[0] = c.x; qs[1] = c.y; qs[2] = c.z; qs[3] = c.w; qs[4] = d.x; qs[5] = d.y; qs[6] = d.z; qs[7] = d.w;
  }
  __device__ void decode(uint32_t *B, const uint32_t *) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      B[j] = qs[j] & 0x0F0F0F0Fu;
      B[8 + j] = (qs[j] >> 4) & 0x0F0F0F0Fu;
    }
  }
  // 6-bit (scale, min) pairs 2p and 2p+1 (SCALE_MIN_K4, kernels.wgsl.js:94-104),
  // extracted for 4 pairs at a time as packed bytes.
  __device__ void scales(uint32_t ti, float *sa, float *sb, float &fa, float &fb) const {
    const uint32_t p = ti & 3u;
    const uint32_t sc_lo = h[1] & 0x3F3F3F3Fu, mn_lo = h[2] & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (h[3] & 0x0F0F0F0Fu) | ((h[1] >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((h[3] >> 4) & 0x0F0F0F0Fu) | ((h[2] >> 2) & 0x30303030u);
    uint32_t sc = p < 2u ? sc_lo : sc_hi, mn = p < 2u ? mn_lo : mn_hi;
    const uint32_t sh = 16u * (p & 1u);
    sc >>= sh;
    mn >>= sh;
    sa[0] = ub(sc, 0); sa[1] = ub(sc, 1);
    sb[0] = ub(mn, 0); sb[1] = ub(mn, 1);
    fa = h2f(h[0] & 0xFFFFu);
    fb = h2f(h[0] >> 16);
  }
  __device__ static uint32_t run_k(uint32_t ti, int r) { return 64u * ti + 16u * (uint32_t)r; }
};

// Task = (block ti/4, half n = (ti>>1)&1, l-range h = ti&1): weights
// 128n + 32g + 16h + i, g = 0..3 (run g), from ql bytes 64n + 32(g&1) + 16h + i
// (nibble g>>1), qh bytes 32n + 16h + i (bits 2g), scale 8n + 2g + h.
template <> struct Task<Q6_K> {
  static constexpr int G = 4;
  static constexpr uint32_t RUN = 32u;  // k distance between runs
  static constexpr uint32_t RB = 840, ALIGN = 2;
  __device__ static uint32_t tbyte(uint32_t ti) { return 210u * (ti >> 2); }
  uint32_t p0[4], p1[4], qh[4], sc0, sc1, d;
  __device__ void read(const uint8_t *p, uint32_t b) {
    const uint8_t *blk = p + 210u * (b >> 2);
    const uint32_t n = (b >> 1) & 1u, h = b & 1u;
    lds16_a2(blk + 64u * n + 16u * h, p0);
    lds16_a2(blk + 64u * n + 32u + 16u * h, p1);
    lds16_a2(blk + 128u + 32u * n + 16u * h, qh);
    const uint8_t *so = blk + 192u + 8u * n;
    const uint32_t sh = (uint32_t)((uintptr_t)so & 3u);
    const uint8_t *sq = so - sh;
    const uint32_t a = lds32(sq), bb = lds32(sq + 4), c = lds32(sq + 8);
    sc0 = __builtin_amdgcn_alignbyte(bb, a, sh);
    sc1 = __builtin_amdgcn_alignbyte(c, bb, sh);
    d = lds16b_a2(blk + 208u);
  }
  __device__ void decode(uint32_t *B, const uint32_t *) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      B[i] = (p0[i] & 0x0F0F0F0Fu) | ((qh[i] << 4) & 0x30303030u);
      B[4 + i] = (p1[i] & 0x0F0F0F0Fu) | ((qh[i] << 2) & 0x30303030u);
      B[8 + i] = ((p0[i] >> 4) & 0x0F0F0F0Fu) | (qh[i] & 0x30303030u);
      B[12 + i] = ((p1[i] >> 4) & 0x0F0F0F0Fu) | ((qh[i] >> 2) & 0x30303030u);
    }
  }
  __device__ void scales(uint32_t ti, float *sa, float *sb, float &fa, float &fb) const {
    const uint32_t h8 = 8u * (ti & 1u);
    sa[0] = (float)(int)__builtin_amdgcn_sbfe((int)sc0, h8, 8);
    sa[1] = (float)(int)__builtin_amdgcn_sbfe((int)sc0, h8 + 16u, 8);
    sa[2] = (float)(int)__builtin_amdgcn_sbfe((int)sc1, h8, 8);
    sa[3] = (float)(int)__builtin_amdgcn_sbfe((int)sc1, h8 + 16u, 8);
#pragma unroll
    for (int g = 0; g < 4; ++g) sb[g] = sa[g];
    fa = h2f(d);
    fb = 32.f * fa;
  }
  __device__ static uint32_t run_k(uint32_t ti, int r) {
    return 256u * (ti >> 2) + 128u * ((ti >> 1) & 1u) + 32u * (uint32_t)r + 16u * (ti & 1u);
  }
};

// Task = (block ti/4, n, h) as Q6_K: qs bytes 32n + 16h + i at bit shift 2g,
// scale byte 8n + 2g + h.
template <> struct Task<Q2_K> {
  static constexpr int G = 4;
  static constexpr uint32_t RUN = 32u;  // k distance between runs
  static constexpr uint32_t RB = 336, ALIGN = 4;
  __device__ static uint32_t tbyte(uint32_t ti) { return 84u * (ti >> 2); }
  uint32_t qs[4], sc0, sc1, dd;
  __device__ void read(const uint8_t *p, uint32_t b) {
    const uint8_t *blk = p + 84u * (b >> 2);
    const uint32_t n = (b >> 1) & 1u, h = b & 1u;
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[i] = lds32(blk + 16u + 32u * n + 16u * h + 4u * i);
    sc0 = lds32(blk + 8u * n);
    sc1 = lds32(blk + 8u * n + 4u);
    dd = lds32(blk + 80u);
  }
  __device__ void decode(uint32_t *B, const uint32_t *) const {
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) B[4 * g + i] = (qs[i] >> (2 * g)) & 0x03030303u;
  }
  __device__ void scales(uint32_t ti, float *sa, float *sb, float &fa, float &fb) const {
    const uint32_t h8 = 8u * (ti & 1u);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t v = ((g < 2 ? sc0 : sc1) >> (h8 + 16u * (g & 1))) & 0xFFu;
      sa[g] = (float)(v & 15u);
      sb[g] = (float)(v >> 4);
    }
    fa = h2f(dd & 0xFFFFu);
    fb = h2f(dd >> 16);
  }
  __device__ static uint32_t run_k(uint32_t ti, int r) {
    return 256u * (ti >> 2) + 128u * ((ti >> 1) & 1u) + 32u * (uint32_t)r + 16u * (ti & 1u);
  }
};

// Task = 32-weight groups 2(ti%4) and 2(ti%4)+1 of block ti/4: per group a
// word of 4 grid indices (8 weights each) and a word of 4 x 7 sign bits and
// the 4-bit scale (kernels.wgsl.js:374-395). The grid entries and the sign
// masks (parity bit added) come from LDS tables.
template <> struct Task<IQ2_XXS> {
  static constexpr int G = 2;
  static constexpr uint32_t RUN = 16u;  // k distance between runs
  static constexpr uint32_t RB = 264, ALIGN = 2;
  __device__ static uint32_t tbyte(uint32_t ti) { return 66u * (ti >> 2); }
  uint32_t q[4], d;
  __device__ void read(const uint8_t *p, uint32_t b) {
    const uint8_t *blk = p + 66u * (b >> 2);
    lds16_a2(blk + 2u + 16u * (b & 3u), q);
    d = lds16b_a2(blk);
  }
  __device__ void decode(uint32_t *B, const uint32_t *tab) const {
#pragma unroll
    for (int gg = 0; gg < 2; ++gg)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t gi = (q[2 * gg] >> (8 * e)) & 0xFFu, sg = (q[2 * gg + 1] >> (7 * e)) & 127u;
        const uint2 g = *(const uint2 *)(tab + 2u * gi);
        const uint2 m = *(const uint2 *)(tab + 512u + 2u * sg);
        // bytes with a set mask are negated: ~g + 1 (grid bytes are never 0)
        B[8 * gg + 2 * e] = (g.x ^ m.x) + (m.x & 0x01010101u);
        B[8 * gg + 2 * e + 1] = (g.y ^ m.y) + (m.y & 0x01010101u);
      }
  }
  __device__ void scales(uint32_t, float *sa, float *sb, float &fa, float &fb) const {
    sa[0] = 0.5f + (float)(q[1] >> 28);
    sa[1] = 0.5f + (float)(q[3] >> 28);
    sb[0] = sb[1] = 0.f;
    fa = 0.25f * h2f(d);
    fb = 0.f;
  }
  __device__ static uint32_t run_k(uint32_t ti, int r) { return 64u * ti + 16u * (uint32_t)r; }
};

// Staging geometry: chunks of 16 bytes per row and pass (covering the region
// from its 4-byte aligned start), 16-byte loads per lane and stage, and the
// stage size in LDS.
template <uint32_t RB, uint32_t ALIGN> struct Stage {
  // regions start at 4-byte aligned offsets (floored by 2 bytes for ALIGN 2)
  static constexpr uint32_t CPR = (RB + (ALIGN < 4u ? 2u : 0u) + 15u) / 16u;
  static constexpr uint32_t LOADS = (4u * CPR + 63u) / 64u;
  static constexpr uint32_t BYTES = LOADS * 1024u;
};

template <int TYPE> struct Stage2 {
  static constexpr uint32_t LOADS = 0, BYTES = 0, CPR = 1;
};
template <> struct Stage2<Q8_0R> : Stage<Task<Q8_0R>::RB2, Task<Q8_0R>::ALIGN2> {};

// IQ2_XXS tables in LDS: the grid (256 x 8 bytes) and, for each 7-bit sign
// field, the byte masks of its 8 signs (parity bit added, kernels.wgsl.js:381-384).
__device__ __forceinline__ void mx_tables(uint32_t *tab, uint64_t g, uint32_t tid) {
  tab[2 * tid] = (uint32_t)g;
  tab[2 * tid + 1] = (uint32_t)(g >> 32);
  if (tid < 128u) {
    const uint32_t s8 = tid | ((uint32_t)(__builtin_popcount(tid) & 1) << 7);
    uint32_t m0 = 0, m1 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m0 |= ((s8 >> j) & 1u) ? (0xFFu << (8 * j)) : 0u;
      m1 |= ((s8 >> (4 + j)) & 1u) ? (0xFFu << (8 * j)) : 0u;
    }
    tab[512 + 2 * tid] = m0;
    tab[512 + 2 * tid + 1] = m1;
  }
}

// Sum over the 16 lanes 4b + c of one c (DPP row rotations, then across the
// 4 rows of 16 lanes); every lane gets the total of its c.
__device__ __forceinline__ float slot_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

}  // namespace

// ---------------------------------------------------------------------------
// A workgroup is NW waves = (NW/S) row quads x S slices of k; a tile is its
// 4*NW/S rows. With S = 1 the workgroups are persistent: workgroup i takes
// tiles i, i + grid, ... and each wave streams through the passes of its row
// quad in every tile. With S > 1 there is one tile per workgroup and the
// slices are added in a fixed order through LDS.
//
// A pass is 16 tasks of the wave's 4 rows. Its bytes (4 rows x RB) are
// fetched with coalesced 16-byte loads (lane i takes chunks i, i+64, ...) two
// passes ahead into registers, and written to the wave's LDS stage just before
// the pass is computed; each lane then reads its own task from the stage.
// Launch geometry, computed on the host so that the kernel's prologue (which
// every workgroup runs before its first load) has no integer divisions.
struct MxGeo {
  uint32_t s_log2;  // S = 2^s_log2 k slices per row quad
  uint32_t ntask;   // 64-weight tasks per slice (k / 64 / S)
  uint32_t passes;  // passes of 16 tasks per slice
  uint32_t tq, tr;  // row tiles = tq * grid + tr
};

// Fused launches over up to 4 matrices of one type and k sharing x
// (ops.gemv.js:166-215). F = 1, sections: the row tiles of matrix q are the
// launch's tiles [tend[q-1], tend[q]), and each matrix writes its own y.
// F = 2, gate + up: the S slices of a row quad are doubled, the waves of the
// upper half reading matrix 1, and y[0] = silu(gate) * up
// (kernels.gemv.wgsl.js:436, 517-518). A row's sums are formed exactly as in a
// one-matrix launch with the same slices, so the outputs are the same bits.
struct MxSec {
  uint32_t n;        // matrices
  uint32_t tend[4];  // sections: end tile of each matrix
  uint32_t rows[4];
  const uint8_t *w[4];
  uint64_t w_bytes[4], scales_off[4];
  float *y[4];
};

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

template <int TYPE, int T, int NW, int F>
__global__ __launch_bounds__(NW * 64) void k_gemv_mx(WeightView wv, const float *__restrict__ x,
                                                     float *__restrict__ y, MxGeo geo, MxSec sec) {
  using TK = Task<TYPE>;
  using ST = Stage<TK::RB, TK::ALIGN>;
  using ST2 = Stage2<TYPE>;
  constexpr bool kTab = TYPE == IQ2_XXS;
  constexpr uint32_t NT = NW * 64u, SBT = ST::BYTES + ST2::BYTES;
  constexpr uint32_t L2N = ST2::LOADS > 0 ? ST2::LOADS : 1u;
  extern __shared__ __align__(16) uint8_t lds[];
  uint32_t *tab = (uint32_t *)lds;
  uint8_t *xl = lds + (kTab ? kMxTables : 0);

  // all kernel arguments in scalar registers at once: one round trip to the
  // argument buffer instead of one per use
  __asm__ volatile("" ::"s"(wv.w), "s"(wv.rows), "s"(wv.k), "s"(wv.bpr), "s"(wv.row_bytes), "s"(wv.w_bytes),
                   "s"(wv.scales_off), "s"(x), "s"(y), "s"(geo.s_log2), "s"(geo.ntask), "s"(geo.passes), "s"(geo.tq),
                   "s"(geo.tr));
  const uint32_t tid = threadIdx.x, lane = tid & 63u, b = lane >> 2, c = lane & 3u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar registers)
  const uint32_t rows = wv.rows, k = wv.k;
  const uint32_t S = 1u << geo.s_log2, G4 = (uint32_t)NW >> geo.s_log2;
  const uint32_t gq = wave >> geo.s_log2, sl = wave & (S - 1u), RPT = 4u * G4;
  // gate + up: SR slices per matrix, this wave's k slice and matrix
  const uint32_t SR = F == 2 ? S >> 1 : S, ksl = sl & (SR - 1u), wmat = F == 2 ? sl / SR : 0u;
  // the section of a tile (F = 1) and its first tile
  auto sec_of = [&](uint32_t tile, uint32_t &first) {
    uint32_t q = 0;
    first = 0;
#pragma unroll
    for (uint32_t i = 0; i < 3u; ++i)
      if (i + 1u < sec.n && tile >= sec.tend[i]) {
        q = i + 1u;
        first = sec.tend[i];
      }
    return q;
  };
  auto src_of = [&](uint32_t q) {
    WeightView m = wv;
    m.w = sec.w[q];
    m.w_bytes = sec.w_bytes[q];
    m.scales_off = sec.scales_off[q];
    return make_src(m, 0);
  };
  BufSrc src = F == 2 ? src_of(wmat) : make_src(wv, 0);
  const uint32_t xbytes = (uint32_t)T * k * 3u + (uint32_t)T * (k / 8u) * 4u;
  uint8_t *const stg = xl + xbytes + wave * SBT;
  float *red = (float *)(xl + xbytes + (uint32_t)NW * SBT);

  const uint32_t ntask = geo.ntask, t0 = ksl * ntask, passes = geo.passes;
  const uint32_t my_tiles = geo.tq + (blockIdx.x < geo.tr ? 1u : 0u), nitems = my_tiles * passes;
  // bytes of a row: GGUF blocks, or the quants of Q8_0R (its scales: 2 per block)
  const uint32_t rbytes = TYPE == Q8_0R ? 32u * wv.bpr : (uint32_t)wv.row_bytes, sbytes = 2u * wv.bpr;
  auto row_of = [&](uint32_t tile, uint32_t r) {
    if constexpr (F == 1) {
      uint32_t first;
      const uint32_t q = sec_of(tile, first);
      return min((tile - first) * RPT + 4u * gq + r, sec.rows[q] - 1u);
    }
    return min(tile * RPT + 4u * gq + r, rows - 1u);
  };

  // This lane's chunks: chunk q = lane + 64j is chunk q % CPR of row q / CPR,
  // stored at byte 16q of the stage.
  uint32_t s_r[ST::LOADS], s_ch[ST::LOADS];
#pragma unroll
  for (uint32_t j = 0; j < ST::LOADS; ++j) {
    const uint32_t q = lane + 64u * j, r = q / ST::CPR;
    s_r[j] = min(r, 3u);
    s_ch[j] = 16u * (r > 3u ? 0u : q - r * ST::CPR);
  }
  uint32_t s2_r = 0, s2_ch = 0;
  if constexpr (ST2::LOADS > 0) {
    const uint32_t r = lane / ST2::CPR;
    s2_r = min(r, 3u);
    s2_ch = 16u * (r > 3u ? 0u : lane - r * ST2::CPR);
  }
  // Per-lane load offsets of the fetch tile (the pass offset comes on top, in
  // the scalar offset of the load when the region start is 4-byte aligned).
  uint32_t vo[ST::LOADS], vo2 = 0;
  auto set_tile = [&](uint32_t tile) {
    if constexpr (F == 1) {
      uint32_t first;
      src = src_of(sec_of(tile, first));
    }
#pragma unroll
    for (uint32_t j = 0; j < ST::LOADS; ++j) vo[j] = row_of(tile, s_r[j]) * rbytes + (TK::ALIGN >= 4u ? s_ch[j] : 0u);
    if constexpr (ST2::LOADS > 0) vo2 = row_of(tile, s2_r) * sbytes + s2_ch;
  };
  struct Regs {
    u32x4 q[ST::LOADS], s[L2N];
  };
  // Cache policy of the weight stream: non-temporal (nt) for the types where it
  // measured faster (Q4_K 2048x8192: 4.66 -> 4.55 us; Q2_K, IQ2_XXS 8192x2048:
  // -6%), the default where it measured slower (Q8_0 +6%, Q8_0R +2%, Q6_K +1%,
  // and the sections mode F = 1, q+k+v Q4_K: 5.14 -> 5.81 us per launch).
  constexpr int kWeightAux = (F != 1 && (TYPE == Q4_K || TYPE == Q2_K || TYPE == IQ2_XXS)) ? 2 : 0;
  auto fetch = [&](uint32_t ps, Regs &R) {
    const uint32_t roff = TK::tbyte(t0 + 16u * ps);
#pragma unroll
    for (uint32_t j = 0; j < ST::LOADS; ++j) {
      if constexpr (TK::ALIGN >= 4u)
        R.q[j] = __builtin_amdgcn_raw_buffer_load_b128(src.q, (int)vo[j], (int)roff, kWeightAux);
      else
        R.q[j] = __builtin_amdgcn_raw_buffer_load_b128(src.q, (int)(((vo[j] + roff) & ~3u) + s_ch[j]), 0, kWeightAux);
    }
    if constexpr (ST2::LOADS > 0)
      R.s[0] = __builtin_amdgcn_raw_buffer_load_b128(src.s, (int)vo2, (int)Task<Q8_0R>::tbyte2(t0 + 16u * ps), 0);
  };
  auto put = [&](const Regs &R) {
#pragma unroll
    for (uint32_t j = 0; j < ST::LOADS; ++j) *(u32x4 *)(stg + 1024u * j + 16u * lane) = R.q[j];
    if constexpr (ST2::LOADS > 0) *(u32x4 *)(stg + ST::BYTES + 16u * lane) = R.s[0];
  };
  // Fetch cursor, two items ahead of the compute cursor; it stops on the last
  // item (fetched again), so the number of loads in flight never changes.
  uint32_t f_tile = blockIdx.x, f_ps = 0, f_n = 0;
  set_tile(f_tile);
  auto fetch_next = [&](Regs &R) {
    fetch(f_ps, R);
    if (f_n + 1u < nitems) {
      ++f_n;
      if (++f_ps == passes) {
        f_ps = 0;
        f_tile += gridDim.x;
        set_tile(f_tile);
      }
    }
  };

  // x (and the IQ2_XXS grid) first, then the weights of the first two items
  const uint32_t noct = (uint32_t)T * (k / 8u);
  XOct xo[kXr];
#pragma unroll
  for (uint32_t i = 0; i < kXr; ++i)
    if (tid + NT * i < noct) x_load<(uint32_t)T>(x, k, tid + NT * i, xo[i]);
  uint64_t gent = 0;
  if constexpr (kTab) gent = c_grid_mx[tid & 255u];
  __asm__ volatile("" ::: "memory");  // keep these loads ahead of the weights

  Regs RA, RB;
  fetch_next(RA);
  fetch_next(RB);

  if constexpr (kTab) {
    if (tid < 256u) mx_tables(tab, gent, tid);
  }
#pragma unroll
  for (uint32_t i = 0; i < kXr; ++i)
    if (tid + NT * i < noct) x_store<(uint32_t)T>(xo[i], k, tid + NT * i, xl, k * 3u, (float *)(xl + (uint64_t)T * k * 3u), k / 8u);
  for (uint32_t o = tid + NT * kXr; o < noct; o += NT) {
    XOct v;
    x_load<(uint32_t)T>(x, k, o, v);
    x_store<(uint32_t)T>(v, k, o, xl, k * 3u, (float *)(xl + (uint64_t)T * k * 3u), k / 8u);
  }
  __syncthreads();

  const uint8_t *dig = xl;
  const float *meta = (const float *)(xl + (uint64_t)T * k * 3u);
  const uint32_t cd = c < 3u ? c : 0u;

  float acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = 0.f;

  constexpr int G = TK::G, RPG = 4 / G;  // runs per scale group
  auto compute = [&](uint32_t tile, uint32_t ps) {
    const uint32_t slot = 16u * ps + b;
    const bool active = slot < ntask;
    const uint32_t ti = t0 + 16u * ps + b;
    const uint32_t roff = TK::tbyte(t0 + 16u * ps);
    TK w;
    if constexpr (TK::ALIGN >= 4u) {
      w.read(stg + c * (ST::CPR * 16u), b);
    } else {
      w.read(stg + c * (ST::CPR * 16u) + ((row_of(tile, c) * rbytes + roff) & 3u), b);
    }
    if constexpr (ST2::LOADS > 0) w.read2(stg + ST::BYTES + c * (ST2::CPR * 16u), b);
    uint32_t B[16];
    w.decode(B, tab);
    float sa[G], sb[G], fa, fb;
    w.scales(ti, sa, sb, fa, fb);
    // x digits and group data of the task's first run; the other runs sit at
    // fixed distances (RUN apart in k)
    const uint32_t kb = active ? TK::run_k(ti, 0) : 0u;
    const bool xh = ((kb / 16u) & 1u) != 0u;  // runs of 16-weight groups: which half of the 32-group
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint8_t *dA = dig + (uint64_t)t * k * 3u + (kb / 16u) * 48u + 16u * cd;
      const float *mA = meta + (uint64_t)t * (k / 8u) + 4u * (kb / 32u);
      float av = 0.f, bv = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        int4v D = {0, 0, 0, 0};
        const float4 M = *(const float4 *)(mA + 4u * ((uint32_t)(g * RPG) * TK::RUN / 32u));
        const float pg = M.x;
        const float xg = RPG == 2 ? M.y + M.z : (xh ? M.z : M.y);
#pragma unroll
        for (int rr = 0; rr < RPG; ++rr) {
          const int r = g * RPG + rr;
          const u32x4 A = *(const u32x4 *)(dA + ((uint32_t)r * TK::RUN / 16u) * 48u);
          D = __builtin_amdgcn_mfma_i32_4x4x4i8((int)A.x, (int)B[4 * r], D, 0, 0, 0);
          D = __builtin_amdgcn_mfma_i32_4x4x4i8((int)A.y, (int)B[4 * r + 1], D, 0, 0, 0);
          D = __builtin_amdgcn_mfma_i32_4x4x4i8((int)A.z, (int)B[4 * r + 2], D, 0, 0, 0);
          D = __builtin_amdgcn_mfma_i32_4x4x4i8((int)A.w, (int)B[4 * r + 3], D, 0, 0, 0);
        }
        const float f = __builtin_fmaf((float)(D.z * 256 + D.y), 256.f, (float)D.x);
        av = __builtin_fmaf(sa[g], pg * f, av);
        bv = __builtin_fmaf(sb[g], xg, bv);
      }
      const float v = __builtin_fmaf(fa, av, -fb * bv);
      acc[t] += active ? v : 0.f;
    }
  };
  // End of a tile: the 16 task slots of each row are added; S = 1 writes y,
  // S > 1 (one tile per workgroup) adds the slices through LDS.
  auto finish = [&](uint32_t tile) {
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = slot_sum(acc[t]);
    // the tile's output: its matrix's y and rows, and the tile within the matrix
    float *yo = y;
    uint32_t ro = rows, lt = tile;
    if constexpr (F == 1) {
      uint32_t first;
      const uint32_t q = sec_of(tile, first);
      yo = sec.y[q];
      ro = sec.rows[q];
      lt = tile - first;
    }
    if (S == 1) {
      const uint32_t r = lt * RPT + 4u * gq + c;
      if (b == 0u && r < ro) {
#pragma unroll
        for (int t = 0; t < T; ++t) yo[(uint64_t)t * ro + r] = acc[t];
      }
    } else {
      if (b == 0u) {
#pragma unroll
        for (int t = 0; t < T; ++t) red[(wave * 4u + c) * (uint32_t)T + t] = acc[t];
      }
      __syncthreads();
      if (tid < RPT * (uint32_t)T) {
        const uint32_t rq = tid / (4u * (uint32_t)T), rc = (tid / (uint32_t)T) % 4u, t = tid % (uint32_t)T;
        auto at = [&](uint32_t q) { return red[((rq * (uint32_t)S + q) * 4u + rc) * (uint32_t)T + t]; };
        float v;
        if constexpr (F == 2) {
          // gate and up, each summed as a one-matrix launch of SR slices sums it
          float g = 0.f, u = 0.f;
          if (SR == 1u) {
            g = at(0);
            u = at(1);
          } else {
            for (uint32_t q = 0; q < SR; ++q) g += at(q);
            for (uint32_t q = 0; q < SR; ++q) u += at(SR + q);
          }
          v = silu(g) * u;
        } else {
          v = 0.f;
          for (uint32_t q = 0; q < (uint32_t)S; ++q) v += at(q);
        }
        const uint32_t r = lt * RPT + 4u * rq + rc;
        if (r < ro) yo[(uint64_t)t * ro + r] = v;
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;
  };
  uint32_t c_tile = blockIdx.x, c_ps = 0;
  // the registers of a pass are free once written to the stage: the fetch two
  // items ahead goes out before the pass is computed
  auto step = [&](Regs &R, bool run) {
    put(R);
    fetch_next(R);
    if (run) {
      compute(c_tile, c_ps);
      if (++c_ps == passes) {
        finish(c_tile);
        c_ps = 0;
        c_tile += gridDim.x;
      }
    }
  };

  // (the second fetch of an iteration is issued even without a second item,
  // so the loads in flight are the same on every path)
  for (uint32_t n = 0; n < nitems; n += 2u) {
    step(RA, true);
    step(RB, n + 1u < nitems);
  }
}

// ---------------------------------------------------------------------------
// Multi-token GEMV: 4 to 16 tokens per launch on v_mfma_i32_16x16x32_i8.
//
// One MFMA multiplies 16 rows of W (B: 32 k x 16 rows of int8 weights u) by
// 4 tokens x 4 digit planes of x (A: 16 x 32 k, row 4 t + plane; plane 3 is
// zero): lane l supplies B row l % 16 at k 8 (l / 16) .. + 7 and A row l % 16
// at the same k, and receives D for token l / 16 of the group, planes 0..3,
// row l % 16. The weights of a 32-k group are decoded once for all tokens,
// and each lane folds D into its (token, row) sum as the 4-row kernel does:
//   acc += s * p * ((D2 * 256 + D1) * 256 + D0) - m * sum(x).
// Types whose scales cover 16 weights (Q2_K, Q6_K) take two MFMAs per group,
// each with the other half's weights zeroed.
//
// A wave owns 16 rows and a slice of k; a workgroup is NW waves = (NW / S)
// row tiles x S slices, the slices added in a fixed order through LDS. k is
// walked in passes of 256: the 16 rows' bytes of a pass are fetched with
// coalesced 16-byte loads two passes ahead, written to the wave's LDS stage,
// and each lane reads its 8 weights of every group from there.
template <int TYPE> struct MtW;

template <int TYPE> constexpr uint32_t mt_block_elems() { return TYPE == Q8_0 ? 32u : 256u; }
template <int TYPE> constexpr uint32_t mt_block_bytes() {
  return TYPE == Q8_0 ? 34u : TYPE == Q4_K ? 144u : TYPE == Q6_K ? 210u : TYPE == Q2_K ? 84u : 66u;
}

// 6-bit (scale, min) pair j of a Q4_K block from its scale words (bytes 4-7,
// 8-11, 12-15 of the block), as SCALE_MIN_K4 (kernels.wgsl.js:94-104)
__device__ __forceinline__ void mt_q4k_sm(uint32_t s1, uint32_t s2, uint32_t s3, uint32_t j, uint32_t &sc,
                                          uint32_t &mn) {
  const uint32_t sh = 8u * (j & 3u);
  if (j < 4u) {
    sc = (s1 >> sh) & 63u;
    mn = (s2 >> sh) & 63u;
  } else {
    const uint32_t a = (s3 >> sh) & 0xFFu, b = (s1 >> sh) & 0xFFu, c = (s2 >> sh) & 0xFFu;
    sc = (a & 0xFu) | ((b >> 6) << 4);
    mn = (a >> 4) | ((c >> 6) << 4);
  }
}

// 8 bytes at a 2-byte aligned LDS address
__device__ __forceinline__ uint2 lds8_a2(const uint8_t *p) {
  const uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
  const uint8_t *q = p - sh;
  const uint32_t v0 = lds32(q), v1 = lds32(q + 4), v2 = lds32(q + 8);
  return make_uint2(__builtin_amdgcn_alignbyte(v1, v0, sh), __builtin_amdgcn_alignbyte(v2, v1, sh));
}
__device__ __forceinline__ float lds_h2f(const uint8_t *p) {
  const uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
  const uint32_t w = lds32(p - sh);
  return h2f(sh ? (w >> 16) : (w & 0xFFFFu));
}

// Per type: pass bytes per row (RB, 256 k), alignment of the pass start
// (ALIGN), scale groups per 32 k (SUB), and the decode of group g of a pass:
// the lane's 8 weights (kq = k / 8 inside the group) and the scales s, m of
// each 16- or 32-weight part, value = s u - m.
template <> struct MtW<Q8_0> {
  static constexpr uint32_t RB = 272, ALIGN = 4, SUB = 1;
  __device__ static void dec(const uint8_t *r, uint32_t g, uint32_t kq, const uint32_t *, uint2 &u, float *s,
                             float *m) {
    u = lds8_a2(r + 34u * g + 2u + 8u * kq);
    s[0] = lds_h2f(r + 34u * g);
    m[0] = 0.f;
  }
};
template <> struct MtW<Q4_K> {
  static constexpr uint32_t RB = 144, ALIGN = 16, SUB = 1;
  __device__ static void dec(const uint8_t *r, uint32_t g, uint32_t kq, const uint32_t *, uint2 &u, float *s,
                             float *m) {
    const uint2 w = *(const uint2 *)(r + 16u + 32u * (g >> 1) + 8u * kq);
    const uint32_t sh = 4u * (g & 1u);
    u = make_uint2((w.x >> sh) & 0x0F0F0F0Fu, (w.y >> sh) & 0x0F0F0F0Fu);
    const uint4 hd = *(const uint4 *)r;
    uint32_t sc, mn;
    mt_q4k_sm(hd.y, hd.z, hd.w, g, sc, mn);
    s[0] = h2f(hd.x & 0xFFFFu) * (float)sc;
    m[0] = h2f(hd.x >> 16) * (float)mn;
  }
};
template <> struct MtW<Q6_K> {
  static constexpr uint32_t RB = 210, ALIGN = 2, SUB = 2;
  __device__ static void dec(const uint8_t *r, uint32_t g, uint32_t kq, const uint32_t *, uint2 &u, float *s,
                             float *m) {
    // weight 32 g + l: ql byte 64 n + 32 (g & 1) + l (nibble (g & 3) >> 1),
    // qh byte 32 n + l (bits 2 (g & 3)), n = g >> 2; u = q in 0..63, m = 32 s
    const uint32_t n = g >> 2, gg = g & 3u;
    const uint2 ql = lds8_a2(r + 64u * n + 32u * (g & 1u) + 8u * kq);
    const uint2 qh = lds8_a2(r + 128u + 32u * n + 8u * kq);
    const uint32_t ls = 4u * (gg >> 1), hs = 2u * gg;
    u.x = ((ql.x >> ls) & 0x0F0F0F0Fu) | (((qh.x >> hs) & 0x03030303u) << 4);
    u.y = ((ql.y >> ls) & 0x0F0F0F0Fu) | (((qh.y >> hs) & 0x03030303u) << 4);
    const float d = lds_h2f(r + 208u);
    const uint8_t *sc = r + 192u + 2u * g;  // int8 scales of weights 32 g .. + 15, + 16 .. + 31
    const uint32_t sh = (uint32_t)((uintptr_t)sc & 3u);
    const uint32_t sw = lds32(sc - sh) >> (8u * sh);
    s[0] = d * (float)(int8_t)(sw & 0xFFu);
    s[1] = d * (float)(int8_t)((sw >> 8) & 0xFFu);
    m[0] = 32.f * s[0];
    m[1] = 32.f * s[1];
  }
};
template <> struct MtW<Q2_K> {
  // The 4-bit scale of each 16 is folded into the weights (u sc <= 45 fits a
  // signed byte): one MFMA per group, s = d, and the mins of both halves.
  static constexpr uint32_t RB = 84, ALIGN = 4, SUB = 1;
  __device__ static void dec(const uint8_t *r, uint32_t g, uint32_t kq, const uint32_t *, uint2 &u, float *s,
                             float *m) {
    // weight 32 g + l: qs byte 32 (g >> 2) + l, bits 2 (g & 3); scale byte 2 g (+1)
    const uint2 w = *(const uint2 *)(r + 16u + 32u * (g >> 2) + 8u * kq);
    const uint32_t sh = 2u * (g & 3u);
    const uint32_t dd = lds32(r + 80u);
    const uint32_t sc = lds32(r + 4u * (g >> 1)) >> (16u * (g & 1u));
    const uint32_t mine = kq < 2u ? (sc & 0xFu) : ((sc >> 8) & 0xFu);
    const uint32_t a = (w.x >> sh) & 0x03030303u, b = (w.y >> sh) & 0x03030303u;
    // u * sc per byte from the two bits of u (no carries: each product < 64)
    u.x = (a & 0x01010101u) * mine + ((a >> 1) & 0x01010101u) * (2u * mine);
    u.y = (b & 0x01010101u) * mine + ((b >> 1) & 0x01010101u) * (2u * mine);
    const float dmin = h2f(dd >> 16);
    s[0] = h2f(dd & 0xFFFFu);
    m[0] = dmin * (float)((sc >> 4) & 0xFu);
    m[1] = dmin * (float)((sc >> 12) & 0xFu);
  }
};
template <> struct MtW<IQ2_XXS> {
  static constexpr uint32_t RB = 66, ALIGN = 2, SUB = 1;
  __device__ static void dec(const uint8_t *r, uint32_t g, uint32_t kq, const uint32_t *tab, uint2 &u, float *s,
                             float *m) {
    // group g: grid indices (a0) and 4 x 7 sign bits + 4-bit scale (a1) at 2 + 8 g
    const uint2 a = lds8_a2(r + 2u + 8u * g);
    const uint32_t gi = (a.x >> (8u * kq)) & 0xFFu, sg = (a.y >> (7u * kq)) & 127u;
    const uint32_t g0 = tab[2u * gi], g1 = tab[2u * gi + 1u];
    const uint32_t m0 = tab[512u + 2u * sg], m1 = tab[512u + 2u * sg + 1u];
    // +g or -g per byte (two's complement, no carries between bytes)
    u.x = (g0 ^ m0) + (m0 & 0x01010101u);
    u.y = (g1 ^ m1) + (m1 & 0x01010101u);
    s[0] = lds_h2f(r) * (0.5f + (float)(a.y >> 28)) * 0.25f;
    m[0] = 0.f;
  }
};

template <int TYPE> struct MtStage {
  using W = MtW<TYPE>;
  // a pass region of a row, staged from its 4-byte aligned start (+2 bytes
  // for 2-byte aligned types), in 16-byte chunks
  static constexpr uint32_t CPR = (W::RB + (W::ALIGN < 4 ? 2u : 0u) + 15u) / 16u;
  static constexpr uint32_t LOADS = (16u * CPR + 63u) / 64u;
  static constexpr uint32_t BYTES = 16u * CPR * 16u;
};

template <int TYPE, int TG, int NW>
__global__ __launch_bounds__(NW * 64) void k_gemv_mt(WeightView wv, const float *__restrict__ x,
                                                     float *__restrict__ y, uint32_t tokens, uint32_t s_log2) {
  using W = MtW<TYPE>;
  using ST = MtStage<TYPE>;
  constexpr bool kTab = TYPE == IQ2_XXS;
  constexpr uint32_t T = 4u * TG, NT = NW * 64u;
  extern __shared__ __align__(16) uint8_t lds[];
  uint32_t *tab = (uint32_t *)lds;
  uint8_t *xl = lds + (kTab ? kMxTables : 0);

  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rows = wv.rows, k = wv.k;
  // S = 2^s_log2 k slices (shifts: no divisions before the first loads)
  const uint32_t S = 1u << s_log2, RT = (uint32_t)NW >> s_log2, rt = wave >> s_log2, sl = wave & (S - 1u);
  const uint32_t r0 = (blockIdx.x * RT + rt) * 16u;  // first row of the wave
  const uint32_t ks = k >> s_log2, k0 = sl * ks, passes = ks / 256u;
  // per token: digits 3 k bytes + 32, group data k / 8 floats + 4 (the
  // padding spreads the 4 tokens of an MFMA over different LDS banks)
  const uint32_t dstr = 3u * k + 32u, mstr = k / 8u + 4u;
  const uint32_t xbytes = T * dstr + T * mstr * 4u;
  float *const metab = (float *)(xl + T * dstr);
  uint8_t *stg = xl + xbytes + 16u + wave * ST::BYTES;
  float *red = (float *)(xl + xbytes + 16u + (uint32_t)NW * ST::BYTES);
  const BufSrc src = make_src(wv, 0);
  const uint32_t rbytes = (uint32_t)wv.row_bytes;

  // Lane chunks: chunk q = lane + 64 j is chunk q % CPR of row q / CPR
  // (rows past the matrix repeat its last row); a pass region is staged from
  // the 4-byte floor of its start.
  uint32_t vr[ST::LOADS], vc[ST::LOADS];
  bool vok[ST::LOADS];
#pragma unroll
  for (uint32_t j = 0; j < ST::LOADS; ++j) {
    const uint32_t q = lane + 64u * j, r = min(q / ST::CPR, 15u);
    vok[j] = q < 16u * ST::CPR;
    vr[j] = min(r0 + r, rows - 1u) * rbytes;
    vc[j] = 16u * (q - r * ST::CPR);
  }
  // pass start inside a row (first block of the pass)
  auto pstart = [&](uint32_t ps) { return (k0 + 256u * ps) / mt_block_elems<TYPE>() * mt_block_bytes<TYPE>(); };
  struct Regs {
    u32x4 q[ST::LOADS];
  };
  auto fetch = [&](uint32_t ps, Regs &R) {
    const uint32_t po = pstart(min(ps, passes - 1u));
#pragma unroll
    for (uint32_t j = 0; j < ST::LOADS; ++j)
      R.q[j] = __builtin_amdgcn_raw_buffer_load_b128(src.q, (int)(((vr[j] + po) & ~3u) + vc[j]), 0, 0);
  };
  auto put = [&](const Regs &R) {
#pragma unroll
    for (uint32_t j = 0; j < ST::LOADS; ++j)
      if (vok[j]) *(u32x4 *)(stg + 1024u * j + 16u * lane) = R.q[j];
  };

  // x (and the IQ2_XXS tables) first, then the weights of the first two passes
  const uint32_t noct = tokens * (k / 8u), ntot = T * (k / 8u);
  XOct xo[kXr];
#pragma unroll
  for (uint32_t i = 0; i < kXr; ++i)
    if (tid + NT * i < noct) x_load<(uint32_t)T>(x, k, tid + NT * i, xo[i]);
  uint64_t gent = 0;
  if constexpr (kTab) gent = c_grid_mx[tid & 255u];
  __asm__ volatile("" ::: "memory");
  Regs RA, RB;
  fetch(0, RA);
  fetch(1, RB);
  if constexpr (kTab) {
    if (tid < 256u) mx_tables(tab, gent, tid);
  }
#pragma unroll
  for (uint32_t i = 0; i < kXr; ++i)
    if (tid + NT * i < noct) x_store<(uint32_t)T>(xo[i], k, tid + NT * i, xl, dstr, metab, mstr);
  for (uint32_t o = tid + NT * kXr; o < noct; o += NT) {
    XOct v;
    x_load<(uint32_t)T>(x, k, o, v);
    x_store<(uint32_t)T>(v, k, o, xl, dstr, metab, mstr);
  }
  if (tid < 4u) ((uint32_t *)(xl + xbytes))[tid] = 0u;  // the zero plane
  // tokens past `tokens`: zero digits and group data
  for (uint32_t o = noct + tid; o < ntot; o += NT) {
    const uint32_t opt = k / 8u, t = o / opt, ko = 8u * (o % opt);
    uint8_t *dig = xl + (uint64_t)t * dstr + (ko / 16u) * 48u + 8u * ((ko / 8u) & 1u);
#pragma unroll
    for (int d = 0; d < 3; ++d) *(uint2 *)(dig + 16 * d) = make_uint2(0u, 0u);
    if ((ko & 31u) == 0u) *(float4 *)(metab + (uint64_t)t * mstr + ko / 8u) = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __syncthreads();

  const uint32_t n = lane & 15u, kq = lane >> 4;
  // A row of the lane: token (lane % 16) / 4 of each group, plane lane % 4;
  // plane 3 reads a zeroed 16 bytes (its address does not advance)
  const uint32_t at = (lane & 15u) >> 2, ap = lane & 3u;
  const uint32_t amul = ap < 3u ? 1u : 0u;
  const uint32_t abase = ap < 3u ? at * dstr + 16u * ap + 8u * (kq & 1u) + 48u * (kq >> 1) : xbytes;
  const float *meta = metab;
  const uint32_t rowb = min(r0 + n, rows - 1u) * rbytes;  // this lane's row (B operand)
  float acc[TG];
#pragma unroll
  for (int t = 0; t < TG; ++t) acc[t] = 0.f;

  // Two groups at a time: both decodes and all their MFMAs are issued before
  // the first fold reads an MFMA result.
  auto compute = [&](uint32_t ps) {
    const uint8_t *rr = stg + n * (ST::CPR * 16u) + (W::ALIGN < 4 ? ((rowb + pstart(ps)) & 3u) : 0u);
    const uint32_t kp = k0 + 256u * ps;
#pragma unroll
    for (uint32_t g0 = 0; g0 < 8u; g0 += 2u) {
      uint2 u[2];
      float s[2][2], m[2][2];
      long A[2][TG];
      float4 M[2][TG];
      int4v D[2][TG][W::SUB];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t g = g0 + (uint32_t)j, kg = kp + 32u * g;
        W::dec(rr, g, kq, tab, u[j], s[j], m[j]);
#pragma unroll
        for (int tg = 0; tg < TG; ++tg) {
          // A: 8 digits of plane ap of token 4 tg + at
          const uint2 av = *(const uint2 *)(xl + abase + amul * (4u * (uint32_t)tg * dstr + (kg / 16u) * 48u));
          A[j][tg] = (long)(((uint64_t)av.y << 32) | av.x);
          M[j][tg] = *(const float4 *)(meta + (uint64_t)(4u * tg + kq) * mstr + 4u * (kg / 32u));
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint64_t b64 = ((uint64_t)u[j].y << 32) | u[j].x;
#pragma unroll
        for (int tg = 0; tg < TG; ++tg) {
          if constexpr (W::SUB == 1) {
            D[j][tg][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[j][tg], (long)b64, int4v{0, 0, 0, 0}, 0, 0, 0);
          } else {
            // the weights of the other 16 are zeroed (kq < 2: k 0..15)
            const long Blo = (long)(kq < 2u ? b64 : 0ull), Bhi = (long)(kq < 2u ? 0ull : b64);
            D[j][tg][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[j][tg], Blo, int4v{0, 0, 0, 0}, 0, 0, 0);
            D[j][tg][W::SUB - 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[j][tg], Bhi, int4v{0, 0, 0, 0}, 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int tg = 0; tg < TG; ++tg) {
          const float4 Mv = M[j][tg];
#pragma unroll
          for (int h = 0; h < (int)W::SUB; ++h) {
            const int4v Dv = D[j][tg][h];
            const float f = __builtin_fmaf((float)(Dv.z * 256 + Dv.y), 256.f, (float)Dv.x);
            acc[tg] = __builtin_fmaf(s[j][h] * Mv.x, f, acc[tg]);
          }
          if (TYPE == Q4_K) acc[tg] = __builtin_fmaf(-m[j][0], Mv.y + Mv.z, acc[tg]);
          if (TYPE == Q2_K || TYPE == Q6_K)
            acc[tg] = __builtin_fmaf(-m[j][1], Mv.z, __builtin_fmaf(-m[j][0], Mv.y, acc[tg]));
        }
    }
  };

  // passes: the registers of a pass are free once written to the stage; the
  // fetch two passes ahead goes out before the pass is computed (past the
  // last pass it repeats the last one, so the loads in flight never change)
  for (uint32_t ps = 0; ps < passes; ps += 2u) {
    put(RA);
    fetch(ps + 2u, RA);
    compute(ps);
    if (ps + 1u < passes) {
      put(RB);
      fetch(ps + 3u, RB);
      compute(ps + 1u);
    }
  }

  // slices of a row tile added in slice order; lane (kq, n) holds token
  // 4 tg + kq, row n
  if (S > 1) {
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) red[(wave * (uint32_t)TG + tg) * 64u + lane] = acc[tg];
    __syncthreads();
    if (sl != 0u) return;
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) {
      float v = 0.f;
      for (uint32_t q = 0; q < (uint32_t)S; ++q) v += red[((wave + q) * (uint32_t)TG + tg) * 64u + lane];
      acc[tg] = v;
    }
  }
  const uint32_t row = r0 + n;
  if (row < rows) {
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) {
      const uint32_t t = 4u * tg + kq;
      if (t < tokens) y[(uint64_t)t * rows + row] = acc[tg];
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.

namespace {

template <int TYPE> constexpr size_t stage_bytes() {
  return (size_t)Stage<Task<TYPE>::RB, Task<TYPE>::ALIGN>::BYTES + Stage2<TYPE>::BYTES;
}

size_t stage_bytes_of(int type) {
  switch (type) {
    case Q8_0: return stage_bytes<Q8_0>();
    case Q8_0R: return stage_bytes<Q8_0R>();
    case Q4_K: return stage_bytes<Q4_K>();
    case Q6_K: return stage_bytes<Q6_K>();
    case Q2_K: return stage_bytes<Q2_K>();
    case IQ2_XXS: return stage_bytes<IQ2_XXS>();
    default: return 0;
  }
}

// LDS: IQ2_XXS tables, x digits, one weight stage per wave, slice sums.
size_t mx_lds_bytes(const WeightView &wv, uint32_t tokens, int nw) {
  return (wv.type == IQ2_XXS ? (size_t)kMxTables : 0) + (size_t)tokens * wv.k * 3u +
         (size_t)tokens * (wv.k / 8u) * 4u + (size_t)nw * stage_bytes_of(wv.type) + (size_t)nw * 4u * tokens * 4u;
}

int g_force_nw = 0, g_force_s = 0;

}  // namespace

void gemv_mx_override(int nw, int s) {
  g_force_nw = nw;
  g_force_s = s;
}

bool gemv_mx_plan(const WeightView &wv, uint32_t tokens, GemvPlan &p) {
  if (tokens < 1 || tokens > 8 || wv.k % 64u) return false;
  if (wv.w_bytes >= (1ull << 32)) return false;  // byte offsets are 32-bit
  const bool kq = wv.type != Q8_0 && wv.type != Q8_0R;
  // a slice holds whole passes' worth of blocks: k % (256 S) for the K types
  auto slice_ok = [&](int s) { return wv.k % ((kq ? 256u : 64u) * (uint32_t)s) == 0; };
  struct Cand { int nw, s; };
  // for equal rows per workgroup the wider workgroup (more waves per CU) comes first
  const Cand cands[] = {{8, 1}, {8, 2}, {4, 1}, {8, 4}, {4, 2}, {4, 4}};
  // The most rows per workgroup (x digits are prepared once for them) that
  // still give one workgroup per CU; failing that, the most workgroups.
  int best = -1;
  uint32_t best_rows = 0;
  bool best_enough = false;
  for (int i = 0; i < 6; ++i) {
    const Cand &cd = cands[i];
    if (g_force_nw && (cd.nw != g_force_nw || cd.s != g_force_s)) continue;
    if (!slice_ok(cd.s) || mx_lds_bytes(wv, tokens, cd.nw) > kMxMaxLds) continue;
    const uint32_t per = 4u * (uint32_t)(cd.nw / cd.s);
    const bool enough = (wv.rows + per - 1u) / per >= 256u;
    const bool better = best < 0 || (enough && !best_enough) ||
                        (enough && best_enough && per > best_rows) || (!enough && !best_enough && per < best_rows);
    if (better) {
      best = i;
      best_rows = per;
      best_enough = enough;
    }
  }
  if (best < 0) return false;
  p = GemvPlan{};
  p.rows_per_wave = 4;
  p.ksplit = cands[best].s;
  p.waves = cands[best].nw;
  p.kc = wv.k / (uint32_t)p.ksplit;
  p.tiles = (wv.rows + best_rows - 1u) / best_rows;
  p.grid = p.tiles;
  p.lds_bytes = mx_lds_bytes(wv, tokens, p.waves);
  return true;
}

// Workgroups resident at once on the current device for this kernel and LDS
// size (persistent grids are sized to it).
template <int TYPE, int T, int NW, int F>
static hipError_t mx_resident(size_t lds, uint32_t &out) {
  static std::atomic<uint64_t> attr{0};
  hipError_t e = lds_limit_once((const void *)k_gemv_mx<TYPE, T, NW, F>, (int)kMxMaxLds, attr);
  if (e != hipSuccess) return e;
  int dev = 0, cus = 0, per = 0;
  e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k_gemv_mx<TYPE, T, NW, F>, NW * 64, lds);
  if (e != hipSuccess) return e;
  out = (uint32_t)(cus > 0 ? cus : 1) * (uint32_t)(per > 0 ? per : 1);
  return hipSuccess;
}

// p.ksplit slices per matrix; `sec` is unused for F = 0. Gate + up runs
// 2 p.ksplit slices per row quad (one tile per workgroup).
template <int TYPE, int T, int NW, int F>
static hipError_t mx_launch(const WeightView &wv, const float *x, float *y, const GemvPlan &p, const MxSec &sec,
                            hipStream_t s) {
  const uint32_t slices = (uint32_t)p.ksplit * (F == 2 ? 2u : 1u);
  uint32_t grid = p.tiles;
  if (slices == 1) {
    uint32_t res = 0;
    const hipError_t e = mx_resident<TYPE, T, NW, F>(p.lds_bytes, res);
    if (e != hipSuccess) return e;
    grid = grid < res ? grid : res;
  } else if (F != 0) {
    // (the attribute is set once per kernel, as the persistent launch does)
    uint32_t res = 0;
    const hipError_t e = mx_resident<TYPE, T, NW, F>(p.lds_bytes, res);
    if (e != hipSuccess) return e;
  }
  MxGeo geo;
  geo.s_log2 = (uint32_t)__builtin_ctz(slices);
  geo.ntask = wv.k / 64u / (uint32_t)p.ksplit;
  geo.passes = (geo.ntask + 15u) / 16u;
  geo.tq = p.tiles / grid;
  geo.tr = p.tiles % grid;
  hipLaunchKernelGGL((k_gemv_mx<TYPE, T, NW, F>), dim3(grid), dim3(NW * 64), p.lds_bytes, s, wv, x, y, geo, sec);
  return hipGetLastError();
}

template <int TYPE, int T>
static hipError_t mx_go(const WeightView &wv, const float *x, float *y, const GemvPlan &p, hipStream_t s) {
  const MxSec none{};
  return p.waves == 8 ? mx_launch<TYPE, T, 8, 0>(wv, x, y, p, none, s) : mx_launch<TYPE, T, 4, 0>(wv, x, y, p, none, s);
}

template <int TYPE>
static hipError_t mx_t(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                       hipStream_t s) {
  switch (tokens) {
    case 1: return mx_go<TYPE, 1>(wv, x, y, p, s);
    case 2: return mx_go<TYPE, 2>(wv, x, y, p, s);
    case 3: return mx_go<TYPE, 3>(wv, x, y, p, s);
    case 4: return mx_go<TYPE, 4>(wv, x, y, p, s);
    case 5: return mx_go<TYPE, 5>(wv, x, y, p, s);
    case 6: return mx_go<TYPE, 6>(wv, x, y, p, s);
    case 7: return mx_go<TYPE, 7>(wv, x, y, p, s);
    case 8: return mx_go<TYPE, 8>(wv, x, y, p, s);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Multi-token GEMV host side.
namespace {

template <int TYPE> constexpr size_t mt_stage_bytes() { return MtStage<TYPE>::BYTES; }

size_t mt_stage_of(int type) {
  switch (type) {
    case Q8_0: return mt_stage_bytes<Q8_0>();
    case Q4_K: return mt_stage_bytes<Q4_K>();
    case Q6_K: return mt_stage_bytes<Q6_K>();
    case Q2_K: return mt_stage_bytes<Q2_K>();
    case IQ2_XXS: return mt_stage_bytes<IQ2_XXS>();
    default: return 0;
  }
}

// LDS: IQ2_XXS tables, x digits of 4 TG tokens, one stage per wave, slice sums.
size_t mt_lds_bytes(const WeightView &wv, uint32_t tg, int nw) {
  const size_t t = 4u * tg;
  return (wv.type == IQ2_XXS ? (size_t)kMxTables : 0) + t * (3u * wv.k + 32u) + t * (wv.k / 8u + 4u) * 4u + 16u +
         (size_t)nw * mt_stage_of(wv.type) + (size_t)nw * tg * 64u * 4u;
}

}  // namespace

bool gemv_mt_plan(const WeightView &wv, uint32_t tokens, GemvPlan &p) {
  if (tokens < 4 || tokens > 16) return false;
  if (wv.type != Q8_0 && wv.type != Q4_K && wv.type != Q6_K && wv.type != Q2_K && wv.type != IQ2_XXS) return false;
  if (wv.k % 256u || wv.w_bytes >= (1ull << 32)) return false;
  const uint32_t tg = (tokens + 3u) / 4u, tiles = (wv.rows + 15u) / 16u;
  struct Cand { int nw, s; };
  // for equal rows per workgroup the wider workgroup comes first
  const Cand cands[] = {{8, 1}, {8, 2}, {4, 1}, {8, 4}, {4, 2}, {8, 8}, {4, 4}};
  int best = -1;
  uint32_t best_rt = 0;
  bool best_enough = false;
  for (int i = 0; i < 7; ++i) {
    const Cand &cd = cands[i];
    if (g_force_nw && (cd.nw != g_force_nw || cd.s != g_force_s)) continue;
    if (wv.k % (256u * (uint32_t)cd.s) || mt_lds_bytes(wv, tg, cd.nw) > kMxMaxLds) continue;
    const uint32_t rt = (uint32_t)(cd.nw / cd.s);
    const bool enough = (tiles + rt - 1u) / rt >= 256u;
    const bool better = best < 0 || (enough && !best_enough) || (enough && best_enough && rt > best_rt) ||
                        (!enough && !best_enough && rt < best_rt);
    if (better) {
      best = i;
      best_rt = rt;
      best_enough = enough;
    }
  }
  if (best < 0) return false;
  p = GemvPlan{};
  p.rows_per_wave = 16;
  p.ksplit = cands[best].s;
  p.waves = cands[best].nw;
  p.kc = wv.k / (uint32_t)p.ksplit;
  p.tiles = (tiles + best_rt - 1u) / best_rt;
  p.grid = p.tiles;
  p.lds_bytes = mt_lds_bytes(wv, tg, p.waves);
  return true;
}

template <int TYPE, int TG, int NW>
static hipError_t mt_launch(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                            hipStream_t s) {
  static std::atomic<uint64_t> attr{0};
  const hipError_t e = lds_limit_once((const void *)k_gemv_mt<TYPE, TG, NW>, (int)kMxMaxLds, attr);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gemv_mt<TYPE, TG, NW>), dim3(p.grid), dim3(NW * 64), p.lds_bytes, s, wv, x, y, tokens,
                     (uint32_t)__builtin_ctz((unsigned)p.ksplit));
  return hipGetLastError();
}

template <int TYPE, int TG>
static hipError_t mt_go(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                        hipStream_t s) {
  return p.waves == 8 ? mt_launch<TYPE, TG, 8>(wv, x, y, tokens, p, s) : mt_launch<TYPE, TG, 4>(wv, x, y, tokens, p, s);
}

template <int TYPE>
static hipError_t mt_t(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                       hipStream_t s) {
  switch ((tokens + 3u) / 4u) {
    case 1: return mt_go<TYPE, 1>(wv, x, y, tokens, p, s);
    case 2: return mt_go<TYPE, 2>(wv, x, y, tokens, p, s);
    case 3: return mt_go<TYPE, 3>(wv, x, y, tokens, p, s);
    case 4: return mt_go<TYPE, 4>(wv, x, y, tokens, p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv_mt(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                          hipStream_t s) {
  switch (wv.type) {
    case Q8_0: return mt_t<Q8_0>(wv, x, y, tokens, p, s);
    case Q4_K: return mt_t<Q4_K>(wv, x, y, tokens, p, s);
    case Q6_K: return mt_t<Q6_K>(wv, x, y, tokens, p, s);
    case Q2_K: return mt_t<Q2_K>(wv, x, y, tokens, p, s);
    case IQ2_XXS: return mt_t<IQ2_XXS>(wv, x, y, tokens, p, s);
    default: return hipErrorInvalidValue;
  }
}

// Fused launches: the plan of matrix 0 (k slices and waves, so that every row
// is summed as its one-matrix launch sums it); gate + up runs 8 waves.
namespace {

bool mx_multi_plan(const WeightView &wv0, uint32_t tokens, int mode, GemvPlan &p) {
  if (tokens < 1 || tokens > 3 || !gemv_mx_plan(wv0, tokens, p)) return false;
  if (mode == 2) {
    p.waves = 8;
    p.lds_bytes = mx_lds_bytes(wv0, tokens, 8);
    if (p.lds_bytes > kMxMaxLds || 2 * p.ksplit > 8) return false;
  }
  return true;
}

template <int TYPE, int T, int F>
hipError_t mx_multi_go(uint32_t n, const WeightView *wvs, const float *x, float *const *ys, const GemvPlan &p0,
                       hipStream_t s) {
  GemvPlan p = p0;
  const uint32_t slices = (uint32_t)p.ksplit * (F == 2 ? 2u : 1u);
  const uint32_t rpt = 4u * (uint32_t)p.waves / slices;
  MxSec sec{};
  sec.n = n;
  uint32_t tiles = 0;
  for (uint32_t q = 0; q < n; ++q) {
    sec.rows[q] = wvs[q].rows;
    sec.w[q] = wvs[q].w;
    sec.w_bytes[q] = wvs[q].w_bytes;
    sec.scales_off[q] = wvs[q].scales_off;
    sec.y[q] = ys[q];
    tiles += F == 1 || q == 0 ? (wvs[q].rows + rpt - 1u) / rpt : 0u;
    sec.tend[q] = tiles;
  }
  p.tiles = tiles;
  if (p.waves == 8) return mx_launch<TYPE, T, 8, F>(wvs[0], x, ys[0], p, sec, s);
  if constexpr (F == 1) return mx_launch<TYPE, T, 4, F>(wvs[0], x, ys[0], p, sec, s);
  return hipErrorInvalidValue;
}

template <int TYPE>
hipError_t mx_multi_t(int mode, uint32_t n, const WeightView *wvs, const float *x, float *const *ys, uint32_t tokens,
                      const GemvPlan &p, hipStream_t s) {
  switch (tokens * 4u + (uint32_t)mode) {
    case 1 * 4 + 1: return mx_multi_go<TYPE, 1, 1>(n, wvs, x, ys, p, s);
    case 2 * 4 + 1: return mx_multi_go<TYPE, 2, 1>(n, wvs, x, ys, p, s);
    case 3 * 4 + 1: return mx_multi_go<TYPE, 3, 1>(n, wvs, x, ys, p, s);
    case 1 * 4 + 2: return mx_multi_go<TYPE, 1, 2>(n, wvs, x, ys, p, s);
    case 2 * 4 + 2: return mx_multi_go<TYPE, 2, 2>(n, wvs, x, ys, p, s);
    case 3 * 4 + 2: return mx_multi_go<TYPE, 3, 2>(n, wvs, x, ys, p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool gemv_mx_multi_applies(const WeightView &wv0, uint32_t tokens, int mode) {
  GemvPlan p;
  return mx_multi_plan(wv0, tokens, mode, p);
}

hipError_t launch_gemv_mx_multi(int mode, uint32_t n, const WeightView *wvs, const float *x, float *const *ys,
                                uint32_t tokens, hipStream_t s) {
  GemvPlan p;
  if (n < 1 || n > 4 || !mx_multi_plan(wvs[0], tokens, mode, p)) return hipErrorInvalidValue;
  switch (wvs[0].type) {
    case Q8_0: return mx_multi_t<Q8_0>(mode, n, wvs, x, ys, tokens, p, s);
    case Q8_0R: return mx_multi_t<Q8_0R>(mode, n, wvs, x, ys, tokens, p, s);
    case Q4_K: return mx_multi_t<Q4_K>(mode, n, wvs, x, ys, tokens, p, s);
    case Q6_K: return mx_multi_t<Q6_K>(mode, n, wvs, x, ys, tokens, p, s);
    case Q2_K: return mx_multi_t<Q2_K>(mode, n, wvs, x, ys, tokens, p, s);
    case IQ2_XXS: return mx_multi_t<IQ2_XXS>(mode, n, wvs, x, ys, tokens, p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv_mx(const WeightView &wv, const float *x, float *y, uint32_t tokens, const GemvPlan &p,
                          hipStream_t s) {
  switch (wv.type) {
    case Q8_0: return mx_t<Q8_0>(wv, x, y, tokens, p, s);
    case Q8_0R: return mx_t<Q8_0R>(wv, x, y, tokens, p, s);
    case Q4_K: return mx_t<Q4_K>(wv, x, y, tokens, p, s);
    case Q6_K: return mx_t<Q6_K>(wv, x, y, tokens, p, s);
    case Q2_K: return mx_t<Q2_K>(wv, x, y, tokens, p, s);
    case IQ2_XXS: return mx_t<IQ2_XXS>(wv, x, y, tokens, p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace eff
