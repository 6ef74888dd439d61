// Quantized matrix products from 2 tokens up for Q2_K, Q4_K, IQ2_XXS, Q8_0
// and Q6_K, to f32 accuracy (the reference runs the K/IQ types through its f32
// generic kernel at every token count, ops.js:1013-1099, and Q8_0 below its
// DRIFT threshold through its f32 tiled GEMM; its f16 GEMMs read Q8_0/Q4_0
// only, kernels.drift.wgsl.js:33, kernels.gemm2.wgsl.js:51):
//   Y[t][row] = sum_k W[row][k] X[t][k].
//
// Weights. Per 256-weight block the decoders of kernels.wgsl.js:154-396 are
// an integer u times a scale, minus a group minimum:
//   Q2_K     w = d (sc & 15) q - dmin (sc >> 4)   u = (sc & 15) q <= 45     (16-weight groups)
//   Q4_K     w = d sc q - dmin m                  u = sc q        <= 945    (32-weight groups)
//   IQ2_XXS  w = (d / 8) (2 ls + 1) (+-g)         u = (2 ls + 1)(+-g) <= 1333
//   Q8_0     w = d_j q                            u = q, |q| <= 127         (scale d_j per 32)
//   Q6_K     w = d sc_j (q - 32)                  u = q - 32, |u| <= 32     (scale d sc_j per 16)
// so for the first three  sum_k w x = d sum_k u x - dmin sum_g mn_g S_g,
// S_g = sum of x over group g, with one scale per block; Q8_0 and Q6_K keep a
// scale per 32 or 16 weights (sc_j u can pass 2048 for Q6_K). Every u is an
// integer below 2048, exact in fp16.
//
// x. Per token and block, x is scaled by 2^-e with max|x| < 2^(e) and split
// into fp16 parts hi = fp16(x 2^(14-e)), lo = fp16(x 2^(14-e) - hi): 22
// significant bits. k_sx_prep writes them (and hi/lo of the group sums) once
// per launch, in the operand order of the matrix instruction.
//
// MFMA. v_mfma_f32_32x32x16_f16 multiplies A = 16 tokens x {hi, lo} (32 rows)
// by B = u of 32 weight rows (16 k): products of fp16 values are exact in the
// f32 accumulator. Lane l holds D for weight row l % 32 and x rows
// 8 (v / 4) + 4 (l / 32) + v % 4: v < 8 the hi part of a token, v + 8 its lo
// part. One more MFMA per block forms the minimum sums (A = group sums, B =
// the group minima), and each block is folded once:
//   acc += ((D_hi + D_lo) d - (Dm_hi + Dm_lo) dmin') 2^(e - 14).
// Q8_0 and Q6_K fold each group of FG steps (2: a 32-weight block, 1: 16
// weights) with its own scale, starting the accumulation over after each:
//   acc += (D_hi + D_lo) s_j 2^(e - 14).
//
// Workgroup: NW waves over the same 32 RF weight rows and TT tiles of 16
// tokens, each wave on its own k blocks; the waves' sums are added in a fixed
// order through LDS. Raw blocks are staged per wave by direct-to-LDS dword
// loads into rows of an odd number of dwords (the 32 rows a matrix
// instruction reads land in 32 different banks).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
#include "eff_formats.h"
#include "eff_kernels.h"

namespace eff {

static __constant__ uint64_t c_grid_sx[256] = {
#include "iq2xxs_grid.inc"
};

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));


// Types with group minima (their group sums of x form a 17th slot)
template <int TYPE>
constexpr bool sx_mins() {
  return TYPE == Q2_K || TYPE == Q4_K;
}

template <int TYPE>
constexpr uint32_t sx_slots() {  // x slots of 1 KB per (token tile, block): 16 steps (+ group sums)
  return sx_mins<TYPE>() ? 17u : 16u;
}

// ---------------------------------------------------------------------------
// x -> fp16 hi/lo parts. A wave per (token, block); lane l holds x values
// 4l .. 4l+3 of the block, i.e. step l / 4, lane half (l / 2) % 2, halves
// 4 (l % 2) .. of the 8 a lane feeds to one matrix instruction.
// Layout per (token tile tt, block b): slot s (1 KB) at ((tt nb + b) NS + s) KB,
// lane L's 16 bytes at 16 L, L = 32 half + 16 part + token % 16.
// xp[(tt nb + b) 16 + token % 16] = 2^(e - 14) (NaN for a block holding a
// non-finite x, which makes every output of that token non-finite).
template <int TYPE>
__global__ __launch_bounds__(256) void k_sx_prep(const float *__restrict__ x, uint32_t tokens, uint32_t k,
                                                 uint8_t *__restrict__ xa, float *__restrict__ xp) {
  constexpr uint32_t NS = sx_slots<TYPE>();
  const uint32_t lane = threadIdx.x & 63u, bi = blockIdx.x, nb = k / 256u;
  const uint32_t t = blockIdx.y * 4u + (threadIdx.x >> 6);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (t < tokens) v = *(const float4 *)(x + (uint64_t)t * k + 256u * bi + 4u * lane);
  const bool fin = isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
  // the block's max |x| as u32 bit patterns (non-negative floats order as
  // their bits; a non-finite value counts as infinity): DPP within rows,
  // then rows 1 and 3 (row_bcast:15), row 3 (row_bcast:31), lane 63
  uint32_t mb = max(max(__float_as_uint(fabsf(v.x)), __float_as_uint(fabsf(v.y))),
                    max(__float_as_uint(fabsf(v.z)), __float_as_uint(fabsf(v.w))));
  mb = fin ? mb : 0x7F800000u;
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x141, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x140, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x142, 0xA, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x143, 0xC, 0xF, false));
  const float m = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)mb, 63));
  const bool ok = m < INFINITY;
  int e = 0;
  if (ok && m > 0.f) (void)frexpf(m, &e);  // m < 2^e
  const int sh = 14 - e;
  float xs[4] = {ldexpf(v.x, sh), ldexpf(v.y, sh), ldexpf(v.z, sh), ldexpf(v.w, sh)};
  if (!ok) xs[0] = xs[1] = xs[2] = xs[3] = 0.f;
  half4 hi, lo;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hi[i] = (_Float16)xs[i];
    lo[i] = (_Float16)(xs[i] - (float)hi[i]);
  }
  const uint32_t tt = t >> 4, tl = t & 15u;
  uint8_t *blk = xa + ((uint64_t)tt * nb + bi) * NS * 1024u;
  uint8_t *slot = blk + (lane >> 2) * 1024u;
  const uint32_t hf = (lane >> 1) & 1u, q = lane & 1u;
  *(half4 *)(slot + 16u * (32u * hf + tl) + 8u * q) = hi;
  *(half4 *)(slot + 16u * (32u * hf + 16u + tl) + 8u * q) = lo;
  if constexpr (sx_mins<TYPE>()) {
    // group sums (16 values for Q2_K, 32 for Q4_K), scaled to the range of x
    constexpr uint32_t GL = TYPE == Q2_K ? 4u : 8u;  // lanes per group
    // the group's lanes: own + lane ^ 1, + lane ^ 2 (quad permutes), and
    // for 8 lanes + the other quad's sum (row_half_mirror: lane 7 - i)
    float sum = (xs[0] + xs[1]) + (xs[2] + xs[3]);
    sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0xB1, 0xF, 0xF, false));
    sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x4E, 0xF, 0xF, false));
    if (GL == 8u)
      sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x141, 0xF, 0xF, false));
    const float sp = sum * (TYPE == Q2_K ? 0.0625f : 0.03125f);
    const _Float16 shi = (_Float16)sp, slo = (_Float16)(sp - (float)shi);
    uint8_t *ms = blk + 16u * 1024u;
    if (lane % GL == 0u) {
      const uint32_t g = lane / GL, hm = g >> 3, jj = g & 7u;
      *(_Float16 *)(ms + 16u * (32u * hm + tl) + 2u * jj) = shi;
      *(_Float16 *)(ms + 16u * (32u * hm + 16u + tl) + 2u * jj) = slo;
    }
    if (TYPE == Q4_K && lane < 2u) *(u32x4 *)(ms + 16u * (32u + 16u * lane + tl)) = u32x4{0u, 0u, 0u, 0u};
  }
  if (lane == 0u) xp[((uint64_t)tt * nb + bi) * 16u + tl] = ok ? ldexpf(1.f, e - 14) : NAN;
}

// ---------------------------------------------------------------------------
// The same preparation inside the product for up to 8 tokens (one block of
// 8 tokens per call, the wave's lanes holding 4 values of each as in
// k_sx_prep, the same arithmetic): into the wave's LDS, whose fragment slots
// hold only the rows of tokens 0..7 (kSxFxSlot bytes: row
// 16 hf + 8 part + token, the MFMA lanes of tokens 8..15 reading zeros), and
// the token's scale into xps[token]. Row r of slot s sits at r ^ (s % 16):
// the 16 slots a store spans are 512 bytes apart, and without the swizzle
// its lanes would fall into the same banks.
constexpr uint32_t kSxFxSlot = 512;

__device__ __forceinline__ uint32_t sx_fx_at(uint32_t s, uint32_t row) { return s * kSxFxSlot + 16u * (row ^ (s & 15u)); }

// All 8 token rows of one block (v[t]: token t's 4 values of the lane; rows
// of absent tokens read zeros), phase by phase across the tokens so that
// their 8 dependent chains interleave.
template <int TYPE>
__device__ __forceinline__ void sx_fill8(const float4 (&v)[8], uint32_t lane, uint8_t *fr, float *xps) {
  // max |x| of each token's block as u32 bit patterns (non-negative floats
  // order as their bits; a non-finite value counts as infinity): DPP within
  // rows, then rows 1 and 3 (row_bcast:15), row 3 (row_bcast:31), lane 63
  uint32_t m[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const bool fin = isfinite(v[t].x) && isfinite(v[t].y) && isfinite(v[t].z) && isfinite(v[t].w);
    const uint32_t a = max(max(__float_as_uint(fabsf(v[t].x)), __float_as_uint(fabsf(v[t].y))),
                           max(__float_as_uint(fabsf(v[t].z)), __float_as_uint(fabsf(v[t].w))));
    m[t] = fin ? a : 0x7F800000u;
  }
#define SX_DPP_MAX(ctrl, rmask)                                                                 \
  _Pragma("unroll") for (int t = 0; t < 8; ++t)                                                 \
    m[t] = max(m[t], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m[t], ctrl, rmask, 0xF, false));
  SX_DPP_MAX(0xB1, 0xF)
  SX_DPP_MAX(0x4E, 0xF)
  SX_DPP_MAX(0x141, 0xF)
  SX_DPP_MAX(0x140, 0xF)
  SX_DPP_MAX(0x142, 0xA)
  SX_DPP_MAX(0x143, 0xC)
#undef SX_DPP_MAX
  float xs[8][4];
  float sc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float mf = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)m[t], 63));
    const bool ok = mf < INFINITY;
    int e = 0;
    if (ok && mf > 0.f) (void)frexpf(mf, &e);  // mf < 2^e
    const int sh = 14 - e;
    xs[t][0] = ok ? ldexpf(v[t].x, sh) : 0.f;
    xs[t][1] = ok ? ldexpf(v[t].y, sh) : 0.f;
    xs[t][2] = ok ? ldexpf(v[t].z, sh) : 0.f;
    xs[t][3] = ok ? ldexpf(v[t].w, sh) : 0.f;
    sc[t] = ok ? ldexpf(1.f, e - 14) : NAN;
  }
  const uint32_t st = lane >> 2, hf = (lane >> 1) & 1u, q = lane & 1u;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    half4 hi, lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hi[i] = (_Float16)xs[t][i];
      lo[i] = (_Float16)(xs[t][i] - (float)hi[i]);
    }
    *(half4 *)(fr + sx_fx_at(st, 16u * hf + t) + 8u * q) = hi;
    *(half4 *)(fr + sx_fx_at(st, 16u * hf + 8u + t) + 8u * q) = lo;
  }
  if constexpr (sx_mins<TYPE>()) {
    static_assert(TYPE == Q2_K, "16-value group sums");
    // group sums: the 4 lanes of a group, (own + lane ^ 1) + (lane ^ 2)'s pair
    float sum[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) sum[t] = (xs[t][0] + xs[t][1]) + (xs[t][2] + xs[t][3]);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      sum[t] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum[t]), 0xB1, 0xF, 0xF, false));
#pragma unroll
    for (int t = 0; t < 8; ++t)
      sum[t] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum[t]), 0x4E, 0xF, 0xF, false));
    if (lane % 4u == 0u) {
      const uint32_t g = lane / 4u, hm = g >> 3, jj = g & 7u;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float sp = sum[t] * 0.0625f;
        const _Float16 shi = (_Float16)sp, slo = (_Float16)(sp - (float)shi);
        *(_Float16 *)(fr + sx_fx_at(16u, 16u * hm + t) + 2u * jj) = shi;
        *(_Float16 *)(fr + sx_fx_at(16u, 16u * hm + 8u + t) + 2u * jj) = slo;
      }
    }
  }
  if (lane < 8u) xps[lane] = lane == 0u ? sc[0] : lane == 1u ? sc[1] : lane == 2u ? sc[2] : lane == 3u ? sc[3]
                            : lane == 4u ? sc[4] : lane == 5u ? sc[5] : lane == 6u ? sc[6] : sc[7];
}

// ---------------------------------------------------------------------------
// Weight operands. `r` points to the staged dwords of the lane's row (the
// block's first byte at byte offset `a` of r[0]); `step` returns the 8
// weights u of step s (k 16 s + 8 h .. + 7 of the block) for lane half h.

// 4 bytes b (each < 1024 after the caller's masking) -> 1024 + b as fp16 pairs
__device__ __forceinline__ half2v h1024_lo(uint32_t v) {
  return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u));
}
__device__ __forceinline__ half2v h1024_hi(uint32_t v) {
  return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
}

// 8 unsigned bytes q (v0: q0..q3, v1: q4..q7) -> sc * q as fp16, exact
// (sc * q < 2048; the fused multiply-add rounds once: (1024 + q) sc - 1024 sc)
__device__ __forceinline__ half8 dec_scaled(uint32_t v0, uint32_t v1, uint32_t sc) {
  const _Float16 s = (_Float16)(float)sc, o = (_Float16)(-1024.f * (float)sc);
  const half2v s2 = {s, s}, o2 = {o, o};
  const half2v a = __builtin_elementwise_fma(h1024_lo(v0), s2, o2);
  const half2v b = __builtin_elementwise_fma(h1024_hi(v0), s2, o2);
  const half2v c = __builtin_elementwise_fma(h1024_lo(v1), s2, o2);
  const half2v d = __builtin_elementwise_fma(h1024_hi(v1), s2, o2);
  return half8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// 8 unsigned bytes -> fp16 (exact below 1024)
__device__ __forceinline__ half8 dec_plain(uint32_t v0, uint32_t v1) {
  const half2v o2 = {(_Float16)-1024.f, (_Float16)-1024.f};
  const half2v a = h1024_lo(v0) + o2, b = h1024_hi(v0) + o2, c = h1024_lo(v1) + o2, d = h1024_hi(v1) + o2;
  return half8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t *w, uint32_t i) { return (w[i >> 2] >> (8u * (i & 3u))) & 0xFFu; }

template <int TYPE> struct SxW;

// Q2_K, 84 bytes: scales[16] | qs[64] | d | dmin (kernels.wgsl.js:194-222).
// Step s = the 16-weight group s: qs bytes 32 n + 16 h' + i at bit shift 2 g
// (s = 8 n + 2 g + h'), scale byte s.
template <> struct SxW<Q2_K> {
  static constexpr uint32_t BB = 84, DW = 21, ST = 21;
  static constexpr bool MINS = true;
  static constexpr int FG = 16;  // steps per fold (one scale for the block)
  uint32_t sc[4];
  float d, dm;
  __device__ void block(const uint32_t *r, uint32_t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = r[i];
    const uint32_t w = r[20];
    d = h2f(w & 0xFFFFu);
    dm = 16.f * h2f(w >> 16);  // group sums are stored divided by 16
  }
  __device__ float scale(int) const { return d; }
  __device__ half8 step(const uint32_t *r, int s, uint32_t h, const uint32_t *) const {
    const int n = s >> 3, hp = s & 1, g = (s >> 1) & 3;
    const uint32_t *p = r + 4 + 8 * n + 4 * hp + 2u * h;
    const uint32_t v0 = (p[0] >> (2 * g)) & 0x03030303u, v1 = (p[1] >> (2 * g)) & 0x03030303u;
    return dec_scaled(v0, v1, byte_of(sc, (uint32_t)s) & 15u);
  }
  // the qs dwords every step of lane half h reads: pr[4 n + 2 h' + i]
  static constexpr int NP = 8;
  __device__ void preload(const uint32_t *r, uint32_t h, uint32_t (&pr)[NP]) const {
#pragma unroll
    for (int i = 0; i < NP; ++i) pr[i] = r[4 + 8 * (i >> 2) + 4 * ((i >> 1) & 1) + 2u * h + (i & 1)];
  }
  __device__ half8 step_pre(const uint32_t (&pr)[NP], int s, uint32_t, const uint32_t *) const {
    const int n = s >> 3, hp = s & 1, g = (s >> 1) & 3;
    const uint32_t v0 = (pr[4 * n + 2 * hp] >> (2 * g)) & 0x03030303u;
    const uint32_t v1 = (pr[4 * n + 2 * hp + 1] >> (2 * g)) & 0x03030303u;
    return dec_scaled(v0, v1, byte_of(sc, (uint32_t)s) & 15u);
  }
  __device__ half8 mins(uint32_t h) const {
    const uint32_t w0 = h ? sc[2] : sc[0], w1 = h ? sc[3] : sc[1];
    return dec_plain((w0 >> 4) & 0x0F0F0F0Fu, (w1 >> 4) & 0x0F0F0F0Fu);
  }
};

// Q4_K, 144 bytes: d | dmin | scales[12] | qs[128] (kernels.wgsl.js:94-104,
// 227-250). Step s: sub-block pair j = s / 4, nibble (s / 2) % 2, qs bytes
// 32 j + 16 (s % 2) + 8 h ..; 6-bit scale and minimum of sub-block s / 2.
template <> struct SxW<Q4_K> {
  static constexpr uint32_t BB = 144, DW = 36, ST = 37;
  static constexpr bool MINS = true;
  static constexpr int FG = 16;
  uint32_t q[3];
  float d, dm;
  __device__ void block(const uint32_t *r, uint32_t) {
    const uint32_t w = r[0];
    d = h2f(w & 0xFFFFu);
    dm = 32.f * h2f(w >> 16);  // group sums are stored divided by 32
    q[0] = r[1];
    q[1] = r[2];
    q[2] = r[3];
  }
  __device__ float scale(int) const { return d; }
  __device__ uint32_t scale(uint32_t i) const {
    return i < 4u ? byte_of(q, i) & 63u : (byte_of(q, i + 4u) & 15u) | ((byte_of(q, i - 4u) >> 6) << 4);
  }
  __device__ uint32_t minv(uint32_t i) const {
    return i < 4u ? byte_of(q, i + 4u) & 63u : (byte_of(q, i + 4u) >> 4) | ((byte_of(q, i) >> 6) << 4);
  }
  __device__ half8 step(const uint32_t *r, int s, uint32_t h, const uint32_t *) const {
    const int j = s >> 2, nib = (s >> 1) & 1;
    const uint32_t *p = r + 4 + 8 * j + 4 * (s & 1) + 2u * h;
    const uint32_t v0 = (p[0] >> (4 * nib)) & 0x0F0F0F0Fu, v1 = (p[1] >> (4 * nib)) & 0x0F0F0F0Fu;
    return dec_scaled(v0, v1, scale((uint32_t)s >> 1));
  }
  // the qs dwords every step of lane half h reads: pr[4 j + 2 (s % 2) + i]
  static constexpr int NP = 16;
  __device__ void preload(const uint32_t *r, uint32_t h, uint32_t (&pr)[NP]) const {
#pragma unroll
    for (int i = 0; i < NP; ++i) pr[i] = r[4 + 8 * (i >> 2) + 4 * ((i >> 1) & 1) + 2u * h + (i & 1)];
  }
  __device__ half8 step_pre(const uint32_t (&pr)[NP], int s, uint32_t, const uint32_t *) const {
    const int j = s >> 2, nib = (s >> 1) & 1;
    const uint32_t v0 = (pr[4 * j + 2 * (s & 1)] >> (4 * nib)) & 0x0F0F0F0Fu;
    const uint32_t v1 = (pr[4 * j + 2 * (s & 1) + 1] >> (4 * nib)) & 0x0F0F0F0Fu;
    return dec_scaled(v0, v1, scale((uint32_t)s >> 1));
  }
  __device__ half8 mins(uint32_t h) const {
    uint32_t v0 = 0, v1 = 0;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      v0 |= minv(i) << (8u * i);
      v1 |= minv(i + 4u) << (8u * i);
    }
    const half8 m = dec_plain(v0, v1);
    const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    return h ? z : m;
  }
};

// IQ2_XXS, 66 bytes: d | 8 x (grid indices a0, signs + scale a1)
// (kernels.wgsl.js:368-396). Step s: group s / 2, grid entry l = 2 (s % 2) + h.
// LDS tables: the grid as fp16 (256 x 16 bytes) and the fp16 sign bits of
// each 7-bit sign field with its parity bit (128 x 16 bytes).
template <> struct SxW<IQ2_XXS> {
  static constexpr uint32_t BB = 66, DW = 17, ST = 17;
  static constexpr bool MINS = false;
  static constexpr int FG = 16;
  uint32_t a;  // byte offset of the block in r[0] (0 or 2)
  float d, dm;
  __device__ void block(const uint32_t *r, uint32_t off) {
    a = off;
    d = 0.125f * h2f(off ? (r[0] >> 16) : (r[0] & 0xFFFFu));
    dm = 0.f;
  }
  __device__ float scale(int) const { return d; }
  __device__ half8 step(const uint32_t *r, int s, uint32_t h, const uint32_t *tab) const {
    const uint32_t ib = (uint32_t)s >> 1, o = a + 2u + 8u * ib, sh = o & 3u;
    const uint32_t *p = r + (o >> 2);
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
    const uint32_t a0 = __builtin_amdgcn_alignbyte(w1, w0, sh), a1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
    const uint32_t l = 2u * ((uint32_t)s & 1u) + h;
    const uint32_t gi = (a0 >> (8u * l)) & 0xFFu, sg = (a1 >> (7u * l)) & 127u;
    const u32x4 g = *(const u32x4 *)(tab + 4u * gi), m = *(const u32x4 *)(tab + 1024u + 4u * sg);
    const _Float16 c = (_Float16)(float)(2u * (a1 >> 28) + 1u);
    const half2v c2 = {c, c};
    const half2v v0 = __builtin_bit_cast(half2v, g.x ^ m.x) * c2, v1 = __builtin_bit_cast(half2v, g.y ^ m.y) * c2;
    const half2v v2 = __builtin_bit_cast(half2v, g.z ^ m.z) * c2, v3 = __builtin_bit_cast(half2v, g.w ^ m.w) * c2;
    return half8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
  }
  __device__ half8 mins(uint32_t) const { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }
  // the block's 17 dwords from the one holding its first group (dword
  // (a + 2) / 4 of the row; the stage's slack covers the last)
  static constexpr int NP = 17;
  __device__ void preload(const uint32_t *r, uint32_t, uint32_t (&pr)[NP]) const {
    const uint32_t *p = r + ((a + 2u) >> 2);
#pragma unroll
    for (int i = 0; i < NP; ++i) pr[i] = p[i];
  }
  __device__ half8 step_pre(const uint32_t (&pr)[NP], int s, uint32_t h, const uint32_t *tab) const {
    const uint32_t ib = (uint32_t)s >> 1, sh = (a + 2u) & 3u;
    const uint32_t w0 = pr[2 * ib], w1 = pr[2 * ib + 1], w2 = pr[2 * ib + 2];
    const uint32_t a0 = __builtin_amdgcn_alignbyte(w1, w0, sh), a1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
    const uint32_t l = 2u * ((uint32_t)s & 1u) + h;
    const uint32_t gi = (a0 >> (8u * l)) & 0xFFu, sg = (a1 >> (7u * l)) & 127u;
    const u32x4 g = *(const u32x4 *)(tab + 4u * gi), m = *(const u32x4 *)(tab + 1024u + 4u * sg);
    const _Float16 c = (_Float16)(float)(2u * (a1 >> 28) + 1u);
    const half2v c2 = {c, c};
    const half2v v0 = __builtin_bit_cast(half2v, g.x ^ m.x) * c2, v1 = __builtin_bit_cast(half2v, g.y ^ m.y) * c2;
    const half2v v2 = __builtin_bit_cast(half2v, g.z ^ m.z) * c2, v3 = __builtin_bit_cast(half2v, g.w ^ m.w) * c2;
    return half8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
  }
};

// 8 signed bytes q -> q as fp16 (exact): 1024 + (q + 128) - 1152
__device__ __forceinline__ half8 dec_signed(uint32_t v0, uint32_t v1) {
  const half2v o2 = {(_Float16)-1152.f, (_Float16)-1152.f};
  v0 ^= 0x80808080u;
  v1 ^= 0x80808080u;
  const half2v a = h1024_lo(v0) + o2, b = h1024_hi(v0) + o2, c = h1024_lo(v1) + o2, d = h1024_hi(v1) + o2;
  return half8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// Q8_0, 256 weights = 8 blocks of 34 bytes, d | q[32] (kernels.wgsl.js:154-160).
// Step s: block s / 2, quants 16 (s % 2) + 8 h .. + 7 (bytes 34 (s / 2) + 2 +
// 16 (s % 2) + 8 h ..), u = q. The 8 blocks have their own d: one fold per
// 2 steps (FG = 2), with that block's d. The 256 weights are 4-byte aligned
// (rows are 272 (k / 256) bytes); the quants of odd blocks are too, those of
// even blocks 2 bytes past a dword.
template <> struct SxW<Q8_0> {
  static constexpr uint32_t BB = 272, DW = 68, ST = 69;
  static constexpr bool MINS = false;
  static constexpr int FG = 2;
  static constexpr int NP = 0;  // steps read the stage (no register copy of the block)
  float d, dm, ds[8];
  __device__ void block(const uint32_t *r, uint32_t) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w = r[(34 * j) >> 2];
      ds[j] = h2f((j & 1) ? (w >> 16) : (w & 0xFFFFu));
    }
    d = 1.f;
    dm = 0.f;
  }
  __device__ float scale(int g) const { return ds[g]; }
  __device__ half8 step(const uint32_t *r, int s, uint32_t h, const uint32_t *) const {
    const uint32_t o = 34u * (uint32_t)(s >> 1) + 2u + 16u * (uint32_t)(s & 1) + 8u * h, sh = o & 3u;
    const uint32_t *p = r + (o >> 2);
    return dec_signed(__builtin_amdgcn_alignbyte(p[1], p[0], sh), __builtin_amdgcn_alignbyte(p[2], p[1], sh));
  }
  __device__ half8 mins(uint32_t) const { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }
  __device__ void preload(const uint32_t *, uint32_t, uint32_t (&)[1]) const {}
  __device__ half8 step_pre(const uint32_t (&)[1], int, uint32_t, const uint32_t *) const { return half8{}; }
};

// Q8_0R, the repacked layout (kernels.bloques.wgsl.js:19-35): the quants of
// the row's 8 blocks (256 bytes, from the quant region) then their 8 scales
// (16 bytes, from the scale region) form one staged row of 68 dwords; the
// decoded weights, and so the outputs, are those of the Q8_0 tensor.
template <> struct SxW<Q8_0R> {
  static constexpr uint32_t BB = 0, DW = 68, ST = 69;   // BB: the regions advance by 256 and 16 per block
  static constexpr bool MINS = false;
  static constexpr int FG = 2;
  static constexpr int NP = 0;
  float d, dm, ds[8];
  __device__ void block(const uint32_t *r, uint32_t) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w = r[64 + (j >> 1)];
      ds[j] = h2f((j & 1) ? (w >> 16) : (w & 0xFFFFu));
    }
    d = 1.f;
    dm = 0.f;
  }
  __device__ float scale(int g) const { return ds[g]; }
  __device__ half8 step(const uint32_t *r, int s, uint32_t h, const uint32_t *) const {
    const uint32_t *p = r + 8u * (uint32_t)(s >> 1) + 4u * (uint32_t)(s & 1) + 2u * h;
    return dec_signed(p[0], p[1]);
  }
  __device__ half8 mins(uint32_t) const { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }
  __device__ void preload(const uint32_t *, uint32_t, uint32_t (&)[1]) const {}
  __device__ half8 step_pre(const uint32_t (&)[1], int, uint32_t, const uint32_t *) const { return half8{}; }
};

// Q6_K, 210 bytes: ql[128] | qh[64] | scales[16] (int8) | d
// (kernels.wgsl.js:269-330). Step s = weights 16 s .. 16 s + 15 of the block:
// n = s / 8, g = (s / 2) % 4, ql bytes 64 n + 32 (g % 2) + 16 (s % 2) + 8 h ..
// (nibble g / 2), qh bytes 128 + 32 n + 16 (s % 2) + 8 h .. (bits 2 g), scale
// s; w = d sc (q - 32). u = q - 32 is exact in fp16 but sc u need not be (up to
// 127 x 32), so each step is folded with its own d sc (FG = 1). Blocks start
// at 2-byte aligned offsets (`a`, 0 or 2, as IQ2_XXS).
template <> struct SxW<Q6_K> {
  static constexpr uint32_t BB = 210, DW = 53, ST = 53;
  static constexpr bool MINS = false;
  static constexpr int FG = 1;
  static constexpr int NP = 0;
  uint32_t a, sc[4];
  float d, dm;
  __device__ void block(const uint32_t *r, uint32_t off) {
    a = off;
    const uint32_t *p = r + ((off + 192u) >> 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = __builtin_amdgcn_alignbyte(p[i + 1], p[i], off);
    const uint32_t w = r[(off + 208u) >> 2];
    d = h2f(off ? (w >> 16) : (w & 0xFFFFu));
    dm = 0.f;
  }
  __device__ float scale(int g) const { return d * (float)(int8_t)byte_of(sc, (uint32_t)g); }
  __device__ half8 step(const uint32_t *r, int s, uint32_t h, const uint32_t *) const {
    const uint32_t n = (uint32_t)s >> 3, g = ((uint32_t)s >> 1) & 3u, o = 16u * ((uint32_t)s & 1u) + 8u * h;
    const uint32_t *pq = r + ((a + 64u * n + 32u * (g & 1u) + o) >> 2);
    const uint32_t *ph = r + ((a + 128u + 32u * n + o) >> 2);
    const uint32_t q0 = __builtin_amdgcn_alignbyte(pq[1], pq[0], a), q1 = __builtin_amdgcn_alignbyte(pq[2], pq[1], a);
    const uint32_t h0 = __builtin_amdgcn_alignbyte(ph[1], ph[0], a), h1 = __builtin_amdgcn_alignbyte(ph[2], ph[1], a);
    const uint32_t ls = 4u * (g >> 1), hs = 2u * g;
    const uint32_t u0 = ((q0 >> ls) & 0x0F0F0F0Fu) | (((h0 >> hs) & 0x03030303u) << 4);
    const uint32_t u1 = ((q1 >> ls) & 0x0F0F0F0Fu) | (((h1 >> hs) & 0x03030303u) << 4);
    // 1024 + q - 1056 = q - 32
    const half2v o2 = {(_Float16)-1056.f, (_Float16)-1056.f};
    const half2v e0 = h1024_lo(u0) + o2, e1 = h1024_hi(u0) + o2, e2 = h1024_lo(u1) + o2, e3 = h1024_hi(u1) + o2;
    return half8{e0.x, e0.y, e1.x, e1.y, e2.x, e2.y, e3.x, e3.y};
  }
  __device__ half8 mins(uint32_t) const { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }
  __device__ void preload(const uint32_t *, uint32_t, uint32_t (&)[1]) const {}
  __device__ half8 step_pre(const uint32_t (&)[1], int, uint32_t, const uint32_t *) const { return half8{}; }
};

constexpr uint32_t kSxTab = 6144;  // IQ2_XXS tables in LDS

template <int TYPE, int TT, int RF, int NW>
struct SxLds {
  using W = SxW<TYPE>;
  static constexpr uint32_t ROWS = 32u * RF;
  static constexpr uint32_t ND = (ROWS * W::ST + 63u) / 64u;  // staging loads per lane and block
  // stage bytes per wave, with 16 bytes of slack: the IQ2_XXS reader takes
  // one dword past a row (unused when the block is 4-byte aligned)
  static constexpr uint32_t SB = ND * 256u + 16u;
  static constexpr uint32_t NE = (uint32_t)TT * RF * 512u;     // sums per wave
  static constexpr uint32_t WORK = NW * SB > NW * NE * 4u ? NW * SB : NW * NE * 4u;
  static constexpr uint32_t TAB = TYPE == IQ2_XXS ? kSxTab : 0u;
  static constexpr uint32_t BYTES = TAB + WORK;
};

// FX: up to 8 tokens, x prepared by the product itself (sx_fill) from the
// f32 xf: per wave, block by block, x's rows go to LDS by direct-to-LDS loads
// issued before the block's weights, so that the preparation runs while the
// weights are in flight. LDS (dynamic): the tables and stages as without FX,
// then per wave sx_fx_bytes<TYPE>(): 8 x 1 KB of raw x, NS fragment slots of
// kSxFxSlot bytes, 16 scales.
template <int TYPE>
constexpr uint32_t sx_fx_bytes() {
  return 8u * 1024u + sx_slots<TYPE>() * kSxFxSlot + 64u;
}

template <int TYPE, int TT, int RF, int NW, bool FX>
__global__ __launch_bounds__(NW * 64) void k_sx(WeightView wv, const uint8_t *__restrict__ xa,
                                                const float *__restrict__ xp, float *__restrict__ y,
                                                uint32_t tokens, uint32_t nbw, uint32_t xa_bytes,
                                                const float *__restrict__ xf, uint32_t ksl,
                                                float *__restrict__ part, uint32_t *__restrict__ cnt) {
  using W = SxW<TYPE>;
  using L = SxLds<TYPE, TT, RF, NW>;
  static_assert(!FX || TT == 1, "the fused preparation covers one token tile");
  constexpr uint32_t NS = sx_slots<TYPE>();
  // steps of x fragments loaded ahead (Q4_K's 37-dword rows take 19 staging
  // offsets per lane: 3 steps ahead at 4 token tiles keep it within the VGPRs;
  // the types folded per group of steps hold more state: fewer steps ahead)
  constexpr bool MS = W::FG < 16;
  constexpr uint32_t P = TT == 1 ? 16u : TT == 2 ? (MS ? 4u : 8u) : TYPE == Q4_K ? 3u : MS ? 2u : 4u;
  constexpr uint32_t ROWS = L::ROWS, ND = L::ND;
  __shared__ __align__(16) uint8_t lds_s[FX ? 16u : L::BYTES];
  extern __shared__ __align__(16) uint8_t lds_d[];
  uint8_t *const lds = FX ? lds_d : lds_s;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, j = lane & 31u, h = lane >> 5;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // k slices: the ksl workgroups of a row tile (adjacent in x) take slices
  // of k, summed by the last of them to finish (ksl = 1: one workgroup)
  const uint32_t kh = blockIdx.x % ksl, rt = blockIdx.x / ksl;
  // nb: blocks of 256 weights per row (Q8_0 rows hold 8 of its 32-weight blocks in each)
  const uint32_t rows = wv.rows, nb = wv.k / 256u, r0 = rt * ROWS, tg = blockIdx.y;
  const uint32_t rb = (uint32_t)wv.row_bytes;
  uint32_t *tab = (uint32_t *)lds;
  uint8_t *stage = lds + L::TAB + wave * L::SB;

  if constexpr (TYPE == IQ2_XXS) {
    if (tid < 256u) {
      const uint64_t g = c_grid_sx[tid];
      const half8 v = dec_plain((uint32_t)g, (uint32_t)(g >> 32));
      *(half8 *)(tab + 4u * tid) = v;
    }
    if (tid < 128u) {
      const uint32_t s8 = tid | ((uint32_t)(__builtin_popcount(tid) & 1) << 7);
      u32x4 m;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        m[i] = (((s8 >> (2 * i)) & 1u) ? 0x8000u : 0u) | (((s8 >> (2 * i + 1)) & 1u) ? 0x80000000u : 0u);
      *(u32x4 *)(tab + 1024u + 4u * tid) = m;
    }
    __syncthreads();
  }

  // staging: dword q = 64 i + lane of the stage is dword q % ST of row q / ST
  // of the tile (the last dwords of a row and of the stage repeat valid ones);
  // Q8_0R: dwords 0..63 from the quant region (256 bytes further per block),
  // 64..67 from the scale region (16 bytes further per block)
  const rsrc_t wsrc = make_rsrc(wv.w, wv.w_bytes);
  uint32_t soff[ND], sadv[ND];
#pragma unroll
  for (uint32_t i = 0; i < ND; ++i) {
    const uint32_t q = 64u * i + lane, rr = q / W::ST, dw = min(q - rr * W::ST, W::DW - 1u);
    const uint32_t row = min(r0 + min(rr, ROWS - 1u), rows - 1u);
    if constexpr (TYPE == Q8_0R) {
      soff[i] = dw < 64u ? 32u * row * wv.bpr + 4u * dw : (uint32_t)wv.scales_off + 2u * row * wv.bpr + 4u * (dw - 64u);
      sadv[i] = dw < 64u ? 256u : 16u;
    } else {
      soff[i] = row * rb + 4u * dw;
      sadv[i] = 0u;
    }
  }
  const rsrc_t xsrc = make_rsrc(xa, xa_bytes);
  // FX: this wave's raw x, fragments and scales
  uint8_t *const xw = lds + L::TAB + L::WORK + wave * sx_fx_bytes<TYPE>();
  uint8_t *const xfr = xw + 8u * 1024u;
  float *const xps = (float *)(xfr + NS * kSxFxSlot);
  const rsrc_t fsrc = make_rsrc(xf, (uint64_t)tokens * wv.k * 4u);
  // the lane's fragment row: lanes of tokens 8..15 read the row of token
  // t - 8 (a D row depends only on its own A row, and those tokens' sums are
  // never written), so that every read is unmasked and can be issued early
  const uint32_t frow = 16u * (lane >> 5) + 8u * ((lane >> 4) & 1u) + (lane & 7u);
  if constexpr (FX) {
    // the rows of tokens past `tokens` and their scales stay zero
    for (uint32_t o = 16u * lane; o < NS * kSxFxSlot + 64u; o += 1024u) *(u32x4 *)(xfr + o) = u32x4{0u, 0u, 0u, 0u};
  }

  float acc[TT][RF][8];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int f = 0; f < RF; ++f)
#pragma unroll
      for (int v = 0; v < 8; ++v) acc[tt][f][v] = 0.f;

  const uint32_t bl = kh * nb / ksl, bh = (kh + 1u) * nb / ksl;
  const uint32_t b0 = bl + wave * nbw, b1 = min(b0 + nbw, bh);
  for (uint32_t bi = b0; bi < b1; ++bi) {
    // FX: the block's x, token by token, ahead of its weights
    if constexpr (FX)
      for (uint32_t t = 0; t < tokens; ++t) dma16(fsrc, xw + 1024u * t, 16u * lane, (t * wv.k + 256u * bi) * 4u);
    // this block of the tile's rows into the wave's stage
    const uint32_t bo = bi * W::BB;
#pragma unroll
    for (uint32_t i = 0; i < ND; ++i) {
      if constexpr (TYPE == Q8_0R)
        dma4(wsrc, stage + 256u * i, soff[i] + bi * sadv[i], 0u);
      else if constexpr ((W::BB & 3u) == 0u)
        dma4(wsrc, stage + 256u * i, soff[i], bo);
      else  // staged from the 4-byte aligned floor of the block's first byte
        dma4(wsrc, stage + 256u * i, (soff[i] + bo) & ~3u, 0u);
    }
    // x fragments of the first steps
    auto xoff = [&](uint32_t tt, uint32_t s) {
      return (((tg * TT + tt) * nb + bi) * NS + s) * 1024u;
    };
    u32x4 A[FX ? 1 : P][TT];
    half8 xfa[FX ? 16 : 1];   // FX: the block's 16 x fragments, read from LDS at once
    half8 am[TT];
    float4 pa[TT], pb[TT];
    if constexpr (FX) {
      // the raw x is in (its loads went out before the weights'); prepare it
      wait_vm<ND>();
      float4 v[8];
#pragma unroll
      for (uint32_t t = 0; t < 8u; ++t)
        v[t] = t < tokens ? *(const float4 *)(xw + 1024u * t + 16u * lane) : make_float4(0.f, 0.f, 0.f, 0.f);
      // all 8 rows every block (tokens past `tokens` read zeros and give zero rows)
      sx_fill8<TYPE>(v, lane, xfr, xps);
      am[0] = half8{0, 0, 0, 0, 0, 0, 0, 0};
      if constexpr (W::MINS) am[0] = *(const half8 *)(xfr + sx_fx_at(16u, frow));
      pa[0] = *(const float4 *)(xps + 4u * h);
      pb[0] = *(const float4 *)(xps + 8u + 4u * h);
#pragma unroll
      for (uint32_t st = 0; st < 16u; ++st) xfa[st] = *(const half8 *)(xfr + sx_fx_at(st, frow));
      wait_vm<0>();
    } else {
    // (each group of loads is followed by a compiler memory barrier, which
    // keeps it where it is: the compiler otherwise moves loads down to their
    // first use, and every step then waits a full round trip)
#pragma unroll
    for (uint32_t s = 0; s < P; ++s)
#pragma unroll
      for (uint32_t tt = 0; tt < (uint32_t)TT; ++tt)
        A[s][tt] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, (int)(16u * lane), (int)xoff(tt, s), 0);
    // the group sums and the tokens' block scales, for the fold (plain loads
    // for the scales: a 16-byte buffer load whose elements are taken one by
    // one as floats is narrowed to one dword by this compiler, every element
    // then reading the first)
#pragma unroll
    for (uint32_t tt = 0; tt < (uint32_t)TT; ++tt) {
      am[tt] = half8{0, 0, 0, 0, 0, 0, 0, 0};
      if constexpr (W::MINS)
        am[tt] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(xsrc, (int)(16u * lane), (int)xoff(tt, 16u), 0));
      const float *pp = xp + ((tg * TT + tt) * nb + bi) * 16u + 4u * h;
      pa[tt] = *(const float4 *)pp;
      pb[tt] = *(const float4 *)(pp + 8);
    }
    __asm__ volatile("" ::: "memory");
    wait_vm<P * TT + (W::MINS ? TT : 0) + 2 * TT>();
    }

    W w[RF];
    const uint32_t *rp[RF];
    // PRE: the weight dwords of all 16 steps in registers before the steps
    // (whose prefetch of x fragments keeps the compiler from hoisting LDS
    // reads); the 4-tile kernels have no registers to spare
    constexpr bool PRE = !FX && TT <= 2 && W::NP > 0;
    uint32_t pr[RF][PRE ? W::NP : 1];
#pragma unroll
    for (int f = 0; f < RF; ++f) {
      const uint32_t row = min(r0 + 32u * f + j, rows - 1u);
      const uint32_t a = (row * rb + bo) & 3u;
      rp[f] = (const uint32_t *)(stage + 4u * W::ST * (32u * f + j));
      w[f].block(rp[f], a);
      if constexpr (PRE) w[f].preload(rp[f], h, pr[f]);
    }
    // the tokens' block scales, for the folds
    float pv[TT][8];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      pv[tt][0] = pa[tt].x; pv[tt][1] = pa[tt].y; pv[tt][2] = pa[tt].z; pv[tt][3] = pa[tt].w;
      pv[tt][4] = pb[tt].x; pv[tt][5] = pb[tt].y; pv[tt][6] = pb[tt].z; pv[tt][7] = pb[tt].w;
    }
    float16v D[TT][RF];
#pragma unroll
    for (uint32_t s = 0; s < 16u; ++s) {
      half8 B[RF];
#pragma unroll
      for (int f = 0; f < RF; ++f) {
        if constexpr (PRE) B[f] = w[f].step_pre(pr[f], (int)s, h, tab);
        else B[f] = w[f].step(rp[f], (int)s, h, tab);
      }
      half8 a8[TT];
      if constexpr (FX) {
        a8[0] = xfa[s];
      } else {
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) a8[tt] = __builtin_bit_cast(half8, A[s % P][tt]);
        if (s + P < 16u) {
#pragma unroll
          for (uint32_t tt = 0; tt < (uint32_t)TT; ++tt)
            A[s % P][tt] = __builtin_amdgcn_raw_buffer_load_b128(xsrc, (int)(16u * lane), (int)xoff(tt, s + P), 0);
          __asm__ volatile("" ::: "memory");
        }
      }
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int f = 0; f < RF; ++f) {
          const float16v c = s % (uint32_t)W::FG == 0u ? float16v{} : D[tt][f];
          D[tt][f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8[tt], B[f], c, 0, 0, 0);
        }
      // types with several scales per block: the fold of each group of FG steps
      if constexpr (W::FG < 16) {
        if (s % (uint32_t)W::FG == (uint32_t)W::FG - 1u) {
#pragma unroll
          for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int f = 0; f < RF; ++f) {
              const float sc = w[f].scale((int)(s / (uint32_t)W::FG));
#pragma unroll
              for (int v = 0; v < 8; ++v)
                acc[tt][f][v] = __builtin_fmaf((D[tt][f][v] + D[tt][f][v + 8]) * sc, pv[tt][v], acc[tt][f][v]);
            }
        }
      }
    }
    // one scale per block: minimum sums, scales of the tokens, and the fold
    if constexpr (W::FG == 16) {
#pragma unroll
      for (uint32_t tt = 0; tt < (uint32_t)TT; ++tt) {
#pragma unroll
        for (int f = 0; f < RF; ++f) {
          float16v Dm{};
          if constexpr (W::MINS) Dm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[tt], w[f].mins(h), float16v{}, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 8; ++v) {
            float t = (D[tt][f][v] + D[tt][f][v + 8]) * w[f].d;
            if constexpr (W::MINS) t = __builtin_fmaf(-(Dm[v] + Dm[v + 8]), w[f].dm, t);
            acc[tt][f][v] = __builtin_fmaf(t, pv[tt][v], acc[tt][f][v]);
          }
        }
      }
    }
  }

  // the waves' sums, added in wave order
  __syncthreads();
  float *red = (float *)(lds + L::TAB);
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int f = 0; f < RF; ++f)
#pragma unroll
      for (int v = 0; v < 8; ++v) red[wave * L::NE + ((tt * RF + f) * 8u + v) * 64u + lane] = acc[tt][f][v];
  __syncthreads();
  constexpr uint32_t NT = NW * 64u, PE = L::NE / NT;   // sums per thread
  static_assert(L::NE % NT == 0u, "sums per thread");
  float sum[PE];
#pragma unroll
  for (uint32_t i = 0; i < PE; ++i) {
    sum[i] = 0.f;
#pragma unroll
    for (uint32_t w = 0; w < (uint32_t)NW; ++w) sum[i] += red[w * L::NE + tid + NT * i];
  }
  if (!FX && ksl > 1u) {
    // k slices: each workgroup of the tile stores its sums; the last of the
    // tile's ksl workgroups to arrive adds the slices in slice order, ((s0 +
    // s1) + s2) ..., which does not depend on the order of arrival, and
    // resets the tile's counter to zero for the next launch. The sums are
    // stored and loaded with the sc1 cache policy (as device-scope atomics
    // are), which the XCDs' L2 caches do not hold stale, and each wave waits
    // for its stores to complete before the barrier ahead of the counter's
    // increment (a fence would write back and invalidate the whole L2).
    constexpr int kSc1 = 16;   // cache policy bit 4: sc1
    __shared__ uint32_t arrived;
    const uint32_t lin = tg * (gridDim.x / ksl) + rt;
    const rsrc_t prs = make_rsrc(part + (uint64_t)lin * ksl * L::NE, (uint64_t)ksl * L::NE * 4u);
#pragma unroll
    for (uint32_t i = 0; i < PE; ++i)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sum[i]), prs, (int)((kh * L::NE + tid + NT * i) * 4u), 0,
                                            kSc1);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0u) arrived = __hip_atomic_fetch_add(cnt + lin, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != ksl - 1u) return;
    if (tid == 0u) __hip_atomic_store(cnt + lin, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (uint32_t i = 0; i < PE; ++i)
      sum[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(prs, (int)((tid + NT * i) * 4u), 0, kSc1));
    for (uint32_t zz = 1; zz < ksl; ++zz) {
#pragma unroll
      for (uint32_t i = 0; i < PE; ++i)
        sum[i] += __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(prs, (int)((zz * L::NE + tid + NT * i) * 4u), 0, kSc1));
    }
  }
#pragma unroll
  for (uint32_t i = 0; i < PE; ++i) {
    const uint32_t e = tid + NT * i;
    const uint32_t le = e & 63u, v = (e >> 6) & 7u, fr = e >> 9, f = fr % RF, tt = fr / RF;
    const uint32_t row = r0 + 32u * f + (le & 31u);
    const uint32_t tok = (tg * TT + tt) * 16u + 8u * (v >> 2) + 4u * (le >> 5) + (v & 3u);
    if (row < rows && tok < tokens) y[(uint64_t)tok * rows + row] = sum[i];
  }
}

// Token tiles of 16 per wave (tt) and token groups (grid y); the x scratch
// covers groups * tt tiles (tokens past `tokens` are zero).
struct SxPlan {
  // cfg 0: 32 rows x 8 waves; 1: 64 rows x 4 waves; ksl: k slices per row tile
  uint32_t tt, cfg, groups, row_tiles, nbw, ksl;
};

// The types folded per group of steps (Q8_0, Q8_0R, Q6_K) take at most 2
// token tiles per wave: with 4 their folds' state does not fit the registers.
uint32_t sx_tt_max(int type) { return type == Q8_0 || type == Q8_0R || type == Q6_K ? 2u : 4u; }

void sx_tiles(int type, uint32_t tokens, uint32_t &tt, uint32_t &groups) {
  const uint32_t ttn = (tokens + 15u) / 16u;
  tt = ttn <= 1u ? 1u : ttn <= 2u || sx_tt_max(type) == 2u ? 2u : 4u;
  groups = (ttn + tt - 1u) / tt;
}

SxPlan sx_plan(const WeightView &wv, uint32_t tokens, int cfg, uint32_t ksl_opt) {
  SxPlan p;
  sx_tiles(wv.type, tokens, p.tt, p.groups);
  // 32 rows x 8 waves, or 64 x 4 (the types of up to 4 token tiles, from 9
  // tokens) where its estimated time is lower: a CU takes ceil(w / 256)
  // workgroups of either kind, one of 64 x 4 costing 1.75 of one of 32 x 8
  // (the rows of two at a higher rate: 0.87-0.92 of the time where both fill
  // whole rounds), 40% more times the fraction of idle CUs below 256. On 9
  // shapes from 6144 x 4096 to 32768 x 2048, 9 to 384 tokens (Q2_K, Q4_K)
  // the choice is 0.1% above the faster of the two summed, the rule before
  // (64 x 4 only for 4 token tiles and 256 or from 512 of its workgroups)
  // 2.6%; us, before / now: 28672 x 4096 at 16 tokens Q4_K 38.0 / 30.2,
  // 14336 x 4096 at 128 69.6 / 60.2, 11008 x 4096 at 64 39.3 / 33.2, 10240
  // x 2048 at 192 40.0 / 36.4. IQ2_XXS weighs 64 x 4 at 1.9 (at one token
  // tile it was 5% slower at 11008 and 14336 rows, 1.2-1.4x faster from 32000);
  // Q4_K at 2 token tiles stays on 32 x 8 (64 x 4 7-10% slower at every
  // measured shape), and so does Q4_K at 8 or fewer tokens below k = 4096.
  // At 5-8 tokens Q2_K and IQ2_XXS take 64 x 4 by the same estimate (us, 5
  // tokens, the one-launch product before / now: Q2_K 65536 x 2048 49.2 /
  // 25.7, 32000 x 4096 41.5 / 26.1; IQ2_XXS 50.8 / 27.4, 42.0 / 26.7). Two k
  // slices over 64 x 4 were slower at every M.
  const uint32_t gr = p.groups, w32 = gr * ((wv.rows + 31u) / 32u), w64 = gr * ((wv.rows + 63u) / 64u);
  const double t32 = (double)((w32 + 255u) / 256u),
               t64 = (wv.type == IQ2_XXS ? 1.9 : 1.75) * (double)((w64 + 255u) / 256u) *
                     (1.0 + (w64 < 256u ? 0.4 * (1.0 - w64 / 256.0) : 0.0));
  const bool wide = sx_tt_max(wv.type) == 4u && (tokens > 8u || wv.type != Q4_K || wv.k >= 4096u) &&
                    !(wv.type == Q4_K && p.tt == 2u) && t64 < t32;
  // cfg 3 (forced): 64 x 4 in two k slices
  p.cfg = cfg ? (cfg == 3 ? 1u : (uint32_t)(cfg - 1)) : wide ? 1u : 0u;
  const uint32_t rows_per = p.cfg ? 64u : 32u, nw = p.cfg ? 4u : 8u, nb = wv.k / 256u;
  p.row_tiles = (wv.rows + rows_per - 1u) / rows_per;
  // Below 192 workgroups (few rows: 2048 rows are 64 tiles of 32), k slices
  // bring the grid to about 256, with 4 blocks of k per slice at least
  // (us, unsliced / 2 / 4 slices, 2048 x 8192 at 9 and 64 tokens: Q4_K 18.9 /
  // 13.9 / 11.5 and 38.6 / 24.3 / 18.5, Q8_0 23.9 / 17.2 / 13.6; 4096 x 14336
  // at 32 tokens, 128 workgroups: Q4_K 42.3 / 27.7 / 30.7, Q6_K 51.3 / 36.3 /
  // 40.4); from 256 workgroups none (Q4_K 2048 x 8192 at 512 tokens: 69.1 /
  // 74.0 / 85.7).
  const uint32_t wgs = p.row_tiles * p.groups;
  const uint32_t ks_auto = wgs < 192u ? min((256u + wgs / 2u) / wgs, max(nb / 4u, 1u)) : 1u;
  p.ksl = ksl_opt ? ksl_opt : cfg == 3 ? 2u : ks_auto;
  p.ksl = max(1u, min(p.ksl, nb));
  p.nbw = ((nb + p.ksl - 1u) / p.ksl + nw - 1u) / nw;
  return p;
}

template <int TYPE, int TT, int RF, int NW>
hipError_t sx_go(const WeightView &wv, const uint8_t *xa, const float *xp, float *y, uint32_t tokens,
                 const SxPlan &p, void *sk, hipStream_t s) {
  const uint64_t tiles = (uint64_t)p.groups * p.tt;
  const uint32_t xa_bytes = (uint32_t)(tiles * (wv.k / 256u) * sx_slots<TYPE>() * 1024u);
  if (p.ksl > 1u && (!sk || (uint64_t)p.row_tiles * p.groups > kSliceCntBytes / 4u)) return hipErrorInvalidValue;
  uint32_t *cnt = (uint32_t *)sk;
  float *part = sk ? (float *)((uint8_t *)sk + kSliceCntBytes) : nullptr;
  hipLaunchKernelGGL((k_sx<TYPE, TT, RF, NW, false>), dim3(p.row_tiles * p.ksl, p.groups), dim3(NW * 64), 0, s, wv,
                     xa, xp, y, tokens, p.nbw, xa_bytes, nullptr, p.ksl, part, cnt);
  return hipGetLastError();
}

// The product with its own preparation (up to 8 tokens, 32 rows x 8 waves).
template <int TYPE>
hipError_t sx_go_fx(const WeightView &wv, const float *x, float *y, uint32_t tokens, const SxPlan &p, hipStream_t s) {
  using L = SxLds<TYPE, 1, 1, 8>;
  constexpr uint32_t lds = L::TAB + L::WORK + 8u * sx_fx_bytes<TYPE>();
  static_assert(lds + 16u <= kMxMaxLds, "fused split-x LDS");
  static std::atomic<uint64_t> attr{0};
  const hipError_t e = lds_limit_once((const void *)k_sx<TYPE, 1, 1, 8, true>, (int)lds, attr);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_sx<TYPE, 1, 1, 8, true>), dim3(p.row_tiles, 1), dim3(8 * 64), lds, s, wv, nullptr, nullptr,
                     y, tokens, p.nbw, 0u, x, 1u, nullptr, nullptr);
  return hipGetLastError();
}

template <int TYPE, int TT>
hipError_t sx_cfg(const WeightView &wv, const uint8_t *xa, const float *xp, float *y, uint32_t tokens,
                  const SxPlan &p, void *sk, hipStream_t s) {
  if (p.cfg == 0u) return sx_go<TYPE, TT, 1, 8>(wv, xa, xp, y, tokens, p, sk, s);
  return sx_go<TYPE, TT, 2, 4>(wv, xa, xp, y, tokens, p, sk, s);
}

// Up to 8 tokens of Q2_K / IQ2_XXS with the automatic plan: one launch, each
// wave preparing its own block's x.
// The one-launch product repeats the preparation of x in every workgroup: it
// saves the preparation's launch where the workgroups times k stay within
// 256 x 2048 (us, 5 tokens, one launch against two: 8192 x 2048 Q2_K 7.8 /
// 8.6; 8192 x 8192 20.5 / 18.2, IQ2_XXS 21.6 / 18.1; 16384 x 2048 IQ2_XXS
// 14.3 / 12.5; 6144 x 4096 11.6 / 11.3).
bool sx_fx(int type, uint32_t tokens, int cfg, const SxPlan &p, uint32_t k) {
  return (type == Q2_K || type == IQ2_XXS) && cfg == 0 && tokens <= 8u && p.cfg == 0u && p.ksl == 1u &&
         (uint64_t)p.row_tiles * p.groups * k <= 256ull * 2048u;
}

// The product from x prepared in `xa` for `tiles` token tiles (at least the
// plan's; the tokens' block scales follow the fragments).
template <int TYPE>
hipError_t sx_main(const WeightView &wv, const uint8_t *xa, uint32_t tiles, float *y, uint32_t tokens,
                   const SxPlan &p, void *sk, hipStream_t s) {
  const float *xp = (const float *)(xa + (uint64_t)tiles * (wv.k / 256u) * sx_slots<TYPE>() * 1024u);
  switch (p.tt) {
    case 1: return sx_cfg<TYPE, 1>(wv, xa, xp, y, tokens, p, sk, s);
    case 2: return sx_cfg<TYPE, 2>(wv, xa, xp, y, tokens, p, sk, s);
    default:
      if constexpr (SxW<TYPE>::FG == 16) return sx_cfg<TYPE, 4>(wv, xa, xp, y, tokens, p, sk, s);
      return hipErrorInvalidValue;   // not planned (sx_tt_max)
  }
}

template <int TYPE>
hipError_t sx_type(const WeightView &wv, const float *x, float *y, uint32_t tokens, uint8_t *scratch, int cfg,
                   uint32_t ksl_opt, void *sk, hipStream_t s) {
  const SxPlan p = sx_plan(wv, tokens, cfg, ksl_opt);
  if constexpr (TYPE == Q2_K || TYPE == IQ2_XXS)
    if (sx_fx(TYPE, tokens, cfg, p, wv.k)) return sx_go_fx<TYPE>(wv, x, y, tokens, p, s);
  const uint32_t tiles = p.groups * p.tt, nb = wv.k / 256u;   // blocks of 256 weights
  uint8_t *xa = scratch;
  float *xp = (float *)(scratch + (uint64_t)tiles * nb * sx_slots<TYPE>() * 1024u);
  hipLaunchKernelGGL((k_sx_prep<TYPE>), dim3(nb, tiles * 4u), dim3(256), 0, s, x, tokens, wv.k, xa, xp);
  return sx_main<TYPE>(wv, xa, tiles, y, tokens, p, sk, s);
}

// Token tiles of a prepared x: a multiple of 4 (the most a plan groups), so
// that the plan of every type of the layout reads inside it.
uint32_t sx_prepared_tiles(uint32_t tokens) { return (tokens + 63u) / 64u * 4u; }

}  // namespace

bool sx_applies(const WeightView &wv, uint32_t tokens) {
  const bool t = wv.type == Q2_K || wv.type == Q4_K || wv.type == IQ2_XXS || wv.type == Q8_0 || wv.type == Q8_0R ||
                 wv.type == Q6_K;
  // Q8_0R is staged with 32-bit offsets from the tensor's first byte
  const bool r = wv.type != Q8_0R || wv.scales_off + 2ull * wv.rows * wv.bpr + 16u < (1ull << 32);
  return t && r && tokens >= 2u && wv.k % 256u == 0u;
}

size_t sx_x_bytes(int type, uint32_t tokens, uint32_t k) {
  uint32_t tt, groups;
  sx_tiles(type, tokens, tt, groups);
  const uint64_t tiles = (uint64_t)tt * groups, nb = k / 256u;
  const uint32_t slots = type == Q2_K || type == Q4_K ? 17u : 16u;   // sx_slots
  return (size_t)(tiles * nb * slots * 1024u + tiles * nb * 64u);
}

size_t sx_sk_bytes(const WeightView &wv, uint32_t tokens, int cfg, uint32_t ksl_opt) {
  const SxPlan p = sx_plan(wv, tokens, cfg, ksl_opt);
  if (p.ksl < 2u || sx_fx(wv.type, tokens, cfg, p, wv.k)) return 0;
  const uint64_t ne = (uint64_t)p.tt * (p.cfg ? 2u : 1u) * 512u;   // sums per workgroup
  return kSliceCntBytes + (size_t)((uint64_t)p.row_tiles * p.groups * p.ksl * ne * 4u);
}

uint32_t sx_x_layout(const WeightView &wv, uint32_t tokens, int cfg, uint32_t ksl_opt) {
  const SxPlan p = sx_plan(wv, tokens, cfg, ksl_opt);
  if (sx_fx(wv.type, tokens, cfg, p, wv.k)) return 0u;
  switch (wv.type) {
    case Q2_K: return kSxLayout | 1u;
    case Q4_K: return kSxLayout | 2u;
    default: return kSxLayout;
  }
}

size_t sx_prepared_bytes(uint32_t layout, uint32_t tokens, uint32_t k) {
  const uint64_t tiles = sx_prepared_tiles(tokens), nb = k / 256u;
  const uint32_t slots = layout == kSxLayout ? 16u : 17u;   // sx_slots
  return (size_t)(tiles * nb * slots * 1024u + tiles * nb * 64u);
}

hipError_t launch_sx_prepare(uint32_t layout, const float *x, uint32_t tokens, uint32_t k, void *xprep,
                             hipStream_t s) {
  const uint32_t tiles = sx_prepared_tiles(tokens), nb = k / 256u;
  uint8_t *xa = (uint8_t *)xprep;
  const uint32_t slots = layout == kSxLayout ? 16u : 17u;
  float *xp = (float *)(xa + (uint64_t)tiles * nb * slots * 1024u);
  // the layouts differ only in the group sums: IQ2_XXS, Q8_0 and Q6_K read
  // the same 16 slots
  switch (layout) {
    case kSxLayout | 1u:
      hipLaunchKernelGGL((k_sx_prep<Q2_K>), dim3(nb, tiles * 4u), dim3(256), 0, s, x, tokens, k, xa, xp);
      break;
    case kSxLayout | 2u:
      hipLaunchKernelGGL((k_sx_prep<Q4_K>), dim3(nb, tiles * 4u), dim3(256), 0, s, x, tokens, k, xa, xp);
      break;
    case kSxLayout:
      hipLaunchKernelGGL((k_sx_prep<IQ2_XXS>), dim3(nb, tiles * 4u), dim3(256), 0, s, x, tokens, k, xa, xp);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_sx_prepared(const WeightView &wv, const void *xprep, float *y, uint32_t tokens, int cfg,
                              uint32_t ksl_opt, void *sk, hipStream_t s) {
  const SxPlan p = sx_plan(wv, tokens, cfg, ksl_opt);
  const uint8_t *xa = (const uint8_t *)xprep;
  const uint32_t tiles = sx_prepared_tiles(tokens);
  switch (wv.type) {
    case Q2_K: return sx_main<Q2_K>(wv, xa, tiles, y, tokens, p, sk, s);
    case Q4_K: return sx_main<Q4_K>(wv, xa, tiles, y, tokens, p, sk, s);
    case IQ2_XXS: return sx_main<IQ2_XXS>(wv, xa, tiles, y, tokens, p, sk, s);
    case Q8_0: return sx_main<Q8_0>(wv, xa, tiles, y, tokens, p, sk, s);
    case Q8_0R: return sx_main<Q8_0R>(wv, xa, tiles, y, tokens, p, sk, s);
    case Q6_K: return sx_main<Q6_K>(wv, xa, tiles, y, tokens, p, sk, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_sx(const WeightView &wv, const float *x, float *y, uint32_t tokens, void *scratch, int cfg,
                     uint32_t ksl_opt, void *sk, hipStream_t s) {
  uint8_t *sc = (uint8_t *)scratch;
  switch (wv.type) {
    case Q2_K: return sx_type<Q2_K>(wv, x, y, tokens, sc, cfg, ksl_opt, sk, s);
    case Q4_K: return sx_type<Q4_K>(wv, x, y, tokens, sc, cfg, ksl_opt, sk, s);
    case IQ2_XXS: return sx_type<IQ2_XXS>(wv, x, y, tokens, sc, cfg, ksl_opt, sk, s);
    case Q8_0: return sx_type<Q8_0>(wv, x, y, tokens, sc, cfg, ksl_opt, sk, s);
    case Q8_0R: return sx_type<Q8_0R>(wv, x, y, tokens, sc, cfg, ksl_opt, sk, s);
    case Q6_K: return sx_type<Q6_K>(wv, x, y, tokens, sc, cfg, ksl_opt, sk, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace eff
