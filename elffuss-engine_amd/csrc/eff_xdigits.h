// x as three signed 8-bit digit planes per group of 32 values, prepared in
// LDS by the GEMV kernels (eff_gemv_mx.hip, eff_gemv_rows.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eff {

// x -> digit planes. One thread per 8 consecutive values ("octet"); the 4
// threads of a quad cover one 32-value group. LDS per token: digits
// [k/16][plane][16 B] (3 B per value), then per 32-value group
// {p, sum x[0..15], sum x[16..31], -}.
//
// Vector loads return in issue order, so the first kXr octets of every thread
// are loaded before the weights and converted while the weights are in
// flight; any further octets are loaded and converted afterwards.
constexpr uint32_t kXr = 4;

struct XOct {
  float4 a, b;
};

// Token t and k offset ko of octet o, for at most TMAX tokens (compares
// instead of a division by k / 8).
template <uint32_t TMAX>
__device__ __forceinline__ void oct_pos(uint32_t k, uint32_t o, uint32_t &t, uint32_t &ko) {
  const uint32_t opt = k / 8u;
  uint32_t n = 0;
#pragma unroll
  for (uint32_t i = 1; i < TMAX; ++i) n += o >= i * opt ? 1u : 0u;
  t = n;
  ko = 8u * (o - n * opt);
}

template <uint32_t TMAX>
__device__ __forceinline__ void x_load(const float *__restrict__ x, uint32_t k, uint32_t o, XOct &v) {
  uint32_t t, ko;
  oct_pos<TMAX>(k, o, t, ko);
  v.a = *(const float4 *)(x + (uint64_t)t * k + ko);
  v.b = *(const float4 *)(x + (uint64_t)t * k + ko + 4u);
}

// dstride: bytes of digits per token (3 k, or padded); mstride: floats of
// group data per token (k / 8, or padded); meta: the group data area.
template <uint32_t TMAX>
__device__ __forceinline__ void x_store(const XOct &v, uint32_t k, uint32_t o, uint8_t *lds, uint32_t dstride,
                                        float *metab, uint32_t mstride) {
  uint32_t t, ko;
  oct_pos<TMAX>(k, o, t, ko);
  const float4 a = v.a, b = v.b;
  float m = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                  fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
  // the quad's maximum (quad_perm [1,0,3,2] then [2,3,0,1])
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, m), 0xB1, 0xF, 0xF, false)));
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, m), 0x4E, 0xF, 0xF, false)));
  // max < 2^E with E = e - 126 (e = biased exponent of m, at least 21 so that
  // p stays a normal number); a group holding an infinity gets p = NaN (a NaN
  // reaches the result through the group sums).
  const uint32_t eb = (__builtin_bit_cast(uint32_t, m) >> 23) & 0xFFu;
  const uint32_t e = eb < 21u ? 21u : (eb > 254u ? 254u : eb);
  const float scale = __builtin_bit_cast(float, (274u - e) << 23);  // 2^(21 - E)
  const float p = eb == 255u ? __builtin_bit_cast(float, 0x7FC00000u) : __builtin_bit_cast(float, (e - 20u) << 23);
  // round(x * scale) + 0x808080 through the f32 magic 1.5 * 2^23: the three
  // low bytes are the digits + 128
  const float v8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t e8[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    e8[i] = __builtin_bit_cast(uint32_t, __builtin_fmaf(v8[i], scale, 12582912.0f)) - 0x4ABF7F80u;
  uint32_t pl[3][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t *q = e8 + 4 * h;
    const uint32_t l01 = __builtin_amdgcn_perm(q[1], q[0], 0x05010400u);  // e0.b0 e1.b0 e0.b1 e1.b1
    const uint32_t l23 = __builtin_amdgcn_perm(q[3], q[2], 0x05010400u);
    const uint32_t h01 = __builtin_amdgcn_perm(q[1], q[0], 0x07030602u);  // e0.b2 e1.b2 e0.b3 e1.b3
    const uint32_t h23 = __builtin_amdgcn_perm(q[3], q[2], 0x07030602u);
    pl[0][h] = __builtin_amdgcn_perm(l23, l01, 0x05040100u) ^ 0x80808080u;
    pl[1][h] = __builtin_amdgcn_perm(l23, l01, 0x07060302u) ^ 0x80808080u;
    pl[2][h] = __builtin_amdgcn_perm(h23, h01, 0x05040100u) ^ 0x80808080u;
  }
  uint8_t *dig = lds + (uint64_t)t * dstride + (ko / 16u) * 48u + 8u * ((ko / 8u) & 1u);
#pragma unroll
  for (int d = 0; d < 3; ++d) *(uint2 *)(dig + 16 * d) = make_uint2(pl[d][0], pl[d][1]);
  // sums over 16 values: this octet + its neighbour in the quad
  float s = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
  s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0xB1, 0xF, 0xF, false));
  float *meta = metab + (uint64_t)t * mstride + 4u * (ko / 32u);
  const uint32_t q4 = (ko / 8u) & 3u;
  if (q4 == 0u) meta[1] = s;
  if (q4 == 2u) meta[2] = s;
  if (q4 == 1u) meta[0] = p;
}

// As x_store for one token, with the group data the row GEMV uses
// (eff_gemv_rows.hip): per 32-value group 8 words {-32 T0, -32 T1, -32 T2, p}
// for values 0..15 and {-32 T0, -32 T1, -32 T2, 0} for values 16..31, where
// T_d is the sum of digit plane d over the 16 values. With weights u in 0..63
// stored for u - 32, sum (u - 32) x~ = p sum_d 256^d (sum u digit_d - 32 T_d),
// and -32 T_d starts the integer sums. Digits at lds (3 k bytes, the layout of
// x_store), group data at meta (k bytes).
__device__ __forceinline__ void x_store_tsum(const XOct &v, uint32_t o, uint8_t *lds, int32_t *meta) {
  const uint32_t ko = 8u * o;
  const float4 a = v.a, b = v.b;
  // the group's largest |x| bit pattern: as unsigned integers NaN > inf > any
  // finite value, so a NaN (which the group sums of x_store carry) also gives
  // eb = 255 and p = NaN here
  const float v8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t mb = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) mb = max(mb, __builtin_bit_cast(uint32_t, v8[i]) & 0x7FFFFFFFu);
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));
  // the exponent rule and digit rounding of x_store
  const uint32_t eb = (mb >> 23) & 0xFFu;
  const uint32_t e = eb < 21u ? 21u : (eb > 254u ? 254u : eb);
  const float scale = __builtin_bit_cast(float, (274u - e) << 23);  // 2^(21 - E)
  const float p = eb == 255u ? __builtin_bit_cast(float, 0x7FC00000u) : __builtin_bit_cast(float, (e - 20u) << 23);
  uint32_t e8[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    e8[i] = __builtin_bit_cast(uint32_t, __builtin_fmaf(v8[i], scale, 12582912.0f)) - 0x4ABF7F80u;
  uint32_t pl[3][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t *q = e8 + 4 * h;
    const uint32_t l01 = __builtin_amdgcn_perm(q[1], q[0], 0x05010400u);
    const uint32_t l23 = __builtin_amdgcn_perm(q[3], q[2], 0x05010400u);
    const uint32_t h01 = __builtin_amdgcn_perm(q[1], q[0], 0x07030602u);
    const uint32_t h23 = __builtin_amdgcn_perm(q[3], q[2], 0x07030602u);
    pl[0][h] = __builtin_amdgcn_perm(l23, l01, 0x05040100u) ^ 0x80808080u;
    pl[1][h] = __builtin_amdgcn_perm(l23, l01, 0x07060302u) ^ 0x80808080u;
    pl[2][h] = __builtin_amdgcn_perm(h23, h01, 0x05040100u) ^ 0x80808080u;
  }
  uint8_t *dig = lds + (ko / 16u) * 48u + 8u * ((ko / 8u) & 1u);
#pragma unroll
  for (int d = 0; d < 3; ++d) *(uint2 *)(dig + 16 * d) = make_uint2(pl[d][0], pl[d][1]);
  // digit sums over 16 values: this octet + its neighbour in the quad
  int ts[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    int t = __builtin_amdgcn_sdot4((int)pl[d][0], 0x01010101, 0, false);
    t = __builtin_amdgcn_sdot4((int)pl[d][1], 0x01010101, t, false);
    ts[d] = t + __builtin_amdgcn_update_dpp(0, t, 0xB1, 0xF, 0xF, false);
  }
  int32_t *mg = meta + 8u * (ko / 32u);
  const uint32_t q4 = (ko / 8u) & 3u;
  if ((q4 & 1u) == 0u) {
    int32_t *mt = mg + 2u * q4;   // words 0..2 (values 0..15) or 4..6 (values 16..31)
    mt[0] = -32 * ts[0];
    mt[1] = -32 * ts[1];
    mt[2] = -32 * ts[2];
  } else {
    mg[2u * q4 + 1u] = q4 == 1u ? __builtin_bit_cast(int32_t, p) : 0;   // word 3 or 7
  }
}

}  // namespace eff
