// Block geometry and scalar conversions shared by the host and device code.
//
// Block layouts are the GGUF ones, as read by the reference decoders
// (kernels.wgsl.js:154-396) and sized by gguf.js:51-64:
//   Q8_0    32 weights,  34 B: f16 d | int8 q[32]
//   Q2_K   256 weights,  84 B: u8 scales[16] (sc | m<<4) | qs[64] | f16 d | f16 dmin
//   Q4_K   256 weights, 144 B: f16 d | f16 dmin | scales[12] (6-bit packed) | qs[128]
//   Q6_K   256 weights, 210 B: ql[128] | qh[64] | int8 scales[16] | f16 d
//   IQ2_XXS 256 weights, 66 B: f16 d | 8 x (u32 grid indices, u32 signs+scale)
//   Q8_0R  the Q8_0 bytes repacked: 32-byte quants of every block first, then
//          the f16 scales from byte 32N (kernels.bloques.wgsl.js:19-35).
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define EFF_HD __host__ __device__ __forceinline__
#else
#define EFF_HD static inline
#endif

namespace eff {

enum Type : int {
  Q8_0 = 8,
  Q2_K = 10,
  Q4_K = 12,
  Q6_K = 14,
  IQ2_XXS = 16,
  Q8_0R = 264,
};

struct Geometry {
  uint32_t elems;
  uint32_t bytes;
};

EFF_HD bool type_known(int t) {
  return t == Q8_0 || t == Q2_K || t == Q4_K || t == Q6_K || t == IQ2_XXS || t == Q8_0R;
}

EFF_HD Geometry geometry(int t) {
  switch (t) {
    case Q8_0:
    case Q8_0R: return {32u, 34u};
    case Q2_K: return {256u, 84u};
    case Q4_K: return {256u, 144u};
    case Q6_K: return {256u, 210u};
    case IQ2_XXS: return {256u, 66u};
    default: return {0u, 0u};
  }
}

// IEEE binary16 -> binary32, exact (subnormals, inf, NaN kept).
EFF_HD float half_to_float(uint32_t h) {
  uint32_t sign = (h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      // Normalise the subnormal: value = man * 2^-24.
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | (uint32_t)(127 - 15 - e) << 23 | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// binary32 -> binary16 with round-to-nearest-even (overflow to inf, NaN kept quiet).
EFF_HD uint32_t float_to_half_rne(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) return sign | 0x7C00u | (man ? 0x200u : 0u);
  int e = (int)exp - 127 + 15;
  if (e >= 31) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;  // below half the smallest subnormal: rounds to zero
    uint32_t m = man | 0x800000u;
    int shift = 14 - e;        // keep 24 - shift bits
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
    return sign | q;           // a carry into bit 10 gives the smallest normal, correctly
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // carry may round up to inf
  return h;
}

}  // namespace eff
