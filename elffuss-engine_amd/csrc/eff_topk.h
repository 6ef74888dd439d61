// Device helpers of the exact top-k (eff_topk.hip) shared with the kernels
// that write its per-group records themselves (eff_gemv_rows.hip).
//
// Elements are compared by the 64-bit composite (order_key(bits) << 32 |
// ~index): unique per element, larger composite = larger value, ties to the
// lower index. order_key maps f32 order to u32 order with -0 = +0
// (kernels.topk.wgsl.js:75-82). A valid element's composite is never 0
// (~index has its top 8 bits set for index < 2^24), so 0 marks "none".
//
// Record of a group of consecutive logits (kTopkRecordBytes = 64): u64 c[4]
// (its 4 largest composites, descending, 0 past the group's elements), u32
// bits[4] (their raw logits), u32 nan flag (1 when the group holds a NaN),
// 12 bytes unused.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "eff_kernels.h"

namespace eff {

__device__ __forceinline__ uint32_t order_key(uint32_t bits) {
  const uint32_t b = bits == 0x80000000u ? 0u : bits;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ bool is_nan_bits(uint32_t bits) { return (bits & 0x7FFFFFFFu) > 0x7F800000u; }

__device__ __forceinline__ uint64_t composite(uint32_t bits, uint32_t idx) {
  return ((uint64_t)order_key(bits) << 32) | (uint64_t)(~idx);
}


// Sorted insertion into a lane's 4 largest (c0 > c1 > c2 > c3).
struct Top4 {
  uint64_t c[4] = {0, 0, 0, 0};
  uint32_t b[4] = {0, 0, 0, 0};
  __device__ __forceinline__ void add(uint64_t v, uint32_t bits) {
    if (v <= c[3]) return;
    c[3] = v;
    b[3] = bits;
#pragma unroll
    for (int i = 3; i > 0; --i) {
      if (c[i] > c[i - 1]) {
        const uint64_t t = c[i];
        c[i] = c[i - 1];
        c[i - 1] = t;
        const uint32_t u = b[i];
        b[i] = b[i - 1];
        b[i - 1] = u;
      }
    }
  }
};

// Wave-wide maximum / minimum of a u32 (every lane active): DPP within rows
// of 16 (quad xor 1, quad xor 2, half-row mirror, row mirror), then the four
// rows through scalar reads. The result is wave-uniform.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext(uint32_t v) {
  auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return op(op(r0, r1), op(r2, r3));
}

// Wave-wide maximum / minimum of a u64, as its high word then the low word
// among the lanes holding that high word.
template <bool MAX>
__device__ __forceinline__ uint64_t wave_ext64(uint64_t v) {
  const uint32_t h = wave_ext<MAX>((uint32_t)(v >> 32));
  const uint32_t l = wave_ext<MAX>((uint32_t)(v >> 32) == h ? (uint32_t)v : (MAX ? 0u : 0xFFFFFFFFu));
  return ((uint64_t)h << 32) | l;
}

// The group's record from the lanes' own 4 largest (every lane of the wave
// active): 4 rounds of a wave maximum over the lanes' heads; lanes 0..3 write
// the 64 bytes at `rec`.
__device__ __forceinline__ void topk_record_wave(Top4 t, bool nan, uint8_t *rec) {
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t out_c[4];
  uint32_t out_b[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t mx = wave_ext64<true>(t.c[0]);
    const bool mine = mx != 0u && t.c[0] == mx;
    const uint64_t win = __ballot(mine);
    const int src = win ? (int)__builtin_ctzll(win) : 0;
    out_c[r] = mx;
    out_b[r] = mx ? (uint32_t)__builtin_amdgcn_readlane((int)t.b[0], src) : 0u;
    if (mine) {  // the winning lane pops its head
      t.c[0] = t.c[1]; t.b[0] = t.b[1];
      t.c[1] = t.c[2]; t.b[1] = t.b[2];
      t.c[2] = t.c[3]; t.b[2] = t.b[3];
      t.c[3] = 0u; t.b[3] = 0u;
    }
  }
  const bool any_nan = __ballot(nan) != 0u;
  if (lane < 4u) {
    uint4 v;
    if (lane < 2u) {
      const uint64_t a = out_c[2 * lane], b = out_c[2 * lane + 1];
      v = make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
    } else if (lane == 2u) {
      v = make_uint4(out_b[0], out_b[1], out_b[2], out_b[3]);
    } else {
      v = make_uint4(any_nan ? 1u : 0u, 0u, 0u, 0u);
    }
    ((uint4 *)rec)[lane] = v;
  }
}

}  // namespace eff
