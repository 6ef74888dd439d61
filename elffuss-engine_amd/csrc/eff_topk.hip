// Exact top-m (m <= 192) of one logits vector, ordered by (f32 value desc
// with -0 == +0, index asc), and the raw logits of the penalised ids, written
// as the reference's output record (kernels.topk.wgsl.js:40-60,
// ops.topk.js:99-165; the order of sample.js:44-67).
//
// Composites, records, the wave helpers and the selection itself
// (topk_pick) are in eff_topk.h, shared with the row GEMV whose last
// workgroup runs the selection over the records it wrote.
//
// Two launches:
//  * k_topk_groups: the vector is cut into G <= 256 groups of
//    gs = 256 ceil(vocab / 65536) consecutive logits, one 64-lane wave per
//    group; the wave writes the group's 4 largest composites and their bits.
//  * k_topk_pick: one workgroup of 256 threads (a wave per SIMD) runs
//    topk_pick over the G records.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_kernels.h"
#include "eff_topk.h"

namespace eff {

namespace {

// Record of group g (kTopkRecordBytes = 64; eff_topk.h): u64 c[4] (0 past the
// group's elements), u32 bits[4], u32 nan flag, 12 bytes unused; c[0] also in
// the maxima array after the gridDim.x records.
__global__ __launch_bounds__(64) void k_topk_groups(const uint32_t *__restrict__ logits, uint32_t vocab,
                                                    uint32_t per, uint8_t *__restrict__ rec) {
  const uint32_t lane = threadIdx.x;
  const uint32_t g = blockIdx.x;
  const uint32_t e0 = g * 64u * per;
  Top4 t;
  bool nan = false;
  for (uint32_t j0 = 0; j0 < per; j0 += 4u) {
    uint32_t bits[4];
    // the loads of four steps first, then their keys
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t e = e0 + 64u * (j0 + (uint32_t)q) + lane;
      bits[q] = (j0 + (uint32_t)q < per && e < vocab) ? logits[e] : 0u;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t e = e0 + 64u * (j0 + (uint32_t)q) + lane;
      if (j0 + (uint32_t)q < per && e < vocab) {
        nan |= is_nan_bits(bits[q]);
        t.add(composite(bits[q], e), bits[q]);
      }
    }
  }
  topk_record_wave(t, nan, rec, g, gridDim.x);
}

constexpr int kPickThreads = 256;

// One record per thread (groups <= 256).
__global__ __launch_bounds__(kPickThreads) void k_topk_pick(const uint32_t *__restrict__ logits, uint32_t vocab,
                                                            uint32_t m, TopkPenal penal, uint32_t n_penal,
                                                            uint32_t serial, uint32_t gs, uint32_t groups,
                                                            const uint8_t *__restrict__ rec,
                                                            uint32_t *__restrict__ out) {
  __shared__ PickLds<kPickThreads, 1> sh;
  topk_pick<kPickThreads, 1>(logits, vocab, m, penal, n_penal, serial, FlatGroups{gs}, groups, rec, out, sh);
}

// The selecting half alone, over `groups` (<= 256) records of groups of `gs`
// consecutive logits.
hipError_t launch_topk_pick(const uint32_t *logits, uint32_t vocab, uint32_t m, const uint32_t *penal_ids,
                            uint32_t n_penal, uint32_t serial, uint32_t gs, uint32_t groups, const uint8_t *rec,
                            uint32_t *out, hipStream_t s) {
  if (groups == 0 || groups > (uint32_t)kPickThreads || (uint64_t)groups * gs < vocab) return hipErrorInvalidValue;
  TopkPenal pen{};
  for (uint32_t i = 0; i < n_penal; ++i) pen.ids[i] = penal_ids[i];
  hipLaunchKernelGGL(k_topk_pick, dim3(1), dim3(kPickThreads), 0, s, logits, vocab, m, pen, n_penal, serial, gs,
                     groups, rec, out);
  return hipGetLastError();
}

}  // namespace

size_t topk_scratch_bytes(uint32_t vocab) { return topk_scratch_bytes_for(vocab); }

hipError_t launch_topk(const uint32_t *logits, uint32_t base, uint32_t vocab, uint32_t m,
                       const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, uint32_t *scratch,
                       uint32_t *out, hipStream_t s) {
  if (vocab == 0 || vocab >= EFF_TOPK_N_MAX || m == 0 || m > EFF_TOPK_M_MAX || n_penal > EFF_TOPK_P_MAX)
    return hipErrorInvalidValue;
  const uint32_t gs = topk_group_size(vocab), groups = topk_groups(vocab);
  if (groups > kTopkGroupsMax) return hipErrorInvalidValue;
  const uint32_t *lg = logits + base;
  hipLaunchKernelGGL(k_topk_groups, dim3(groups), dim3(64), 0, s, lg, vocab, gs / 64u, (uint8_t *)scratch);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_topk_pick(lg, vocab, m, penal_ids, n_penal, serial, gs, groups, (const uint8_t *)scratch, out, s);
}

}  // namespace eff
