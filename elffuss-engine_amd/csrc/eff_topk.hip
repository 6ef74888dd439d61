// Exact top-m (m <= 192) of one logits vector, ordered by (f32 value desc
// with -0 == +0, index asc), and the raw logits of the penalised ids, written
// as the reference's output record (kernels.topk.wgsl.js:40-60,
// ops.topk.js:99-165; the order of sample.js:44-67).
//
// Composites, records and the wave helpers are in eff_topk.h.
//
// Two launches:
//  * k_topk_groups: the vector is cut into G <= 256 groups of
//    gs = 256 ceil(vocab / 65536) consecutive logits, one 64-lane wave per
//    group; the wave writes the group's 4 largest composites and their bits.
//  * k_topk_pick: one workgroup of 256 threads (a wave per SIMD), thread t
//    holding group t's record. tau = the m-th largest group maximum: each of
//    the m largest elements is >= tau, and only the m groups whose maximum is
//    >= tau list composites >= tau, so the m largest of the listed
//    composites >= tau (ranked by counting) are the answer, unless some group
//    has more than 4 elements and its 4th listed composite is among them
//    ("saturated"): an element a group does not list is below its 4th, and
//    if that 4th is not selected, m listed composites beat it. Otherwise the
//    select runs again over the unsaturated groups' lists plus every element
//    of the saturated groups, read from memory. The m winners are written
//    sorted by (value desc, index asc).
// Selections are radix selects whose 8-bit digit window sits at the highest
// bit where the smallest and largest candidate still in play differ, so the
// histogram's bins spread the candidates.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_kernels.h"
#include "eff_topk.h"

namespace eff {

namespace {

struct TopkPenal {
  uint32_t ids[EFF_TOPK_P_MAX];
};

// Record of a group (kTopkRecordBytes = 64): u64 c[4] (0 past the group's
// elements), u32 bits[4], u32 nan flag, 12 bytes unused.
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
  topk_record_wave(t, nan, rec + (uint64_t)g * kTopkRecordBytes);
}

constexpr int kPickThreads = 256;
constexpr int kPickWaves = kPickThreads / 64;
constexpr uint32_t kCandMax = 4u * EFF_TOPK_M_MAX;   // listed composites >= tau at most

// Inclusive prefix sum over the 64 lanes of a wave (every lane active): DPP
// shifts within rows of 16, then the row totals broadcast to the rows above.
__device__ __forceinline__ uint32_t wave_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);   // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);   // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

struct PickShared {
  uint32_t hist[256];   // bin 255 - d counts digit d (descending digits in ascending bins)
  uint32_t st[4];
  uint64_t wmin[kPickWaves], wmax[kPickWaves];
};

// Radix select over distinct 64-bit candidates: returns T such that exactly
// `need` candidates are >= T (1 <= need <= number of candidates). Each round
// finds the smallest and largest candidate still in play, places an 8-bit
// digit window at their highest differing bit, and keeps the bin that holds
// the need-th largest. `visit(f)` calls f(c) for each candidate the calling
// thread holds. Every thread of the workgroup calls it.
template <class Visit>
__device__ uint64_t select_top(uint32_t need, Visit visit, PickShared &sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t lo = 0, hi = ~(uint64_t)0;
  uint32_t rem = need;
  for (int round = 0; round < 16; ++round) {
    uint64_t mn = ~(uint64_t)0, mx = 0;
    visit([&](uint64_t c) {
      if (c >= lo && c <= hi) {
        mn = c < mn ? c : mn;
        mx = c > mx ? c : mx;
      }
    });
    mn = wave_ext64<false>(mn);
    mx = wave_ext64<true>(mx);
    if (lane == 0) {
      sh.wmin[wave] = mn;
      sh.wmax[wave] = mx;
    }
    sh.hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kPickWaves; ++w) {
      mn = sh.wmin[w] < mn ? sh.wmin[w] : mn;
      mx = sh.wmax[w] > mx ? sh.wmax[w] : mx;
    }
    if (mn == mx) return mn;  // one candidate left in play: the need-th
    const int hb = 63 - __builtin_clzll(mn ^ mx);
    const int shift = hb >= 7 ? hb - 7 : 0;
    const uint64_t top = shift + 8 >= 64 ? 0 : (mx >> (shift + 8)) << (shift + 8);  // bits above the window
    visit([&](uint64_t c) {
      if (c >= lo && c <= hi) atomicAdd(&sh.hist[255u - ((uint32_t)(c >> shift) & 255u)], 1u);
    });
    __syncthreads();
    if (wave == 0) {
      // lane l holds bins 4l .. 4l+3, i.e. digits 255 - 4l down to 252 - 4l
      const uint4 h = *(const uint4 *)(sh.hist + 4 * lane);
      const uint32_t hh[4] = {h.x, h.y, h.z, h.w};
      const uint32_t tot = h.x + h.y + h.z + h.w;
      uint32_t above = wave_scan(tot) - tot;  // candidates in play with larger digits
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (above < rem && above + hh[q] >= rem) {
          sh.st[0] = 255u - (uint32_t)(4 * lane + q);
          sh.st[1] = rem - above;
          sh.st[2] = hh[q] == rem - above ? 1u : 0u;
        }
        above += hh[q];
      }
    }
    __syncthreads();
    const uint32_t digit = sh.st[0];
    const uint64_t blo = top | ((uint64_t)digit << shift);
    if (sh.st[2]) return blo;   // the bin and everything above it: exactly need
    rem = sh.st[1];
    lo = blo;
    hi = blo + (((uint64_t)1 << shift) - 1u);
  }
  return lo;  // not reached: each round narrows the candidates in play
}

// R records per thread: thread t holds the records of groups t + 256 r.
template <int R>
__global__ __launch_bounds__(kPickThreads) void k_topk_pick(const uint32_t *__restrict__ logits, uint32_t vocab,
                                                            uint32_t m, TopkPenal penal, uint32_t n_penal,
                                                            uint32_t serial, uint32_t gs, uint32_t groups,
                                                            const uint8_t *__restrict__ rec,
                                                            uint32_t *__restrict__ out) {
  __shared__ PickShared sh;
  __shared__ uint32_t flags, nsat, ncand, nsel;
  __shared__ uint32_t satg[kPickThreads * R];
  __shared__ uint64_t cand_c[kCandMax];
  __shared__ uint32_t cand_b[kCandMax];
  __shared__ uint32_t cand_r[kCandMax];
  const int tid = threadIdx.x, lane = tid & 63;
  uint64_t c[R][4];
  uint32_t b[R][4];
  uint32_t nan = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t g = (uint32_t)tid + kPickThreads * r;
#pragma unroll
    for (int i = 0; i < 4; ++i) { c[r][i] = 0u; b[r][i] = 0u; }
    if (g < groups) {
      const uint4 *rp = (const uint4 *)(rec + (uint64_t)g * kTopkRecordBytes);
      const uint4 q0 = rp[0], q1 = rp[1], q2 = rp[2], q3 = rp[3];
      c[r][0] = ((uint64_t)q0.y << 32) | q0.x;
      c[r][1] = ((uint64_t)q0.w << 32) | q0.z;
      c[r][2] = ((uint64_t)q1.y << 32) | q1.x;
      c[r][3] = ((uint64_t)q1.w << 32) | q1.z;
      b[r][0] = q2.x; b[r][1] = q2.y; b[r][2] = q2.z; b[r][3] = q2.w;
      nan |= q3.x;
    }
  }
  // penalised ids: their raw logits (the penalty itself is applied by the sampler)
  uint32_t pv = 0u;
  if ((uint32_t)tid < n_penal && penal.ids[tid] < vocab) pv = logits[penal.ids[tid]];
  const bool wnan = __ballot(nan != 0u) != 0u;
  if (tid == 0) {
    flags = 0u;
    nsat = 0u;
    ncand = 0u;
    nsel = 0u;
  }
  __syncthreads();
  if (lane == 0 && wnan) atomicOr(&flags, 2u);
  const uint32_t need = min(m, vocab);
  // tau: the need-th largest group maximum (0 when there are no more groups).
  // Every one of the overall need largest is >= tau, and only the `need`
  // groups whose maximum is >= tau list composites >= tau.
  uint64_t tau = 0;
  if (groups > need) {
    tau = select_top(need, [&](auto f) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (c[r][0]) f(c[r][0]);
    }, sh);
  }
  // the listed composites >= tau: at most 4 need of them
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (c[r][i] && c[r][i] >= tau) {
        const uint32_t q = atomicAdd(&ncand, 1u);
        if (q < kCandMax) {
          cand_c[q] = c[r][i];
          cand_b[q] = b[r][i];
        }
      }
    }
  __syncthreads();
  const uint32_t nc = min(ncand, kCandMax);
  uint64_t T = 0;        // exactly `need` candidates (of the final set) are >= T
  bool ranked = false;   // cand_r holds every candidate's rank
  if (nc <= need) {
    // exactly the need candidates >= tau; or, with no more groups than need,
    // every listed composite (groups with more than 4 elements then count as
    // saturated below and are read whole)
    T = groups > need ? tau : 0;
  } else {
    // rank = candidates above, counted by P threads of one wave per candidate
    uint32_t P = 64;
    while (P > 1 && nc * P > (uint32_t)kPickThreads) P >>= 1;
    for (uint32_t i0 = 0; i0 < nc; i0 += kPickThreads / P) {
      const uint32_t i = i0 + (uint32_t)tid / P, part = (uint32_t)tid % P;
      uint32_t rank = 0;
      uint64_t ci = 0;
      if (i < nc) {
        ci = cand_c[i];
        for (uint32_t j = part; j < nc; j += P) rank += cand_c[j] > ci ? 1u : 0u;
      }
      for (uint32_t o = 1; o < P; o <<= 1) rank += (uint32_t)__shfl_xor((int)rank, (int)o, 64);
      if (i < nc && part == 0u) {
        cand_r[i] = rank;
        if (rank == need - 1u) sh.wmin[0] = ci;   // the need-th largest candidate
      }
    }
    __syncthreads();
    T = sh.wmin[0];
    ranked = true;
  }
  // saturated groups: more than 4 elements and the 4th listed one selected
  bool sat[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t g = (uint32_t)tid + kPickThreads * r;
    const uint32_t gcount = g < groups ? min(gs, vocab - g * gs) : 0u;
    sat[r] = gcount > 4u && c[r][3] >= T;
    if (sat[r]) satg[atomicAdd(&nsat, 1u)] = g;
  }
  __syncthreads();
  const uint32_t ns = nsat;
  uint32_t *pairs = out + EFF_TOPK_HEADER + EFF_TOPK_P_MAX;
  uint32_t n = need;
  if (ns == 0u && ranked) {
    // the candidates' ranks are final: the winners go straight to their slots
    for (uint32_t i = (uint32_t)tid; i < nc; i += kPickThreads) {
      if (cand_r[i] < need) {
        pairs[2 * cand_r[i]] = ~(uint32_t)cand_c[i];
        pairs[2 * cand_r[i] + 1] = cand_b[i];
      }
    }
  } else {
    auto stream = [&](auto f) {
      for (uint32_t i = (uint32_t)tid; i < ns * gs; i += kPickThreads) {
        const uint32_t e = satg[i / gs] * gs + i % gs;
        if (e < vocab) {
          const uint32_t bits = logits[e];
          f(composite(bits, e), bits);
        }
      }
    };
    if (ns) {
      // the unsaturated groups' lists plus every element of the saturated groups
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (sat[r]) c[r][0] = c[r][1] = c[r][2] = c[r][3] = 0u;
      T = select_top(need, [&](auto f) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (c[r][i]) f(c[r][i]);
        stream([&](uint64_t v, uint32_t) { f(v); });
      }, sh);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (c[r][i] && c[r][i] >= T) {
            const uint32_t q = atomicAdd(&nsel, 1u);
            if (q < EFF_TOPK_M_MAX) { cand_c[q] = c[r][i]; cand_b[q] = b[r][i]; }
          }
        }
      stream([&](uint64_t v, uint32_t bits) {
        if (v >= T) {
          const uint32_t q = atomicAdd(&nsel, 1u);
          if (q < EFF_TOPK_M_MAX) { cand_c[q] = v; cand_b[q] = bits; }
        }
      });
    } else {
      // winners among the candidates in LDS (all of them: nc <= need), in place
      if (tid == 0) nsel = nc;
    }
    __syncthreads();
    n = min(nsel, (uint32_t)EFF_TOPK_M_MAX);
    // rank = winners above, counted by one thread per winner
    for (uint32_t i = (uint32_t)tid; i < n; i += kPickThreads) {
      const uint64_t ci = cand_c[i];
      uint32_t rank = 0;
      for (uint32_t j = 0; j < n; ++j) rank += cand_c[j] > ci ? 1u : 0u;
      pairs[2 * rank] = ~(uint32_t)ci;
      pairs[2 * rank + 1] = cand_b[i];
    }
  }
  // unused pair slots, the penalised logits and the header
  for (uint32_t slot = n + (uint32_t)tid; slot < EFF_TOPK_CAP; slot += kPickThreads) {
    pairs[2 * slot] = 0u;
    pairs[2 * slot + 1] = 0u;
  }
  if (tid < (int)EFF_TOPK_P_MAX) out[EFF_TOPK_HEADER + tid] = pv;
  if (tid == 0) {
    out[0] = n;
    out[1] = flags | (n != need ? 4u : 0u);
    out[2] = n_penal;
    out[3] = (vocab + kTopkRecordChunk - 1u) / kTopkRecordChunk;
    out[4] = serial;
    out[5] = out[6] = out[7] = 0u;
  }
}

}  // namespace

size_t topk_scratch_bytes(uint32_t vocab) { return topk_scratch_bytes_for(vocab); }

hipError_t launch_topk_pick(const uint32_t *logits, uint32_t vocab, uint32_t m, const uint32_t *penal_ids,
                            uint32_t n_penal, uint32_t serial, uint32_t gs, uint32_t groups, const uint8_t *rec,
                            uint32_t *out, hipStream_t s) {
  if (vocab == 0 || vocab >= EFF_TOPK_N_MAX || m == 0 || m > EFF_TOPK_M_MAX || n_penal > EFF_TOPK_P_MAX ||
      groups == 0 || groups > kTopkPickGroupsMax || (uint64_t)groups * gs < vocab)
    return hipErrorInvalidValue;
  TopkPenal pen{};
  for (uint32_t i = 0; i < n_penal; ++i) pen.ids[i] = penal_ids[i];
  if (groups <= (uint32_t)kPickThreads)
    hipLaunchKernelGGL((k_topk_pick<1>), dim3(1), dim3(kPickThreads), 0, s, logits, vocab, m, pen, n_penal, serial, gs,
                       groups, rec, out);
  else if (groups <= 2u * kPickThreads)
    hipLaunchKernelGGL((k_topk_pick<2>), dim3(1), dim3(kPickThreads), 0, s, logits, vocab, m, pen, n_penal, serial, gs,
                       groups, rec, out);
  else
    hipLaunchKernelGGL((k_topk_pick<4>), dim3(1), dim3(kPickThreads), 0, s, logits, vocab, m, pen, n_penal, serial, gs,
                       groups, rec, out);
  return hipGetLastError();
}

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
