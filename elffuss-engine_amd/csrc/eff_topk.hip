// Exact top-m (m <= 192) of one logits vector, ordered by (f32 value desc
// with -0 == +0, index asc), and the raw logits of the penalised ids, written
// as the reference's output record (kernels.topk.wgsl.js:40-60,
// ops.topk.js:99-165; the order of sample.js:44-67).
//
// Elements are compared by the 64-bit composite (order_key(bits) << 32 |
// ~index): unique per element, larger composite = larger value, ties to the
// lower index. order_key maps f32 order to u32 order with -0 = +0
// (kernels.topk.wgsl.js:75-82). A valid element's composite is never 0
// (~index has its top 8 bits set for index < 2^24), so 0 marks "none".
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

namespace eff {

namespace {

__device__ __forceinline__ uint32_t order_key(uint32_t bits) {
  const uint32_t b = bits == 0x80000000u ? 0u : bits;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ bool is_nan_bits(uint32_t bits) { return (bits & 0x7FFFFFFFu) > 0x7F800000u; }

__device__ __forceinline__ uint64_t composite(uint32_t bits, uint32_t idx) {
  return ((uint64_t)order_key(bits) << 32) | (uint64_t)(~idx);
}

struct TopkPenal {
  uint32_t ids[EFF_TOPK_P_MAX];
};

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
  // the group's 4 largest: 4 rounds of a wave maximum over the lanes' heads
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
    uint4 *dst = (uint4 *)(rec + (uint64_t)g * kTopkRecordBytes);
    uint4 v;
    if (lane < 2u) {
      const uint64_t a = out_c[2 * lane], b = out_c[2 * lane + 1];
      v = make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
    } else if (lane == 2u) {
      v = make_uint4(out_b[0], out_b[1], out_b[2], out_b[3]);
    } else {
      v = make_uint4(any_nan ? 1u : 0u, 0u, 0u, 0u);
    }
    dst[lane] = v;
  }
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

__global__ __launch_bounds__(kPickThreads) void k_topk_pick(const uint32_t *__restrict__ logits, uint32_t vocab,
                                                            uint32_t m, TopkPenal penal, uint32_t n_penal,
                                                            uint32_t serial, uint32_t per, uint32_t groups,
                                                            const uint8_t *__restrict__ rec,
                                                            uint32_t *__restrict__ out) {
  __shared__ PickShared sh;
  __shared__ uint32_t flags, nsat, ncand, nsel;
  __shared__ uint32_t satg[kTopkGroupsMax];
  __shared__ uint64_t cand_c[kCandMax];
  __shared__ uint32_t cand_b[kCandMax];
  __shared__ uint32_t cand_r[kCandMax];
  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t gs = 64u * per;
  uint64_t c[4] = {0, 0, 0, 0};
  uint32_t b[4] = {0, 0, 0, 0};
  uint32_t nan = 0;
  if ((uint32_t)tid < groups) {
    const uint4 *r = (const uint4 *)(rec + (uint64_t)tid * kTopkRecordBytes);
    const uint4 q0 = r[0], q1 = r[1], q2 = r[2], q3 = r[3];
    c[0] = ((uint64_t)q0.y << 32) | q0.x;
    c[1] = ((uint64_t)q0.w << 32) | q0.z;
    c[2] = ((uint64_t)q1.y << 32) | q1.x;
    c[3] = ((uint64_t)q1.w << 32) | q1.z;
    b[0] = q2.x; b[1] = q2.y; b[2] = q2.z; b[3] = q2.w;
    nan = q3.x;
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
  uint64_t tau = 0;
  if (groups > need) tau = select_top(need, [&](auto f) { if (c[0]) f(c[0]); }, sh);
  // the listed composites >= tau: at most 4 need of them
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (c[i] && c[i] >= tau) {
      const uint32_t q = atomicAdd(&ncand, 1u);
      if (q < kCandMax) {
        cand_c[q] = c[i];
        cand_b[q] = b[i];
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
  const uint32_t gcount = (uint32_t)tid < groups ? min(gs, vocab - (uint32_t)tid * gs) : 0u;
  const bool sat = gcount > 4u && c[3] >= T;
  if (sat) satg[atomicAdd(&nsat, 1u)] = (uint32_t)tid;
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
      if (sat) c[0] = c[1] = c[2] = c[3] = 0u;
      T = select_top(need, [&](auto f) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (c[i]) f(c[i]);
        stream([&](uint64_t v, uint32_t) { f(v); });
      }, sh);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (c[i] && c[i] >= T) {
          const uint32_t q = atomicAdd(&nsel, 1u);
          if (q < EFF_TOPK_M_MAX) { cand_c[q] = c[i]; cand_b[q] = b[i]; }
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

hipError_t launch_topk(const uint32_t *logits, uint32_t base, uint32_t vocab, uint32_t m,
                       const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, uint32_t *scratch,
                       uint32_t *out, hipStream_t s) {
  if (vocab == 0 || vocab >= EFF_TOPK_N_MAX || m == 0 || m > EFF_TOPK_M_MAX || n_penal > EFF_TOPK_P_MAX)
    return hipErrorInvalidValue;
  const uint32_t gs = topk_group_size(vocab), groups = topk_groups(vocab);
  if (groups > kTopkGroupsMax) return hipErrorInvalidValue;
  TopkPenal pen{};
  for (uint32_t i = 0; i < n_penal; ++i) pen.ids[i] = penal_ids[i];
  const uint32_t *lg = logits + base;
  hipLaunchKernelGGL(k_topk_groups, dim3(groups), dim3(64), 0, s, lg, vocab, gs / 64u, (uint8_t *)scratch);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_topk_pick, dim3(1), dim3(kPickThreads), 0, s, lg, vocab, m, pen, n_penal, serial, gs / 64u,
                     groups, (const uint8_t *)scratch, out);
  return hipGetLastError();
}

}  // namespace eff
