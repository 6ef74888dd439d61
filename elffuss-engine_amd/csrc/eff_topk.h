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
// 12 bytes unused. The G records of a selection are followed by an array of
// the G groups' largest composites (c[0] again, 8 bytes each), so that the
// selection's first step reads 8 contiguous bytes per group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
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
// of 16 (quad xor 1, quad xor 2, half-row mirror, row mirror), then rows 0 + 1
// into row 1 and 2 + 3 into row 3 (row_bcast:15), rows 1 into 3
// (row_bcast:31), and lane 63 read out. The result is wave-uniform. The DPP
// moves read the operation's identity where a row takes no source, so each
// fuses into the operation.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext(uint32_t v) {
  auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  constexpr int id = MAX ? 0 : -1;
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0xB1, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x4E, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x141, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x140, 0xF, 0xF, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x142, 0xA, 0xF, false));   // row_bcast:15
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x143, 0xC, 0xF, false));   // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Wave-wide maximum / minimum of a u64, as its high word then the low word
// among the lanes holding that high word.
template <bool MAX>
__device__ __forceinline__ uint64_t wave_ext64(uint64_t v) {
  const uint32_t h = wave_ext<MAX>((uint32_t)(v >> 32));
  const uint32_t l = wave_ext<MAX>((uint32_t)(v >> 32) == h ? (uint32_t)v : (MAX ? 0u : 0xFFFFFFFFu));
  return ((uint64_t)h << 32) | l;
}

// Group g's record from the lanes' own 4 largest (every lane of the wave
// active): 4 rounds of a wave maximum over the lanes' heads; lanes 0..3 write
// the 64 bytes of record g of `recs`, lane 4 the group's largest composite
// into the array after the `groups` records.
__device__ __forceinline__ void topk_record_wave(Top4 t, bool nan, uint8_t *recs, uint32_t g, uint32_t groups) {
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
  uint8_t *const rec = recs + (uint64_t)g * kTopkRecordBytes;
  if (lane == 4u) *(uint64_t *)(recs + (uint64_t)groups * kTopkRecordBytes + 8u * g) = out_c[0];
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

// ---- the selection over the records (k_topk_pick, k_rows_pick) -------------

struct TopkPenal {
  uint32_t ids[EFF_TOPK_P_MAX];
};

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

// LDS of a selection by NT threads holding R records each.
template <int NT, int R>
struct PickLds {
  uint32_t hist[256];   // bin 255 - d counts digit d (descending digits in ascending bins)
  uint32_t st[4];
  uint32_t flags, nsat, nsel;
  uint64_t wmin[NT / 64], wmax[NT / 64], wkth[NT / 64];
  uint32_t wtot[NT / 64];   // the waves' candidate counts
  uint32_t fsat;            // a saturated group's 4th listed composite was selected
  uint32_t satg[NT * R];
  alignas(16) uint64_t cand_c[kCandMax + 4];   // 4 zero entries past the candidates (rank reads in pairs)
  uint32_t cand_b[kCandMax];
  uint32_t cand_f[kCandMax];   // 1: the 4th listed composite of a group of more than 4 elements
};

// Sum of v over aligned groups of P consecutive lanes (P a power of two <= 64,
// wave-uniform; every lane active), each lane getting its group's sum: DPP
// within rows (quad swaps, half-row and row mirrors), then lane shuffles.
__device__ __forceinline__ uint32_t group_sum(uint32_t v, uint32_t P) {
  if (P >= 2u) v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
  if (P >= 4u) v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
  if (P >= 8u) v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false);
  if (P >= 16u) v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false);
  if (P >= 32u) v += (uint32_t)__shfl_xor((int)v, 16, 64);
  if (P >= 64u) v += (uint32_t)__shfl_xor((int)v, 32, 64);
  return v;
}

// Radix select over distinct 64-bit candidates: returns T such that exactly
// `need` candidates are >= T (1 <= need <= number of candidates). Each round
// finds the smallest and largest candidate still in play, places an 8-bit
// digit window at their highest differing bit, and keeps the bin that holds
// the need-th largest. `visit(f)` calls f(c) for each candidate the calling
// thread holds. Every thread of the workgroup calls it.
template <int NT, class Visit, class L>
__device__ uint64_t select_top(uint32_t need, Visit visit, L &sh) {
  constexpr int NW = NT / 64;
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
    if (tid < 256) sh.hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NW; ++w) {
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

// Groups of gs consecutive logits: group g is logits g gs .. g gs + gs - 1.
struct FlatGroups {
  uint32_t gs;
  __device__ uint32_t size() const { return gs; }   // elements of the largest group
  __device__ uint32_t elem(uint32_t g, uint32_t j) const { return g * gs + j; }
  __device__ uint32_t count(uint32_t g, uint32_t vocab) const {   // its elements below vocab
    return g * gs < vocab ? min(gs, vocab - g * gs) : 0u;
  }
};

// The top-m selection over `groups` records (record g at rec + 64 g), by the
// NT threads of one workgroup, thread t holding the records of groups
// t + NT r (r < R); writes the output record of kernels.topk.wgsl.js:40-60.
// `map` gives the logits of group g: map.elem(g, j) for j < map.size(), those
// below vocab counted by map.count(g, vocab) (FlatGroups, or the head GEMV's
// tiles).
//
// tau: a lower bound of the need-th largest group maximum. Every one of the
// overall need largest elements is >= the need-th largest maximum, so the
// need largest of the listed composites >= tau (ranked by counting) are the
// answer, unless some group has more than 4 elements and its 4th listed
// composite is among them ("saturated"): an element a group does not list is
// below its 4th, and if that 4th is not selected, need listed composites beat
// it. Otherwise the select runs again over the unsaturated groups' lists plus
// every element of the saturated groups, read from memory. The winners are
// written sorted by (value desc, index asc).
//
// tau is first the smallest of the waves' kw-th largest maxima, kw =
// ceil(need / NW) (NW kw >= need of the maxima are >= it, so it is a lower
// bound; need <= 64 here): kw rounds of a wave maximum, no selection. When that leaves more listed composites
// than the candidate space, or need > 64, tau is the need-th largest maximum
// exactly, by select_top (then at most 4 need composites are listed >= it).
template <int NT, int R, class Map>
__device__ void topk_pick(const uint32_t *__restrict__ logits, uint32_t vocab, uint32_t m, const TopkPenal &penal,
                          uint32_t n_penal, uint32_t serial, const Map &map, uint32_t groups,
                          const uint8_t *__restrict__ rec, uint32_t *__restrict__ out, PickLds<NT, R> &sh) {
  constexpr int NW = NT / 64, KW = 64 / NW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t c[R][4];
  uint32_t b[R][4];
  uint32_t nan = 0;
  // the groups' maxima, then their records, through buffer descriptors of
  // their bytes: a group past the last reads as zeros (no composites, no NaN)
  const rsrc_t ms = make_rsrc(rec + (uint64_t)groups * kTopkRecordBytes, (uint64_t)groups * 8u);
  const rsrc_t rs = make_rsrc(rec, (uint64_t)groups * kTopkRecordBytes);
  uint32_t mk[R];   // the maxima's high words (order keys)
#pragma unroll
  for (int r = 0; r < R; ++r) mk[r] = __builtin_amdgcn_raw_buffer_load_b32(ms, (tid + NT * r) * 8 + 4, 0, 0);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int off = (tid + NT * r) * (int)kTopkRecordBytes;
    const u32x4 q0 = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
    const u32x4 q1 = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0);
    const u32x4 q2 = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 32, 0, 0);
    const uint32_t q3 = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 48, 0, 0);
    c[r][0] = ((uint64_t)q0.y << 32) | q0.x;
    c[r][1] = ((uint64_t)q0.w << 32) | q0.z;
    c[r][2] = ((uint64_t)q1.y << 32) | q1.x;
    c[r][3] = ((uint64_t)q1.w << 32) | q1.z;
    b[r][0] = q2.x; b[r][1] = q2.y; b[r][2] = q2.z; b[r][3] = q2.w;
    nan |= q3;
  }
  // penalised ids: their raw logits (the penalty itself is applied by the
  // sampler). Every thread loads, from clamped places, after the maxima and
  // the records: the loads complete in order, and the first step waits only
  // for the maxima.
  const uint32_t pid = penal.ids[min((uint32_t)tid, (uint32_t)EFF_TOPK_P_MAX - 1u)];
  if (tid == 0) {
    sh.flags = 0u;
    sh.nsat = 0u;
    sh.nsel = 0u;
    sh.fsat = 0u;
  }
  const uint32_t need = min(m, vocab);
  uint32_t *const pairs = out + EFF_TOPK_HEADER + EFF_TOPK_P_MAX;
  // group g of the thread's record r holds more than 4 elements
  auto over4 = [&](int r) {
    const uint32_t g = (uint32_t)tid + NT * r;
    return g < groups && map.count(g, vocab) > 4u;
  };
  // the listed composites >= th into the candidate space in thread order (a
  // wave prefix sum of the lanes' counts, the waves' totals through LDS);
  // returns their number (only the first kCandMax are stored)
  auto compact = [&](uint64_t th) {
    uint32_t cnt = 0;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) cnt += (c[r][i] && c[r][i] >= th) ? 1u : 0u;
    const uint32_t incl = wave_scan(cnt);
    if (lane == 63) sh.wtot[wave] = incl;
    __syncthreads();
    uint32_t q = incl - cnt, tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t t = sh.wtot[w];
      q += w < wave ? t : 0u;
      tot += t;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (c[r][i] && c[r][i] >= th) {
          if (q < kCandMax) {
            sh.cand_c[q] = c[r][i];
            sh.cand_b[q] = b[r][i];
            sh.cand_f[q] = i == 3 && over4(r) ? 1u : 0u;
          }
          ++q;
        }
      }
    return tot;
  };
  const bool fast = groups > need && need <= (uint32_t)(NW * KW);
  if (fast) {
    // on the maxima's high words (order keys): kth = the wave's kw-th largest
    // distinct key (0 once the wave's maxima run out). Equal keys leave at
    // most fewer distinct values, so the smallest of the waves' kth stays a
    // lower bound.
    uint32_t v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = mk[r];
    uint32_t kth = 0;
    const int kw = (int)((need + NW - 1u) / NW);   // NW kw >= need of the maxima are >= tq
    for (int q = 0; q < kw; ++q) {
      uint32_t lb = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) lb = v[r] > lb ? v[r] : lb;
      kth = wave_ext<true>(lb);
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = v[r] == kth ? 0u : v[r];
    }
    if (lane == 0) sh.wkth[wave] = (uint64_t)kth << 32;
  }
  const bool pok = (uint32_t)tid < n_penal && pid < vocab;
  const uint32_t pl = logits[pok ? pid : 0u];
  const uint32_t pv = pok ? pl : 0u;
  __syncthreads();
  const bool wnan = __ballot(nan != 0u) != 0u;   // every lane active
  if (lane == 0 && wnan) atomicOr(&sh.flags, 2u);
  uint64_t tau = 0;
  uint32_t nc = ~0u;
  if (fast) {
    uint64_t tq = ~(uint64_t)0;
#pragma unroll
    for (int w = 0; w < NW; ++w) tq = sh.wkth[w] < tq ? sh.wkth[w] : tq;
    if (tq != 0u) {
      nc = compact(tq);
      tau = tq;
    }
  }
  if (nc > kCandMax) {
    // no bound, or too many candidates: tau = the need-th largest group
    // maximum exactly (at most 4 need composites are listed >= it), or 0 with
    // no more groups than need (at most 4 need listed composites in all)
    tau = 0;
    if (groups > need) {
      tau = select_top<NT>(need, [&](auto f) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (c[r][0]) f(c[r][0]);
      }, sh);
    }
    nc = min(compact(tau), kCandMax);
  }
  if (tid < 4) sh.cand_c[nc + tid] = 0u;   // the zero entries past the candidates
  __syncthreads();
  // the slots past need stay empty: stores issued once the records are used
  // (the count of memory operations in flight is in order, so a wait for a
  // load issued earlier would also wait for these)
  for (uint32_t slot = need + (uint32_t)tid; slot < EFF_TOPK_CAP; slot += NT) {
    pairs[2 * slot] = 0u;
    pairs[2 * slot + 1] = 0u;
  }
  // rank = candidates above, counted by P threads of one wave per candidate,
  // each over a contiguous quarter-aligned range read in pairs (the zero
  // entries past the candidates count for nothing: every composite is > 0).
  // The need largest go straight to their slots; a group's 4th listed
  // composite among them means the group may hold more of the answer.
  {
    uint32_t lp = 6;   // P = 2^lp threads per candidate
    while (lp > 0 && (nc << lp) > (uint32_t)NT) --lp;
    const uint32_t P = 1u << lp;
    const uint32_t span = (((nc + P - 1u) >> lp) + 3u) & ~3u;
    for (uint32_t i0 = 0; i0 < nc; i0 += (uint32_t)NT >> lp) {
      const uint32_t i = i0 + ((uint32_t)tid >> lp), part = (uint32_t)tid & (P - 1u);
      uint32_t rank = 0;
      uint64_t ci = 0;
      if (i < nc) {
        ci = sh.cand_c[i];
        const uint32_t j0 = part * span, j1 = min(j0 + span, (nc + 3u) & ~3u);
#pragma unroll 4
        for (uint32_t j = j0; j < j1; j += 4u) {
          const ulonglong2 p0 = *(const ulonglong2 *)(sh.cand_c + j);
          const ulonglong2 p1 = *(const ulonglong2 *)(sh.cand_c + j + 2);
          rank += (p0.x > ci ? 1u : 0u) + (p0.y > ci ? 1u : 0u) + (p1.x > ci ? 1u : 0u) + (p1.y > ci ? 1u : 0u);
        }
      }
      rank = group_sum(rank, P);
      if (i < nc && part == 0u && rank < need) {
        pairs[2 * rank] = ~(uint32_t)ci;
        pairs[2 * rank + 1] = sh.cand_b[i];
        if (rank == need - 1u) sh.wmin[0] = ci;   // the need-th largest candidate
        if (sh.cand_f[i]) sh.fsat = 1u;
      }
    }
  }
  __syncthreads();
  uint32_t n = min(nc, need);
  if (sh.fsat) {
    // saturated groups: more than 4 elements and the 4th listed one selected.
    // T: exactly `need` candidates are >= T (every candidate when they are
    // at most need).
    const uint64_t T = nc > need ? sh.wmin[0] : (groups > need ? tau : 0u);
    bool sat[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sat[r] = over4(r) && c[r][3] >= T;
      if (sat[r]) sh.satg[atomicAdd(&sh.nsat, 1u)] = (uint32_t)tid + NT * r;
    }
    __syncthreads();
    const uint32_t ns = sh.nsat;
    const uint32_t gs = map.size();
    auto stream = [&](auto f) {
      for (uint32_t i = (uint32_t)tid; i < ns * gs; i += NT) {
        const uint32_t g = sh.satg[i / gs], j = i % gs;
        const uint32_t e = map.elem(g, j);   // past vocab for j past the group's elements
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
      const uint64_t T2 = select_top<NT>(need, [&](auto f) {
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
          if (c[r][i] && c[r][i] >= T2) {
            const uint32_t q = atomicAdd(&sh.nsel, 1u);
            if (q < EFF_TOPK_M_MAX) { sh.cand_c[q] = c[r][i]; sh.cand_b[q] = b[r][i]; }
          }
        }
      stream([&](uint64_t v, uint32_t bits) {
        if (v >= T2) {
          const uint32_t q = atomicAdd(&sh.nsel, 1u);
          if (q < EFF_TOPK_M_MAX) { sh.cand_c[q] = v; sh.cand_b[q] = bits; }
        }
      });
    } else if (tid == 0) {
      sh.nsel = n;   // not reached (a selected 4th listed composite is >= T): the candidates as ranked
    }
    __syncthreads();
    n = min(sh.nsel, (uint32_t)EFF_TOPK_M_MAX);
    // rank = winners above, counted by one thread per winner
    for (uint32_t i = (uint32_t)tid; i < n; i += NT) {
      const uint64_t ci = sh.cand_c[i];
      uint32_t rank = 0;
      for (uint32_t j = 0; j < n; ++j) rank += sh.cand_c[j] > ci ? 1u : 0u;
      pairs[2 * rank] = ~(uint32_t)ci;
      pairs[2 * rank + 1] = sh.cand_b[i];
    }
  }
  // slots below need left empty, the penalised logits and the header
  for (uint32_t slot = n + (uint32_t)tid; slot < need; slot += NT) {
    pairs[2 * slot] = 0u;
    pairs[2 * slot + 1] = 0u;
  }
  if (tid < (int)EFF_TOPK_P_MAX) out[EFF_TOPK_HEADER + tid] = pv;
  if (tid == 0) {
    out[0] = n;
    out[1] = sh.flags | (n != need ? 4u : 0u);
    out[2] = n_penal;
    out[3] = (vocab + kTopkRecordChunk - 1u) / kTopkRecordChunk;
    out[4] = serial;
    out[5] = out[6] = out[7] = 0u;
  }
}

}  // namespace eff
