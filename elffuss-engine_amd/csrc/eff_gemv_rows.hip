// One-token GEMV for Q6_K matrices with many rows (the output projection,
// rows >= kRowsMin): y[row] = sum_k W[row][k] x[k], with every lane owning
// half of a row's 256-weight block, so the rows' sums need no cross-lane
// reduction and x is read as a broadcast.
//
// Weights. A wave owns a tile of 32 rows x one block column. The tile's bytes
// (32 x 210, each row from its 4-byte aligned start, 240-byte LDS rows) come
// in by direct-to-LDS loads (coalesced 16-byte chunks), into one 8 KB buffer
// per wave; the load of the next block column goes out as soon as the
// current tile is in registers. Lane l < 32 takes weights 0..127 of row l,
// lane l + 32 weights 128..255 (the halves n = 0, 1 of kernels.wgsl.js:
// 269-330): ql bytes 64n.., qh bytes 32n.., scales 8n..8n+7 and d. With the
// 240-byte row pitch the 16-byte reads of 16 lanes fall in 16 different bank
// quads.
//
// Arithmetic. As k_gemv_mx: x as three signed 8-bit digit planes per group of
// 32 values (22 bits of each group's maximum, eff_xdigits.h), weights as
// u = ql nibble | qh bits << 4 in 0..63, so that per run of 16 weights with
// int8 scale sc
//   sum w x = d sc (p ((D2 256 + D1) 256 + D0) - 32 sum_16 x),
// the three integer sums D_i = sum u d_i formed exactly by v_dot4_i32_i8
// against digits read as LDS broadcasts (all lanes of a half read the same
// address).
//
// Workgroup: 8 waves = 4 row groups x 2 k slices (each wave walks half of the
// block columns); the two slices of a row are added in a fixed order. With
// REC the workgroup also writes the top-k record of its 128 rows (their 4
// largest logits, eff_topk.h), so that the top-k over the logits only has to
// select from the records.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
#include "eff_formats.h"
#include "eff_kernels.h"
#include "eff_topk.h"
#include "eff_xdigits.h"

namespace eff {

namespace {

constexpr uint32_t kRowsWaves = 8, kRowsKS = 2, kRowsGroups = kRowsWaves / kRowsKS;
constexpr uint32_t kRowsTile = 32;                    // rows per wave tile
constexpr uint32_t kRowsPerWG = kRowsGroups * kRowsTile;
constexpr uint32_t kRowsPitch = 240;                  // LDS bytes per tile row (15 chunks)
constexpr uint32_t kRowsBuf = 8192;                   // LDS bytes per wave (8 loads of 1 KB)
constexpr uint32_t kRowsMin = 32768;
constexpr uint32_t kRowsMaxK = 16384;

template <bool REC>
__global__ __launch_bounds__(kRowsWaves * 64) void k_gemv_rows_q6k(WeightView wv, const float *__restrict__ x,
                                                                    float *__restrict__ y, uint8_t *__restrict__ rec) {
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t k = wv.k, bpr = wv.bpr, rows = wv.rows;
  uint8_t *const tile = lds + wave * kRowsBuf;
  uint8_t *const xl = lds + kRowsWaves * kRowsBuf;
  const uint32_t rg = wave / kRowsKS, ks = wave % kRowsKS;
  const uint32_t r0 = (blockIdx.x * kRowsGroups + rg) * kRowsTile;
  const uint32_t j0 = ks * bpr / kRowsKS, j1 = (ks + 1u) * bpr / kRowsKS;
  const rsrc_t src = make_rsrc(wv.w, wv.w_bytes);

  // Load i of the lane fills LDS chunk s = 64 i + lane = row s / 15, chunk
  // s % 15 of that row; chunk 14 repeats 13 (a cache hit) so that rows are
  // 240 bytes apart; slots past the 32 rows repeat row 31.
  uint32_t srow[8], sch[8];
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) {
    const uint32_t sl = 64u * i + lane, r = sl / 15u, c = sl - 15u * r;
    srow[i] = min(r0 + min(r, kRowsTile - 1u), rows - 1u);
    sch[i] = r >= kRowsTile ? 0u : 16u * min(c, 13u);
  }
  auto issue = [&](uint32_t j) {
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) dma16(src, tile + 1024u * i, (((srow[i] * bpr + j) * 210u) & ~3u) + sch[i], 0);
  };
  if (j0 < j1) issue(j0);

  // x digits of the whole k, once per workgroup
  for (uint32_t o = tid; o < k / 8u; o += kRowsWaves * 64u) {
    XOct v;
    x_load<1>(x, k, o, v);
    x_store<1>(v, k, o, xl, k * 3u, (float *)(xl + k * 3u), k / 8u);
  }
  __syncthreads();
  const uint8_t *dig = xl;
  const float *meta = (const float *)(xl + k * 3u);

  const uint32_t rr = lane & 31u, n = lane >> 5;
  const uint32_t row = r0 + rr, rowc = min(row, rows - 1u);
  float acc = 0.f;
  for (uint32_t j = j0; j < j1; ++j) {
    wait_vm<0>();   // this tile's loads (the only ones in flight)
    const uint8_t *t = tile + kRowsPitch * rr;
    uint32_t a[20], q[12], sv[8];
#pragma unroll
    for (uint32_t i = 0; i < 5; ++i) {
      const u32x4 v = *(const u32x4 *)(t + 64u * n + 16u * i);
      a[4 * i] = v.x; a[4 * i + 1] = v.y; a[4 * i + 2] = v.z; a[4 * i + 3] = v.w;
    }
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i) {
      const u32x4 v = *(const u32x4 *)(t + 128u + 32u * n + 16u * i);
      q[4 * i] = v.x; q[4 * i + 1] = v.y; q[4 * i + 2] = v.z; q[4 * i + 3] = v.w;
    }
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
      const u32x4 v = *(const u32x4 *)(t + 192u + 16u * i);
      sv[4 * i] = v.x; sv[4 * i + 1] = v.y; sv[4 * i + 2] = v.z; sv[4 * i + 3] = v.w;
    }
    // the tile is in registers: the buffer takes the next block column
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    if (j + 1u < j1) issue(j + 1u);
    // the block starts sh = 0 or 2 bytes past the aligned start of its row's copy
    const uint32_t sh = ((rowc * bpr + j) * 210u) & 3u;
    uint32_t QL[16], QH[8];
#pragma unroll
    for (int i = 0; i < 16; ++i) QL[i] = __builtin_amdgcn_alignbyte(a[i + 1], a[i], sh);
#pragma unroll
    for (int i = 0; i < 8; ++i) QH[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], sh);
    const uint32_t s0 = __builtin_amdgcn_alignbyte(sv[2 * n + 1], sv[2 * n], sh);
    const uint32_t s1 = __builtin_amdgcn_alignbyte(sv[2 * n + 2], sv[2 * n + 1], sh);
    const uint32_t dw = __builtin_amdgcn_alignbyte(sv[5], sv[4], sh);
    // this half's x: 8 runs of 16 from k = 256 j + 128 n
    const uint8_t *dj = dig + (16u * j + 8u * n) * 48u;
    const float *mj = meta + 4u * (8u * j + 4u * n);
    float accb = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        // weights 32 g + 16 hh + 4 i .. + 3 of the half (ql nibble, 2 bits of qh)
        uint32_t u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int lc = 4 * hh + i;
          const uint32_t ql = QL[8 * (g & 1) + lc], qh = QH[lc];
          const uint32_t lo = (g & 2) ? (ql >> 4) : ql;
          const uint32_t hi = g == 0 ? (qh << 4) : g == 1 ? (qh << 2) : g == 2 ? qh : (qh >> 2);
          u[i] = (lo & 0x0F0F0F0Fu) | (hi & 0x30303030u);
        }
        const uint32_t run = 2u * g + hh;   // 16-weight run of the half
        const uint8_t *dA = dj + run * 48u;
        int D[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          const u32x4 X = *(const u32x4 *)(dA + 16 * p);
          int d = __builtin_amdgcn_sdot4((int)u[0], (int)X.x, 0, false);
          d = __builtin_amdgcn_sdot4((int)u[1], (int)X.y, d, false);
          d = __builtin_amdgcn_sdot4((int)u[2], (int)X.z, d, false);
          D[p] = __builtin_amdgcn_sdot4((int)u[3], (int)X.w, d, false);
        }
        const float4 M = *(const float4 *)(mj + 4u * (run / 2u));   // {p, sum x[0..15], sum x[16..31]}
        const float s16 = hh ? M.z : M.y;
        const float sc = (float)(int)__builtin_amdgcn_sbfe((int)(run < 4u ? s0 : s1), 8u * (run & 3u), 8);
        const float f = __builtin_fmaf((float)(D[2] * 256 + D[1]), 256.f, (float)D[0]);
        accb = __builtin_fmaf(sc, __builtin_fmaf(M.x, f, -32.f * s16), accb);
      }
    acc = __builtin_fmaf(h2f(dw & 0xFFFFu), accb, acc);
  }
  // the two halves of a row, then its two k slices in order
  acc += __shfl_xor(acc, 32);
  float *red = (float *)xl;   // the x digits are no longer read
  __syncthreads();
  if (n == 0u) red[wave * kRowsTile + rr] = acc;
  __syncthreads();
  uint32_t *fin = (uint32_t *)(xl + 1024u);   // the workgroup's outputs, for the record
  if (ks == 0u && n == 0u) {
    float v = red[wave * kRowsTile + rr];
#pragma unroll
    for (uint32_t q2 = 1; q2 < kRowsKS; ++q2) v += red[(wave + q2) * kRowsTile + rr];
    if (row < rows) y[row] = v;
    if constexpr (REC) fin[rg * kRowsTile + rr] = __builtin_bit_cast(uint32_t, v);
  }
  if constexpr (REC) {
    __syncthreads();
    if (wave == 0u) {
      // rows l and l + 64 of the workgroup's 128
      const uint32_t base = blockIdx.x * kRowsPerWG;
      Top4 t;
      bool nan = false;
#pragma unroll
      for (uint32_t h = 0; h < 2u; ++h) {
        const uint32_t i = lane + 64u * h, e = base + i;
        if (e < rows) {
          const uint32_t bits = fin[i];
          nan |= is_nan_bits(bits);
          t.add(composite(bits, e), bits);
        }
      }
      topk_record_wave(t, nan, rec + (uint64_t)blockIdx.x * kTopkRecordBytes);
    }
  }
}

}  // namespace

bool gemv_rows_applies(const WeightView &wv, uint32_t tokens) {
  return wv.type == Q6_K && tokens == 1u && wv.rows >= kRowsMin && wv.k <= kRowsMaxK && wv.bpr >= kRowsKS &&
         (uint64_t)wv.rows * wv.row_bytes + 16u < (1ull << 32);   // 32-bit byte offsets
}

uint32_t gemv_rows_groups(const WeightView &wv) { return (wv.rows + kRowsPerWG - 1u) / kRowsPerWG; }
uint32_t gemv_rows_group_size() { return kRowsPerWG; }

hipError_t launch_gemv_rows(const WeightView &wv, const float *x, float *y, uint8_t *rec, hipStream_t s) {
  if (!gemv_rows_applies(wv, 1u)) return hipErrorInvalidValue;
  static bool attr[2] = {false, false};
  const void *fn = rec ? (const void *)k_gemv_rows_q6k<true> : (const void *)k_gemv_rows_q6k<false>;
  if (!attr[rec ? 1 : 0]) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMxMaxLds);
    if (e != hipSuccess) return e;
    attr[rec ? 1 : 0] = true;
  }
  // the x digits region also holds the slice sums (1 KB) and the outputs (512 B) at the end
  const uint32_t xbytes = wv.k * 3u + (wv.k / 8u) * 4u;
  const uint32_t lds = kRowsWaves * kRowsBuf + (xbytes > 1536u ? xbytes : 1536u);
  const uint32_t grid = gemv_rows_groups(wv);
  if (rec)
    hipLaunchKernelGGL((k_gemv_rows_q6k<true>), dim3(grid), dim3(kRowsWaves * 64), lds, s, wv, x, y, rec);
  else
    hipLaunchKernelGGL((k_gemv_rows_q6k<false>), dim3(grid), dim3(kRowsWaves * 64), lds, s, wv, x, y, rec);
  return hipGetLastError();
}

}  // namespace eff
