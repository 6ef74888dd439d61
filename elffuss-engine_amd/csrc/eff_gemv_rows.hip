// One-token GEMV for Q6_K matrices with many rows (the output projection,
// rows >= kRowsMin): y[row] = sum_k W[row][k] x[k], with every lane owning
// half of a row's 256-weight block, so the rows' sums need no cross-lane
// reduction and x is read as a broadcast.
//
// Weights. A wave owns a tile of 32 rows x one block column at a time. The
// tile's bytes (32 x 210, each row from its 4-byte aligned start, 240-byte LDS
// rows) come in by direct-to-LDS loads (coalesced 16-byte chunks), into one
// 8 KB buffer per wave; the load of the next tile goes out as soon as the
// current one is in registers. Lane l < 32 takes weights 0..127 of row l,
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
// Workgroup: 128 rows on average (tiles of 32 rows, RowsSched below), 8 waves
// = RG row groups x KS k slices (KS = 8 when the matrix has at least 8 block
// columns). Slice s takes the block columns
// s, s + KS, s + 2 KS, ... of each of its tiles, so the KS waves of a row group
// load neighbouring blocks of the same 32 rows at about the same time: the
// 128-byte lines two neighbouring blocks share are fetched from memory once
// and found in L2 by the second wave. (When one wave walks consecutive block
// columns of its rows, the shared lines have left L2 before its next load and
// the kernel reads 1.3 x the matrix.) A row's KS slice sums are added in a
// fixed order. With REC the workgroup also writes the top-k record of its rows
// (their 4 largest logits, eff_topk.h), so that the top-k over the logits
// only has to select from the records.
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

constexpr uint32_t kRowsWaves = 8;
constexpr uint32_t kRowsTile = 32;                    // rows per wave tile
constexpr uint32_t kRowsPerWG = 128;                  // rows per workgroup on average (4 tiles)
constexpr uint32_t kRowsTilesPair = 2u * (kRowsPerWG / kRowsTile);   // tiles of a CU's two workgroups
constexpr uint32_t kRowsTilesFirst[2] = {7, 3};       // tiles of the grid's first half (KS = 8), without / with REC
constexpr uint32_t kRowsTilesMax = 7;                 // of any workgroup
constexpr uint32_t kRowsPitch = 240;                  // LDS bytes per tile row (15 chunks)
constexpr uint32_t kRowsBuf = 8192;                   // LDS bytes per wave (8 loads of 1 KB)
constexpr uint32_t kRowsRed = kRowsTilesMax * kRowsTile * 8u * 4u;   // LDS bytes of the slice sums (rows x up to 8 slices)
constexpr uint32_t kRowsMin = 32768;
constexpr uint32_t kRowsMaxK = 16384;
static_assert(kRowsTilesFirst[0] < kRowsTilesPair && kRowsTilesFirst[1] < kRowsTilesPair &&
                  kRowsTilesFirst[0] <= kRowsTilesMax && kRowsTilesFirst[1] <= kRowsTilesMax &&
                  kRowsTilesPair - kRowsTilesFirst[0] <= kRowsTilesMax &&
                  kRowsTilesPair - kRowsTilesFirst[1] <= kRowsTilesMax,
              "every workgroup has tiles (and writes its record), at most kRowsTilesMax");

// The tiles of 32 rows of the G workgroups (G even, H = G / 2; A tiles for
// workgroup b < H, B for the others, A + B = 8: 128 rows per workgroup on
// average). In round q < m = min(A, B) every workgroup b takes tile q G + b,
// so that the workgroups running at once read one region of the matrix
// rather than G far apart; then the half with more tiles takes tile
// m G + (q - m) H + b mod H in round q >= m. The dispatcher places the
// workgroups in index order, so every CU holds one workgroup of each half,
// and the first half's loads are served ahead: with 4 tiles each, its
// workgroups ended after 13.4 us, the second half's after 19.1 (C4). For the
// GEMV A = 7, B = 1 measured fastest (C4: 20.9-21.0 us against 21.5-21.7 for
// 4 + 4; 3 + 5 21.0-21.5, 5 + 3 21.4-21.9, 6 + 2 22.0-22.5, 8 tiles on one
// workgroup per CU 21.9). It also maps the head's top-k groups for topk_pick.
struct RowsSched {
  uint32_t G, H, A, B;   // A tiles for b < H, B for the others
  __host__ __device__ uint32_t ntiles(uint32_t b) const { return b < H ? A : B; }
  __host__ __device__ uint32_t tile(uint32_t b, uint32_t q) const {
    const uint32_t m = A < B ? A : B;
    return q < m ? q * G + b : m * G + (q - m) * H + (b < H ? b : b - H);
  }
  // The record of workgroup b is group rec_group(b) of the top-k: the two
  // halves alternate, so that every wave of the selection holds as many
  // groups of each size (its threshold is a bound over each wave's largest
  // group maxima: with the short groups in waves of their own it falls to
  // their maxima, and 3 to 4 times as many listed logits pass it).
  __device__ uint32_t rec_group(uint32_t b) const { return b < H ? 2u * b : 2u * (b - H) + 1u; }
  __device__ uint32_t wg_of(uint32_t g) const { return (g & 1u) ? H + (g >> 1) : g >> 1; }
  // topk_pick's group map: element j of group g is row j % 32 of the tile
  // j / 32 of workgroup wg_of(g)
  __device__ uint32_t size() const { return (A > B ? A : B) * kRowsTile; }
  __device__ uint32_t elem(uint32_t g, uint32_t j) const {
    const uint32_t b = wg_of(g);
    return j < ntiles(b) * kRowsTile ? tile(b, j / kRowsTile) * kRowsTile + j % kRowsTile : ~0u;
  }
  __device__ uint32_t count(uint32_t g, uint32_t vocab) const {
    const uint32_t b = wg_of(g);
    uint32_t n = 0;
    for (uint32_t q = 0; q < ntiles(b); ++q) {
      const uint32_t e0 = tile(b, q) * kRowsTile;
      n += e0 < vocab ? min(kRowsTile, vocab - e0) : 0u;
    }
    return n;
  }
};

// KS = 8 (one row group) splits the tiles unevenly (a wave takes all of its
// workgroup's tiles), 7 + 1 for the GEMV and 3 + 5 with the records (C4 with
// the selection: 26.68 us per step against 26.83 for 7 + 1 and 27.15 for
// 4 + 4); fewer k slices give every workgroup 4 tiles.
template <uint32_t KS, bool REC>
__host__ __device__ RowsSched rows_sched(uint32_t G) {
  const bool split = KS == 8u;
  const uint32_t a = kRowsTilesFirst[REC ? 1 : 0];
  return RowsSched{G, G / 2u, split ? a : kRowsTilesPair / 2u, split ? kRowsTilesPair - a : kRowsTilesPair / 2u};
}

// The selection's arguments for the head's top-k.
struct RowsPick {
  uint32_t *out;
  uint32_t m, n_penal, serial;
  RowsSched sched;   // the GEMV's tiles
  TopkPenal penal;
};

// LDS: the x region first (digits, 3 k bytes, then the group data, k bytes),
// so that its reads' offsets fit the 16-bit offset field of the LDS
// instructions; then the slice sums (kRowsRed) and the workgroup's outputs
// (4 bytes per row); then the 8 wave buffers.
__host__ __device__ constexpr uint32_t rows_tiles_at(uint32_t k) {
  return 4u * k + kRowsRed + 4u * kRowsTilesMax * kRowsTile;
}

// One lane's half row-block (128 weights): the tile row's ql/qh words `a`, `q`
// (aligned copies of LDS), its scale words and d, the block's byte shift, and
// the x digits and group data of block column j; acc += d * sum (w x).
__device__ __forceinline__ void rows_half_block(float &acc, const uint32_t (&a)[20], const uint32_t (&q)[12], uint2 sw,
                                                uint32_t sw2, uint2 dd, uint32_t sh, const uint8_t *xl,
                                                const int32_t *meta, uint32_t j, uint32_t n) {
  uint32_t QL[16], QH[8];
#pragma unroll
  for (int i = 0; i < 16; ++i) QL[i] = __builtin_amdgcn_alignbyte(a[i + 1], a[i], sh);
#pragma unroll
  for (int i = 0; i < 8; ++i) QH[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], sh);
  const uint32_t s0 = __builtin_amdgcn_alignbyte(sw.y, sw.x, sh);
  const uint32_t s1 = __builtin_amdgcn_alignbyte(sw2, sw.y, sh);
  const uint32_t dw = __builtin_amdgcn_alignbyte(dd.y, dd.x, sh);
  // this half's x: 8 runs of 16 from k = 256 j + 128 n; its 4 groups' data
  const uint8_t *dj = xl + (16u * j + 8u * n) * 48u;
  const int32_t *mj = meta + 8u * (8u * j + 4u * n);
  float accb = 0.f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int4 Ma = *(const int4 *)(mj + 8 * g);       // -32 T of values 0..15, p
    const int4 Mb = *(const int4 *)(mj + 8 * g + 4);   // -32 T of values 16..31
    float accg = 0.f;
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
      const int init[3] = {hh ? Mb.x : Ma.x, hh ? Mb.y : Ma.y, hh ? Mb.z : Ma.z};
      int D[3];
#pragma unroll
      for (int pp = 0; pp < 3; ++pp) {
        const u32x4 X = *(const u32x4 *)(dA + 16 * pp);
        int d = __builtin_amdgcn_sdot4((int)u[0], (int)X.x, init[pp], false);
        d = __builtin_amdgcn_sdot4((int)u[1], (int)X.y, d, false);
        d = __builtin_amdgcn_sdot4((int)u[2], (int)X.z, d, false);
        D[pp] = __builtin_amdgcn_sdot4((int)u[3], (int)X.w, d, false);
      }
      // sum (u - 32) digits, as sum over planes of 256^d D_d (|D_d| < 2^17)
      const float f = __builtin_fmaf((float)(D[2] * 256 + D[1]), 256.f, (float)D[0]);
      const float sc = (float)(int)__builtin_amdgcn_sbfe((int)(run < 4u ? s0 : s1), 8u * (run & 3u), 8);
      accg = __builtin_fmaf(sc, f, accg);
    }
    accb = __builtin_fmaf(__builtin_bit_cast(float, Ma.w), accg, accb);
  }
  acc = __builtin_fmaf(h2f(dw & 0xFFFFu), accb, acc);
}

// A lane's tile row into registers: ql/qh words of its half, its scale
// words and d (the tile row starts 16-byte aligned).
__device__ __forceinline__ void rows_read(const uint8_t *tp, uint32_t n, uint32_t (&a)[20], uint32_t (&q)[12],
                                          uint2 &sw, uint32_t &sw2, uint2 &dd) {
#pragma unroll
  for (uint32_t i = 0; i < 5; ++i) {
    const u32x4 v = *(const u32x4 *)(tp + 64u * n + 16u * i);
    a[4 * i] = v.x; a[4 * i + 1] = v.y; a[4 * i + 2] = v.z; a[4 * i + 3] = v.w;
  }
#pragma unroll
  for (uint32_t i = 0; i < 3; ++i) {
    const u32x4 v = *(const u32x4 *)(tp + 128u + 32u * n + 16u * i);
    q[4 * i] = v.x; q[4 * i + 1] = v.y; q[4 * i + 2] = v.z; q[4 * i + 3] = v.w;
  }
  // this half's 8 scales (bytes 192 + 8n ..) and d (bytes 208, 209)
  sw = *(const uint2 *)(tp + 192u + 8u * n);
  sw2 = *(const uint32_t *)(tp + 200u + 8u * n);
  dd = *(const uint2 *)(tp + 208u);
}

// REC: the decode head. Each workgroup also writes the top-k record of its
// tiles (their 4 largest logits, eff_topk.h), for k_rows_pick.
template <bool REC, uint32_t KS>
// amdgpu_waves_per_eu(4): at most 128 VGPRs, so that two workgroups share a CU.
__global__ __launch_bounds__(kRowsWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_gemv_rows_q6k(
    WeightView wv, const float *__restrict__ x, float *__restrict__ y, uint8_t *__restrict__ rec) {
  constexpr uint32_t RG = kRowsWaves / KS;                 // row groups
  const RowsSched sc = rows_sched<KS, REC>(gridDim.x);
  const uint32_t nt = sc.ntiles(blockIdx.x);               // the workgroup's tiles
  const uint32_t T = nt / RG;                              // tiles per wave
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t k = wv.k, bpr = wv.bpr, rows = wv.rows;
  uint8_t *const xl = lds;
  uint8_t *const tile = lds + rows_tiles_at(k) + wave * kRowsBuf;
  float *const red = (float *)(lds + 4u * k);                   // slice sums
  uint32_t *const fin = (uint32_t *)(lds + 4u * k + kRowsRed);   // the workgroup's outputs, for the record
  const uint32_t rg = wave / KS, ks = wave % KS;
  const uint32_t ncol = bpr > ks ? (bpr - ks + KS - 1u) / KS : 0u;   // block columns of this slice
  const rsrc_t src = make_rsrc(wv.w, wv.w_bytes);
  // first row of tile t of this wave (the workgroup's tile t RG + rg)
  auto tile_row = [&](uint32_t t) { return sc.tile(blockIdx.x, t * RG + rg) * kRowsTile; };

  // Load i of the lane fills LDS chunk s = 64 i + lane = row s / 15, chunk
  // s % 15 of that row; chunk 14 repeats 13 (a cache hit) so that rows are
  // 240 bytes apart; slots past the 32 rows repeat row 31. A tile row starts
  // at its block's 4-byte aligned byte. Block (r, j) starts at
  // B = (r bpr + j) 210, B mod 4 = 2 ((r bpr + j) mod 2); with tile rows
  // r = r0 + rsub (r0 even) and bpr even, B - B mod 4 = S + rsub bpr 210 for
  // S = (r0 bpr + j) 210 - 2 (j mod 2): a per-lane constant plus S.
  auto slot = [&](uint32_t i, uint32_t &rs, uint32_t &ch) {
    const uint32_t sl = 64u * i + lane, r = sl / 15u, c = sl - 15u * r;
    rs = min(r, kRowsTile - 1u);
    ch = r >= kRowsTile ? 0u : 16u * min(c, 13u);
  };
  uint32_t voff[8];
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) {
    uint32_t rs, ch;
    slot(i, rs, ch);
    voff[i] = rs * bpr * 210u + ch;
  }
  const bool even = (bpr & 1u) == 0u;
  auto issue = [&](uint32_t t, uint32_t j) {
    const uint32_t r0 = tile_row(t);
    if (even && r0 + kRowsTile <= rows) {
      const uint32_t S = (r0 * bpr + j) * 210u - 2u * (j & 1u);
#pragma unroll
      for (uint32_t i = 0; i < 8; ++i) dma16(src, tile + 1024u * i, S + voff[i], 0);
    } else {
      // odd block count or the matrix's last rows: each row's own start, rows clamped
#pragma unroll
      for (uint32_t i = 0; i < 8; ++i) {
        uint32_t rs, ch;
        slot(i, rs, ch);
        const uint32_t r = min(r0 + rs, rows - 1u);
        dma16(src, tile + 1024u * i, (((r * bpr + j) * 210u) & ~3u) + ch, 0);
      }
    }
  };
  if (ncol) issue(0u, ks);

  // x digits and group data of the whole k, once per workgroup
  int32_t *const meta = (int32_t *)(xl + 3u * k);
  for (uint32_t o = tid; o < k / 8u; o += kRowsWaves * 64u) {
    XOct v;
    x_load<1>(x, k, o, v);
    x_store_tsum(v, o, xl, meta);
  }
  __syncthreads();

  const uint32_t rr = lane & 31u, n = lane >> 5;
  const uint8_t *tp = tile + kRowsPitch * rr;         // this lane's tile row
#pragma unroll 1
  for (uint32_t t = 0; t < T; ++t) {
    float acc = 0.f;
    const uint32_t rowc = min(tile_row(t) + rr, rows - 1u);
    // block (rowc, j) starts sh = B mod 4 bytes past its row's copy in LDS
    const uint32_t par = even ? 0u : ((rowc * bpr) & 1u);
    for (uint32_t c = 0; c < ncol; ++c) {
      const uint32_t j = ks + KS * c;
      wait_vm<0>();   // this tile's loads (the only ones in flight)
      uint32_t a[20], q[12], sw2;
      uint2 sw, dd;
      rows_read(tp, n, a, q, sw, sw2, dd);
      // the tile is in registers: the buffer takes the next one
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
      {
        const bool last = c + 1u >= ncol;
        const uint32_t tn = last ? t + 1u : t;
        if (tn < T) issue(tn, last ? ks : j + KS);
      }
      rows_half_block(acc, a, q, sw, sw2, dd, 2u * ((par + j) & 1u), xl, meta, j, n);
    }
    // the two halves of a row; the slice sum of the row
    acc += __shfl_xor(acc, 32);
    if (n == 0u) red[((t * RG + rg) * KS + ks) * kRowsTile + rr] = acc;
  }
  // a row's KS slice sums in order
  __syncthreads();
  if (tid < nt * kRowsTile) {
    const uint32_t qt = tid / kRowsTile, r = tid % kRowsTile, row = sc.tile(blockIdx.x, qt) * kRowsTile + r;
    float v = red[qt * KS * kRowsTile + r];
#pragma unroll
    for (uint32_t s2 = 1; s2 < KS; ++s2) v += red[(qt * KS + s2) * kRowsTile + r];
    if (row < rows) y[row] = v;
    if constexpr (REC) fin[tid] = __builtin_bit_cast(uint32_t, v);
  }
  if constexpr (REC) {
    __syncthreads();
    if (wave == 0u) {
      // outputs l, l + 64, .. of the workgroup's 32 nt (tile i / 32, row i % 32)
      Top4 t;
      bool nan = false;
#pragma unroll
      for (uint32_t h = 0; h < (kRowsTilesMax * kRowsTile + 63u) / 64u; ++h) {
        const uint32_t i = lane + 64u * h;
        const uint32_t e = i < nt * kRowsTile ? sc.tile(blockIdx.x, i / kRowsTile) * kRowsTile + i % kRowsTile : ~0u;
        if (e < rows) {
          const uint32_t bits = fin[i];
          nan |= is_nan_bits(bits);
          t.add(composite(bits, e), bits);
        }
      }
      topk_record_wave(t, nan, rec, sc.rec_group(blockIdx.x), gridDim.x);
    }
  }
}

// The selection over the records a k_gemv_rows_q6k<true, KS> launch wrote,
// by 512 threads with R records each (topk_pick, eff_topk.h).
template <int R>
__global__ __launch_bounds__(kRowsWaves * 64) void k_rows_pick(const uint32_t *__restrict__ logits, uint32_t vocab,
                                                               RowsPick pk, uint32_t groups,
                                                               const uint8_t *__restrict__ rec) {
  __shared__ PickLds<kRowsWaves * 64, R> sh;
  topk_pick<kRowsWaves * 64, R>(logits, vocab, pk.m, pk.penal, pk.n_penal, pk.serial, pk.sched, groups, rec, pk.out,
                                sh);
}

template <bool REC, uint32_t KS>
hipError_t launch_rows_ks(const WeightView &wv, const float *x, float *y, uint8_t *rec, uint32_t lds, hipStream_t s) {
  static std::atomic<uint64_t> attr{0};
  const hipError_t e = lds_limit_once((const void *)k_gemv_rows_q6k<REC, KS>, (int)kMxMaxLds, attr);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gemv_rows_q6k<REC, KS>), dim3(gemv_rows_groups(wv)), dim3(kRowsWaves * 64), lds, s, wv, x, y,
                     rec);
  return hipGetLastError();
}

template <bool REC>
hipError_t launch_rows(const WeightView &wv, const float *x, float *y, uint8_t *rec, uint32_t lds, hipStream_t s) {
  // as many k slices as block columns, up to the 8 waves
  if (wv.bpr >= 8u) return launch_rows_ks<REC, 8>(wv, x, y, rec, lds, s);
  if (wv.bpr >= 4u) return launch_rows_ks<REC, 4>(wv, x, y, rec, lds, s);
  return launch_rows_ks<REC, 2>(wv, x, y, rec, lds, s);
}

}  // namespace

bool gemv_rows_applies(const WeightView &wv, uint32_t tokens) {
  return wv.type == Q6_K && tokens == 1u && wv.rows >= kRowsMin && wv.k <= kRowsMaxK && wv.bpr >= 2u &&
         (uint64_t)wv.rows * wv.row_bytes + 16u < (1ull << 32);   // 32-bit byte offsets
}

// an even count, for the two halves of the grid
uint32_t gemv_rows_groups(const WeightView &wv) { return ((wv.rows + 2u * kRowsPerWG - 1u) / (2u * kRowsPerWG)) * 2u; }

hipError_t launch_gemv_rows(const WeightView &wv, const float *x, float *y, hipStream_t s) {
  if (!gemv_rows_applies(wv, 1u)) return hipErrorInvalidValue;
  const uint32_t lds = rows_tiles_at(wv.k) + kRowsWaves * kRowsBuf;
  return launch_rows<false>(wv, x, y, nullptr, lds, s);
}

hipError_t launch_gemv_rows_topk(const WeightView &wv, const float *x, float *y, uint8_t *rec, uint32_t m,
                                 const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, uint32_t *out,
                                 hipStream_t s) {
  const uint32_t groups = gemv_rows_groups(wv);
  if (!gemv_rows_applies(wv, 1u) || groups > kRowsTopkGroupsMax || m == 0 || m > EFF_TOPK_M_MAX ||
      n_penal > EFF_TOPK_P_MAX || wv.rows >= EFF_TOPK_N_MAX)
    return hipErrorInvalidValue;
  RowsPick pk{};
  pk.out = out;
  pk.m = m;
  pk.n_penal = n_penal;
  pk.serial = serial;
  const uint32_t G = gemv_rows_groups(wv);
  pk.sched = wv.bpr >= 8u ? rows_sched<8, true>(G) : wv.bpr >= 4u ? rows_sched<4, true>(G) : rows_sched<2, true>(G);
  for (uint32_t i = 0; i < n_penal; ++i) pk.penal.ids[i] = penal_ids[i];
  hipError_t e = launch_rows<true>(wv, x, y, rec, rows_tiles_at(wv.k) + kRowsWaves * kRowsBuf, s);
  if (e != hipSuccess) return e;
  if (groups <= kRowsWaves * 64u)
    hipLaunchKernelGGL((k_rows_pick<1>), dim3(1), dim3(kRowsWaves * 64), 0, s, (const uint32_t *)y, wv.rows, pk,
                       groups, rec);
  else
    hipLaunchKernelGGL((k_rows_pick<2>), dim3(1), dim3(kRowsWaves * 64), 0, s, (const uint32_t *)y, wv.rows, pk,
                       groups, rec);
  return hipGetLastError();
}

}  // namespace eff
