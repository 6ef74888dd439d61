// Prefill GEMM for Q8_0 (and Q8_0R) weights from 64 tokens (at every token
// count below 6144 rows):
//   Y[t][row] = sum_k fp16(W[row][k]) fp16(X[t][k]), fp32 accumulation
// (the operand roundings of kernels.drift.wgsl.js:65-142 and the f16 tiles of
// ops.gemm2.js).
//
// A workgroup of 4 waves (one per SIMD) computes a BM-token x BN-row tile
// (64 x 128 to 256 x 256, chosen by an estimate of each one's time: big_plan); the
// waves are WM along tokens x 4 / WM along rows, each over (BM / WM / 32) x
// (BN / (4 / WM) / 32) fragments of v_mfma_f32_32x32x16_f16 (256
// accumulators for 256 x 256). Each A fragment is read once per k slot and
// used by the wave's row fragments of that slot, each B fragment by its
// token fragments.
//
// k steps of 64 (two Q8_0 blocks) flow through NS LDS stages (3 to 6)
// filled by direct-to-LDS loads (buffer_load ... lds), issued NS - 1 steps
// ahead:
//  * x: the fp16 x of the step (prepared by k_x_to_f16 as one contiguous run
//    of BM x 64 halves), 16-byte chunk c of token t stored at chunk
//    c ^ ((t >> 1) & 7) of the token's 128-byte row, so that the 16 lanes
//    one LDS cycle serves (16 x 16 bytes over the 64 banks) read 16
//    different bank quads when a fragment reads one chunk column;
//  * W: the raw bytes of each row's two blocks (68 bytes, read as five
//    16-byte chunks from the 4-byte aligned start), 80 bytes per row.
// The MFMA waves decode their weight fragments from the raw bytes in
// registers: the 8 quants of a lane are re-aligned with v_alignbyte, placed
// under a 0x64 byte (fp16 1024 + q + 128), offset by -1152 (exact) and
// multiplied by the block scale (one rounding: fp16(d * q), the value of the
// reference's f16 weight tiles).
//
// The k order inside an MFMA is free as long as both operands follow it:
// slot m (16 k) of a step takes, in lane half h, the 8 weights
// 16 h + 8 (m & 1) .. + 7 of block m / 2 of the step.
//
// Q8_0R (QR): the repacked tensor keeps the quants and the scales in two
// regions (kernels.bloques.wgsl.js:19-35), so a row's step is staged as its
// 64 quant bytes (four 16-byte chunks from the quant region, 16-byte aligned)
// and one chunk from the scale region holding its two scales: the same
// 80-byte LDS row, with the quants aligned and the scales at byte 64. The
// decoded weights, and so the outputs, are those of the Q8_0 tensor it was
// repacked from.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
#include "eff_formats.h"
#include "eff_kernels.h"

namespace eff {

namespace {

constexpr uint32_t kBK = 64;              // k per step
constexpr uint32_t kRB = 80;              // raw weight bytes per row and stage
constexpr uint32_t kNW = 4;               // waves per workgroup (one per SIMD)
constexpr uint32_t kCntBytes = kSliceCntBytes;   // the k-slice counters

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) { return *(const uint32_t *)p; }

// BM tokens x BN rows per tile. The 4 waves are WM along tokens x 4 / WM
// along rows; NS stages (3..6), loads issued NS - 1 steps ahead.
template <uint32_t BM, uint32_t BN, uint32_t WM, uint32_t NS, bool QR>
__global__ __launch_bounds__(kNW * 64) void k_gemm_q8(WeightView wv, const _Float16 *__restrict__ xh,
                                                 float *__restrict__ y, uint32_t tokens, uint32_t row_tiles,
                                                 uint32_t tok_tiles, uint32_t ksl, uint32_t per,
                                                 float *__restrict__ part, uint32_t *__restrict__ cnt) {
  constexpr uint32_t kWM = WM, kWN = kNW / WM;
  static_assert(kNW % WM == 0 && NS >= 3 && NS <= 6, "layout");
  constexpr uint32_t kWS = BN * kRB;                  // weight stage bytes
  constexpr uint32_t kWG = kWS / 1024;                // weight loads per step (64 lanes x 16 bytes each)
  constexpr uint32_t kFN = BN / 32 / kWN;             // 32 x 32 fragments along rows per wave
  constexpr uint32_t kWDma = (kWG + kNW - 1) / kNW;   // weight loads of a wave per step (at most)
  static_assert(kWS % 1024 == 0 && kFN >= 1, "whole loads");
  constexpr uint32_t kXS = BM * kBK * 2;   // x stage bytes
  constexpr uint32_t kXDma = kXS / 1024 / kNW;  // x loads per wave and step
  static_assert(kXS % (1024 * kNW) == 0, "x loads");
  constexpr uint32_t kFM = BM / 32 / kWM;
  // NS stages, each x (kXS bytes) then W (kWS bytes); separate objects,
  // so that the compiler can tell loads into one stage from reads of another
  // (every stage index below is a compile-time constant)
  constexpr uint32_t kSt = kXS + kWS;
  __shared__ __align__(16) uint8_t st0[kSt];
  __shared__ __align__(16) uint8_t st1[kSt];
  __shared__ __align__(16) uint8_t st2[kSt];
  __shared__ __align__(16) uint8_t st3[NS > 3 ? kSt : 16];
  __shared__ __align__(16) uint8_t st4[NS > 4 ? kSt : 16];
  __shared__ __align__(16) uint8_t st5[NS > 5 ? kSt : 16];
  auto stage = [&](uint32_t i) -> const uint8_t * {
    switch (i) {
      case 0: return st0;
      case 1: return st1;
      case 2: return st2;
      case 3: return st3;
      case 4: return st4;
      default: return st5;
    }
  };

  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = wave / kWN, wn = wave % kWN;

  // Workgroups are dealt so that those of one XCD (blockIdx % 8) take a
  // contiguous run of (k slice, tile) pairs, token tiles fastest and k slices
  // slowest: they share x and W slices through that XCD's L2.
  const uint32_t ntiles = row_tiles * tok_tiles, nwg = ntiles * ksl;
  uint32_t u = blockIdx.x;
  if (nwg % 8u == 0u) u = (blockIdx.x % 8u) * (nwg / 8u) + blockIdx.x / 8u;
  const uint32_t z = u / ntiles, lin = u - z * ntiles;
  const uint32_t n0 = (lin / tok_tiles) * BN, tt = lin % tok_tiles, t0 = tt * BM;
  const uint32_t rows = wv.rows, k = wv.k;
  // k slice z: steps s0 .. s0 + steps - 1 of 64 (every slice holds one at least)
  const uint32_t steps_all = (k + kBK - 1u) / kBK;
  const uint32_t s0 = z * per, steps = min(per, steps_all - s0), last = steps - 1u;

  // Sources: x run of this token tile from the slice's first step, weight
  // rows from the tile's first row (QR: the whole tensor, addressed by
  // absolute 32-bit offsets).
  const rsrc_t xsrc =
      make_rsrc(xh + ((uint64_t)tt * steps_all + s0) * (BM * kBK), (uint64_t)steps * kXS);
  const BufSrc src = make_src(wv, QR ? 0ull : (uint64_t)n0 * wv.bpr);
  const rsrc_t wsrc = QR ? make_rsrc(wv.w, wv.w_bytes) : src.q;
  const uint32_t rb = (uint32_t)wv.row_bytes;
  const uint32_t rmax = rows - 1u - n0;  // last valid row of the tile (rows past it repeat it)

  // Per-lane load offsets. x: load i of wave w fills the 1 KB slot
  // kXDma w + i, i.e. tokens t = 8 slot + lane / 8, stored chunk p = lane % 8,
  // holding x chunk c = p ^ ((t >> 1) & 7) = p ^ (4 (slot & 1) + lane / 16)
  // (kXDma is even, so slot & 1 = i & 1).
  static_assert(kXDma % 2 == 0, "x slot parity");
  const uint32_t xl0 = (lane >> 3) * 128u + (((lane & 7u) ^ (lane >> 4)) << 4);
  const uint32_t xl1 = (lane >> 3) * 128u + (((lane & 7u) ^ (4u + (lane >> 4))) << 4);
  // W: load j of wave w is load g = w + kNW j of the step (those with
  // g < kWG); its chunk q = 64 g + lane is chunk q % 5 of row q / 5.
  const uint32_t nwl = wave < kWG % kNW || kWG % kNW == 0 ? kWDma : kWDma - 1u;
  uint32_t wl[kWDma], ws_[kWDma];   // offset at step 0 and per step
#pragma unroll
  for (uint32_t j = 0; j < kWDma; ++j) {
    const uint32_t q = 64u * min(wave + kNW * j, kWG - 1u) + lane, r = q / 5u, c = q - 5u * r;
    const uint32_t row = n0 + min(r, rmax);
    if constexpr (QR) {
      // chunks 0..3: quants 32 (row bpr + 2 s) + 16 c; chunk 4: scales at
      // scales_off + 2 (row bpr + 2 s)
      ws_[j] = c < 4u ? 64u : 4u;
      wl[j] = (c < 4u ? 32u * row * wv.bpr + 16u * c : (uint32_t)wv.scales_off + 2u * row * wv.bpr) + s0 * ws_[j];
    } else {
      ws_[j] = 68u;
      wl[j] = (row - n0) * rb + 16u * c + s0 * 68u;
    }
  }
  // The loads of one step, in four groups (issued one per k slot, so that
  // the texture unit, shared by the CU's waves, is busy all step long).
  auto issue_group = [&](int g, uint32_t s, const uint8_t *xs, const uint8_t *ws) {
#pragma unroll
    for (uint32_t i = 0; i < kXDma + kWDma; ++i) {
      if ((int)(i % 4u) != g) continue;
      if (i < kXDma) {
        const uint32_t slot = kXDma * wave + i;
        dma16(xsrc, xs + 1024u * slot, ((i & 1u) ? xl1 : xl0) + 1024u * slot, s * kXS);
      } else {
        const uint32_t j = i - kXDma;
        if (j < nwl) {
          if constexpr (QR)
            dma16(wsrc, ws + 1024u * (wave + kNW * j), wl[j] + s * ws_[j], 0u);
          else
            dma16(wsrc, ws + 1024u * (wave + kNW * j), wl[j], s * 68u);
        }
      }
    }
  };
  // wait until this wave's loads of the oldest step in flight are complete
  // (those of the NS - 2 later steps may be outstanding)
  auto wait_prev = [&]() {
    if (kWG % kNW == 0 || nwl == kWDma)
      wait_vm<(NS - 2u) * (kXDma + kWDma)>();
    else
      wait_vm<(NS - 2u) * (kXDma + kWDma - 1u)>();
  };
  auto issue = [&](uint32_t s, const uint8_t *xs, const uint8_t *ws) {
#pragma unroll
    for (int g = 0; g < 4; ++g) issue_group(g, s, xs, ws);
  };

  // Fragment geometry. A: token 128 wm + 32 fi + n, chunk (2 m + h) stored
  // at ((2 m + h) ^ ((n >> 1) & 7)); B: row 128 wn + 32 fj + n.
  const uint32_t n = lane & 31u, h = lane >> 5;
  const uint32_t abase = (kFM * 32u * wm + n) * 128u;
  uint32_t acol[4];
#pragma unroll
  for (uint32_t m = 0; m < 4; ++m) acol[m] = ((4u * (m >> 1) + 2u * h + (m & 1u)) ^ ((n >> 1) & 7u)) << 4;
  const uint32_t brow = (kFN * 32u * wn + n) * kRB;

  float16v acc[kFM][kFN];
#pragma unroll
  for (int i = 0; i < (int)kFM; ++i)
#pragma unroll
    for (int j = 0; j < (int)kFN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  const half2v off = {(_Float16)-1152.0f, (_Float16)-1152.0f};

  // Operands. Slot m takes, in lane half h, the weights 16 h + 8 (m & 1) ..
  // + 7 of block m / 2 (and the same k of x). A fragments come from the x
  // stage; the B fragments of both slots of block u are decoded from the
  // two 16-byte chunks at byte 32 u + 16 h of the row (read whole: 16-byte
  // reads of 8 rows hit 8 different bank groups, as the 80-byte row stride
  // is 5 chunks), in which the lane's 16 quants start 2 + 2 u bytes in
  // (re-aligned with v_alignbyte, which shifts by 0..3 bytes, for block 0).
  auto load_a = [&](const uint8_t *xs, int m, half8 *a) {
#pragma unroll
    for (int fi = 0; fi < (int)kFM; ++fi) a[fi] = *(const half8 *)(xs + abase + fi * 4096u + acol[m]);
  };
  auto load_b = [&](const uint8_t *ws, int u, uint32_t (*q)[4]) {
#pragma unroll
    for (int fj = 0; fj < (int)kFN; ++fj) {
      const uint8_t *rp = ws + brow + fj * (32u * kRB) + 32u * (uint32_t)u + 16u * h;
      if constexpr (QR) {   // the lane's 16 quants, aligned
        const u32x4 c = *(const u32x4 *)rp;
        q[fj][0] = c.x; q[fj][1] = c.y; q[fj][2] = c.z; q[fj][3] = c.w;
        continue;
      }
      const u32x4 c0 = *(const u32x4 *)rp, c1 = *(const u32x4 *)(rp + 16);
      if (u == 0) {
        q[fj][0] = __builtin_amdgcn_alignbyte(c0.y, c0.x, 2);
        q[fj][1] = __builtin_amdgcn_alignbyte(c0.z, c0.y, 2);
        q[fj][2] = __builtin_amdgcn_alignbyte(c0.w, c0.z, 2);
        q[fj][3] = __builtin_amdgcn_alignbyte(c1.x, c0.w, 2);
      } else {
        q[fj][0] = c0.y; q[fj][1] = c0.z; q[fj][2] = c0.w; q[fj][3] = c1.x;
      }
    }
  };
  // quants q0, q1 (8 signed bytes) -> fp16(d * q)
  auto decode8 = [&](uint32_t q0, uint32_t q1, half2v d) {
    q0 ^= 0x80808080u;
    q1 ^= 0x80808080u;
    const half2v e0 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q0, 0x04010400u));
    const half2v e1 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q0, 0x04030402u));
    const half2v e2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q1, 0x04010400u));
    const half2v e3 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q1, 0x04030402u));
    const half2v v0 = (e0 + off) * d, v1 = (e1 + off) * d, v2 = (e2 + off) * d, v3 = (e3 + off) * d;
    return half8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
  };

  // Block scales of the lane's rows in stage ws: byte 0 (block 0) and byte
  // 34 (block 1); `full` is false on a last step holding one block only
  // (k % 64 == 32): the second block's weights are then zero.
  half2v d0[kFN], d1[kFN];
  auto scales = [&](const uint8_t *ws, bool full) {
#pragma unroll
    for (int fj = 0; fj < (int)kFN; ++fj) {
      const uint8_t *rp = ws + brow + fj * (32u * kRB);
      // Q8_0: the scales at bytes 0 and 34 (read as the dwords at 0 and 32);
      // Q8_0R: both in the dword at 64
      const uint32_t w0 = lds_u32(rp + (QR ? 64u : 0u)), w1 = QR ? w0 : lds_u32(rp + 32);
      const _Float16 s0 = __builtin_bit_cast(_Float16, (uint16_t)(w0 & 0xFFFFu));
      const _Float16 s1 = full ? __builtin_bit_cast(_Float16, (uint16_t)(w1 >> 16)) : (_Float16)0.0f;
      d0[fj] = half2v{s0, s0};
      d1[fj] = half2v{s1, s1};
    }
  };
  half8 a[2][kFM], bb[2][2][kFN];   // A per slot; B per block (both slots)
  uint32_t q[kFN][4];
  // operands of slot m (from stage st): A, and for an even slot the B of its block
  auto operands = [&](const uint8_t *st, int m) {
    load_a(st, m, a[m & 1]);
    if ((m & 1) == 0) {
      const int u = m >> 1;
      load_b(st + kXS, u, q);
#pragma unroll
      for (int fj = 0; fj < (int)kFN; ++fj) {
        const half2v d = u == 0 ? d0[fj] : d1[fj];
        bb[u][0][fj] = decode8(q[fj][0], q[fj][1], d);
        bb[u][1][fj] = decode8(q[fj][2], q[fj][3], d);
      }
    }
  };

  // the last step of k (in the last slice) holds one block
  const bool tail_half = (k % kBK) != 0u && z + 1u == ksl;
  // Step s computes from stage s % NS; the operands of slot m + 1 are read
  // and decoded while the MFMAs of slot m run, and the loads of step
  // s + NS - 1 go to stage tgt (the one step s - 1 read) in four groups.
  // Before the last slot's MFMAs, the wave waits for its loads of step s + 1
  // (those of steps s + 2 .. s + NS - 1 may still be outstanding) and meets
  // the others at a barrier: stage nxt is then complete, and every wave is
  // done reading stage cur, which the loads issued during step s + 1
  // overwrite. Slot 0 of step s + 1 is then prepared during the last MFMAs
  // of step s. Past the last step the loads repeat it into stages no step
  // reads any more, so every step issues the same number of loads.
  auto step = [&](uint32_t s, const uint8_t *cur, const uint8_t *nxt, const uint8_t *tgt) {
    const uint32_t sn = min(s + NS - 1u, last);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      issue_group(m, sn, tgt, tgt + kXS);
      if (m < 3) {
        operands(cur, m + 1);
      } else {
        wait_prev();
        __builtin_amdgcn_s_barrier();
        scales(nxt + kXS, !(tail_half && s + 1u == last));
        operands(nxt, 0);
      }
#pragma unroll
      for (int fi = 0; fi < (int)kFM; ++fi)
#pragma unroll
        for (int fj = 0; fj < (int)kFN; ++fj)
          acc[fi][fj] =
              __builtin_amdgcn_mfma_f32_32x32x16_f16(a[m & 1][fi], bb[m >> 1][m & 1][fj], acc[fi][fj], 0, 0, 0);
      // schedule: the next slot's LDS reads first, three MFMAs while they
      // land, then the decode of the next block (odd m) interleaved with
      // the remaining MFMAs
      if (m == 3)
        __builtin_amdgcn_sched_group_barrier(0x100, kFM + 4 * kFN, 0);  // A, B and next scales
      else if (m == 1)
        __builtin_amdgcn_sched_group_barrier(0x100, kFM + 2 * kFN, 0);  // A and B
      else
        __builtin_amdgcn_sched_group_barrier(0x100, kFM, 0);            // A
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);                // 3 MFMA
#pragma unroll
      for (int i = 0; i < (int)(kFM * kFN) - 3; ++i) {
        if (m & 1)
          __builtin_amdgcn_sched_group_barrier(0x002, (34 * kFN + kFM * kFN - 4) / (kFM * kFN - 3), 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                            // 1 MFMA
      }
    }
  };

#pragma unroll
  for (uint32_t j = 0; j + 1u < NS; ++j) issue(min(j, last), stage(j), stage(j) + kXS);
  wait_prev();
  __builtin_amdgcn_s_barrier();
  scales(st0 + kXS, !(tail_half && last == 0u));
  operands(st0, 0);
  // NS steps per iteration, so that the stages are fixed objects; the last
  // steps after the loop (no branch inside the loop: the accumulators stay
  // in place). After the last step, the reads of a following step see stale
  // stage contents and are not used.
  uint32_t s = 0;
  for (; s + NS <= steps; s += NS) {
#pragma unroll
    for (uint32_t j = 0; j < NS; ++j) step(s + j, stage(j), stage((j + 1u) % NS), stage((j + NS - 1u) % NS));
  }
#pragma unroll
  for (uint32_t j = 0; j + 1u < NS; ++j)
    if (s + j < steps) step(s + j, stage(j), stage((j + 1u) % NS), stage((j + NS - 1u) % NS));
  wait_vm<0>();

  // D[tok][row]: lane holds row (column) n of each fragment and tokens
  // 8 (v / 4) + 4 h + v % 4. The lane number is read again here (an asm
  // statement the compiler cannot merge with the first read), so that n, h
  // and the thread index are not held across the main loop: at 256 x 256
  // every register is in use there, and they would be spilled to scratch.
  uint32_t lane_e;
  __asm__ volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
  const uint32_t ne = lane_e & 31u, he = lane_e >> 5;
  // outputs v = 4 q .. 4 q + 3 of fragment (fi, fj)
  auto put = [&](int fi, int fj, int q, float4 v) {
    const uint32_t row = n0 + kFN * 32u * wn + 32u * (uint32_t)fj + ne;
    const uint32_t tok = t0 + kFM * 32u * wm + 32u * (uint32_t)fi + 8u * (uint32_t)q + 4u * he;
    if (row >= rows) return;
    if (tok < tokens) y[(uint64_t)tok * rows + row] = v.x;
    if (tok + 1u < tokens) y[(uint64_t)(tok + 1u) * rows + row] = v.y;
    if (tok + 2u < tokens) y[(uint64_t)(tok + 2u) * rows + row] = v.z;
    if (tok + 3u < tokens) y[(uint64_t)(tok + 3u) * rows + row] = v.w;
  };
  auto mine = [&](int fi, int fj, int q) {
    return make_float4(acc[fi][fj][4 * q], acc[fi][fj][4 * q + 1], acc[fi][fj][4 * q + 2], acc[fi][fj][4 * q + 3]);
  };
  // (256 x 256 tiles take no k slices: their sums would not fit the
  // registers beside the accumulators)
  if (BM * BN < 256u * 256u && ksl > 1u) {
    // k slices: each workgroup of the tile stores its sums (in its register
    // layout, 16 bytes per lane and store); the last of the tile's ksl
    // workgroups to arrive adds the slices in slice order, ((s0 + s1) + s2)
    // ..., which does not depend on the order of arrival, writes y, and
    // resets the tile's counter to zero for the next launch. The sums are
    // stored and loaded with the sc1 cache policy (as device-scope atomics
    // are), which the XCDs' L2 caches do not hold stale, and each wave waits
    // for its stores to complete before the barrier that precedes the
    // counter's increment: no fence, whose L2 write-back and invalidation
    // would take the cached x and W from the workgroups still running.
    constexpr int kSc1 = 16;   // cache policy bit 4: sc1
    const uint32_t tid_e = wave * 64u + lane_e;
    const rsrc_t prs = make_rsrc(part + (uint64_t)lin * ksl * (BM * BN), (uint64_t)ksl * (BM * BN * 4u));
    auto off = [&](uint32_t zz, int fi, int fj, int q) {
      return (int)(zz * (BM * BN * 4u) + ((((uint32_t)fi * kFN + fj) * 4u + q) * (kNW * 64u) + tid_e) * 16u);
    };
#pragma unroll
    for (int fi = 0; fi < (int)kFM; ++fi)
#pragma unroll
      for (int fj = 0; fj < (int)kFN; ++fj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 v = {__float_as_uint(acc[fi][fj][4 * q]), __float_as_uint(acc[fi][fj][4 * q + 1]),
                           __float_as_uint(acc[fi][fj][4 * q + 2]), __float_as_uint(acc[fi][fj][4 * q + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, prs, off(z, fi, fj, q), 0, kSc1);
        }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();   // every wave is past its loads and LDS reads: st0 is free
    if (tid_e == 0u)
      *(uint32_t *)st0 = __hip_atomic_fetch_add(cnt + lin, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*(const uint32_t *)st0 != ksl - 1u) return;
    if (tid_e == 0u) __hip_atomic_store(cnt + lin, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // a slice at a time (its own included, complete in memory), its loads
    // in flight together, added onto the accumulators
#pragma unroll
    for (int fi = 0; fi < (int)kFM; ++fi)
#pragma unroll
      for (int fj = 0; fj < (int)kFN; ++fj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(prs, off(0u, fi, fj, q), 0, kSc1);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[fi][fj][4 * q + c] = __uint_as_float(v[c]);
        }
    for (uint32_t zz = 1; zz < ksl; ++zz) {
#pragma unroll
      for (int fi = 0; fi < (int)kFM; ++fi)
#pragma unroll
        for (int fj = 0; fj < (int)kFN; ++fj)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(prs, off(zz, fi, fj, q), 0, kSc1);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[fi][fj][4 * q + c] += __uint_as_float(v[c]);
          }
    }
  }
#pragma unroll
  for (int fi = 0; fi < (int)kFM; ++fi)
#pragma unroll
    for (int fj = 0; fj < (int)kFN; ++fj)
#pragma unroll
      for (int q = 0; q < 4; ++q) put(fi, fj, q, mine(fi, fj, q));
}


template <uint32_t BM, uint32_t BN, uint32_t WM, uint32_t NS>
hipError_t gemm_q8_go(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, uint32_t ksl, uint32_t per,
                      void *scratch, hipStream_t s) {
  const uint32_t tok_tiles = (tokens + BM - 1) / BM, row_tiles = (wv.rows + BN - 1) / BN;
  // Q8_0R is addressed from the tensor's first byte with 32-bit offsets: its
  // quant and scale regions must end below 4 GiB (so does any tensor a buffer
  // descriptor covers)
  if (wv.type == Q8_0R && wv.scales_off + 2ull * wv.rows * wv.bpr + 16u >= (1ull << 32)) return hipErrorInvalidValue;
  if (ksl > 1u && (!scratch || (uint64_t)tok_tiles * row_tiles > kCntBytes / 4u)) return hipErrorInvalidValue;
  // scratch: the tiles' arrival counters, then the slices' sums
  uint32_t *cnt = (uint32_t *)scratch;
  float *part = scratch ? (float *)((uint8_t *)scratch + kCntBytes) : nullptr;
  const dim3 grid(row_tiles * tok_tiles * ksl);
  if (wv.type == Q8_0R)
    hipLaunchKernelGGL((k_gemm_q8<BM, BN, WM, NS, true>), grid, dim3(kNW * 64), 0, s, wv, xh, y, tokens, row_tiles,
                       tok_tiles, ksl, per, part, cnt);
  else
    hipLaunchKernelGGL((k_gemm_q8<BM, BN, WM, NS, false>), grid, dim3(kNW * 64), 0, s, wv, xh, y, tokens, row_tiles,
                       tok_tiles, ksl, per, part, cnt);
  return hipGetLastError();
}

// Tile configurations (tokens x rows per workgroup, waves along tokens, LDS
// stages): 1: 256 x 256, 1, 3; 2: 128 x 128, 1, 3; 3: 128 x 128, 1, 6;
// 4: 64 x 128, 1, 4; 5: 128 x 256, 1, 4; 6: 256 x 128, 2, 3. Configurations
// 2 and 4 fit two workgroups per CU, the others one.
uint32_t cfg_bm(uint32_t c) { return c == 1u || c == 6u ? 256u : c == 4u ? 64u : 128u; }
uint32_t cfg_bn(uint32_t c) { return c == 1u || c == 5u ? 256u : 128u; }

uint32_t cfg_tiles(uint32_t c, uint32_t plan, uint32_t rows) {
  return ((plan + cfg_bm(c) - 1u) / cfg_bm(c)) * ((rows + cfg_bn(c) - 1u) / cfg_bn(c));
}

// k slices for t tiles of configuration c: none from 192 tiles, else about
// 256 workgroups in all with slices of 8 steps at least; 256 x 256 tiles take
// none (their slices' sums do not fit the registers beside the 256
// accumulators: 2048 x 8192, 2048 tokens, us: in 4 slices 290, 128 x 128
// unsliced 111). 2048 x 8192, us against unsliced: 129 tokens 25.9 / 68.4,
// 256 29.1 / 68.1, 512 44.2 / 85.5, 1024 66.0 / 95.5.
uint32_t cfg_slices(uint32_t c, uint32_t t, uint32_t steps) {
  return c != 1u && t < 192u ? min((256u + t / 2u) / t, max(steps / 8u, 1u)) : 1u;
}

// Estimated us of one launch of configuration c in ksl slices. A CU holds
// n = ceil(workgroups / 256) of them; a workgroup's time is linear in its k
// steps, alone on its CU or, where two fit, as a pair. The coefficients are a
// least-squares fit (8% rms error) to 1,100 timed launches: every
// configuration and slice count at 15 shapes from 1024 x 4096 to 65536 x 2048
// and 64 to 2048 tokens. Choosing by it, against the token-count rule it
// replaces (us with the x conversion): 65536 x 2048 at 256 / 512 tokens
// 139 / 229 -> 85 / 158, 14336 x 4096 at 256 / 1024 65 / 167 -> 53 / 134,
// 8192 x 8192 at 256 72 -> 61; 0.6% above the best configuration of each
// shape summed over the sweep (measured again with this choice), the rule
// 11.5%.
double cfg_cost(uint32_t c, uint32_t plan, uint32_t rows, uint32_t steps, uint32_t ksl) {
  static const double one[7][2] = {{0, 0}, {22.9, 1.47}, {6.85, 0.686}, {7.73, 0.643},
                                   {3.46, 0.534}, {13.5, 1.04}, {13.2, 1.01}};
  static const double two[7][2] = {{0, 0}, {0, 0}, {6.76, 1.19}, {0, 0}, {3.23, 0.871}, {0, 0}, {0, 0}};
  const uint32_t per = (steps + ksl - 1u) / ksl;
  ksl = (steps + per - 1u) / per;
  const uint64_t n = ((uint64_t)cfg_tiles(c, plan, rows) * ksl + 255u) / 256u;
  const double single = one[c][0] + one[c][1] * per;
  double t = two[c][0] > 0 ? (double)(n / 2u) * (two[c][0] + two[c][1] * per) + (double)(n % 2u) * single
                           : (double)n * single;
  if (ksl > 1u) t += 6.2 + 2.15e-6 * plan * rows * (ksl - 1u);
  return t;
}

struct BigPlan {
  uint32_t cfg, ksl, per;
};

// The automatic configuration is the one of least estimated time, with its
// slices; the slice count follows the automatic choice also under a forced
// configuration, so that every configuration sums each output in the same
// order (the same bits).
BigPlan big_plan(uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg, uint32_t ksl_opt) {
  const uint32_t steps = (k + kBK - 1u) / kBK;
  uint32_t c = 0u, ksl_auto = 1u;
  double best = 0;
  for (uint32_t i = 1u; i <= 6u; ++i) {
    const uint32_t sl = cfg_slices(i, cfg_tiles(i, plan, rows), steps);
    const double t = cfg_cost(i, plan, rows, steps, sl);
    if (c == 0u || t < best) c = i, best = t, ksl_auto = sl;
  }
  BigPlan b;
  b.cfg = cfg >= 1u && cfg <= 6u ? cfg : c;
  // 256 x 256 tiles take no k slices: where the automatic choice slices k
  // they run 128 x 128, and a forced slice count leaves them whole (the
  // tiles, and so the x layout, do not depend on the forced count)
  if (b.cfg == 1u && ksl_auto > 1u) b.cfg = 2u;
  const uint32_t ksl = b.cfg == 1u ? 1u : max(1u, min(ksl_opt ? ksl_opt : ksl_auto, steps));
  b.per = (steps + ksl - 1u) / ksl;
  b.ksl = (steps + b.per - 1u) / b.per;
  return b;
}

}  // namespace

// From the GEMM's threshold (64 tokens) at every row count, and at any token
// count below 6144 rows (where the general kernel's 32-row tiles are fewer
// than 192 workgroups). With the tiles and k slices of big_plan this kernel is
// the faster from 64 tokens (us, 64 / 128 tokens, general kernel against this
// one: 8192 x 2048 22.2 / 22.7 against 16.9 / 18.9, 14336 x 4096 60.9 / 62.2
// against 28.9 / 40.9, 65536 x 2048 140.5 / 144.5 against 48.6 / 60.6, 8192 x
// 8192 54.8 / 56.1 against 31.3 / 40.2; below 6144 rows: 2048 x 8192 54.3 /
// 54.8 against 22.5 / 22.3, 4096 x 14336 86.0 / 86.6 against 31.0 / 42.4).
// Before big_plan estimated each configuration's time, the general kernel's
// one 128-token tile was as fast up to 128 tokens at 8192 x 2048 (21.5 / 22.0
// against 22.8 / 22.5), and this kernel took over only from 129 there.
bool gemm_big_applies(int type, uint32_t tokens, uint32_t k, uint32_t rows) {
  return (type == Q8_0 || type == Q8_0R) && (tokens >= 64u || (rows + 31u) / 32u < 192u) && k % 32u == 0;
}

uint32_t gemm_big_tile_log2(uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg) {
  switch (big_plan(plan, k, rows, cfg, 0u).cfg) {
    case 1: case 6: return 8u;
    case 4: return 6u;
    default: return 7u;
  }
}

size_t gemm_big_scratch_bytes(uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg,
                              uint32_t ksl_opt) {
  const BigPlan b = big_plan(plan, k, rows, cfg, ksl_opt);
  if (b.ksl < 2u) return 0;
  const uint32_t bm = cfg_bm(b.cfg), bn = cfg_bn(b.cfg);
  const uint64_t tiles = (uint64_t)((tokens + bm - 1u) / bm) * ((rows + bn - 1u) / bn);
  return kCntBytes + (size_t)(tiles * b.ksl * bm * bn * 4u);
}

hipError_t launch_gemm_big(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, uint32_t plan,
                           uint32_t cfg, uint32_t ksl_opt, void *scratch, hipStream_t s) {
  const BigPlan b = big_plan(plan, wv.k, wv.rows, cfg, ksl_opt);
  switch (b.cfg) {
    case 1: return gemm_q8_go<256, 256, 1, 3>(wv, xh, y, tokens, b.ksl, b.per, scratch, s);
    case 2: return gemm_q8_go<128, 128, 1, 3>(wv, xh, y, tokens, b.ksl, b.per, scratch, s);
    case 3: return gemm_q8_go<128, 128, 1, 6>(wv, xh, y, tokens, b.ksl, b.per, scratch, s);
    case 4: return gemm_q8_go<64, 128, 1, 4>(wv, xh, y, tokens, b.ksl, b.per, scratch, s);
    case 5: return gemm_q8_go<128, 256, 1, 4>(wv, xh, y, tokens, b.ksl, b.per, scratch, s);
    case 6: return gemm_q8_go<256, 128, 2, 3>(wv, xh, y, tokens, b.ksl, b.per, scratch, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace eff
