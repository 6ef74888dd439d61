// Prefill GEMM for Q8_0 weights at >= 1024 tokens:
//   Y[t][row] = sum_k fp16(W[row][k]) fp16(X[t][k]), fp32 accumulation
// (the operand roundings of kernels.drift.wgsl.js:65-142 and the f16 tiles of
// ops.gemm2.js).
//
// A workgroup of 4 waves computes a 256-token x 256-row tile; wave (wm, wn)
// owns tokens 128 wm.. and rows 128 wn.., i.e. 4 x 4 fragments of
// v_mfma_f32_32x32x16_f16 (256 accumulators). Each fragment operand is read
// once per k slot and used by 4 MFMAs, which keeps the LDS traffic per MFMA
// at a level the LDS can sustain (about 128 bytes per clock per CU).
//
// k steps of 64 (two Q8_0 blocks) flow through three LDS stages filled by
// direct-to-LDS loads (buffer_load ... lds), issued two steps ahead:
//  * x: the fp16 x of the step (prepared by k_x_to_f16 as one contiguous run
//    of 256 x 64 halves), 16-byte chunk c of token t stored at chunk
//    c ^ (t & 7) of the token's 128-byte row, so that the 32 tokens of a
//    fragment read one chunk column without bank conflicts;
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
// 16 m + 8 h .. 16 m + 8 h + 7 of the step (block m / 2).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
#include "eff_formats.h"
#include "eff_kernels.h"

namespace eff {

namespace {

constexpr uint32_t kBM = 256, kBN = 256, kBK = 64;
constexpr uint32_t kXS = kBM * kBK * 2;   // x stage bytes (32 KB)
constexpr uint32_t kRB = 80;              // raw weight bytes per row and stage
constexpr uint32_t kWS = kBN * kRB;       // weight stage bytes (20 KB)
constexpr uint32_t kXDma = kXS / 4096;    // x loads per wave and step (64 lanes x 16 bytes)
constexpr uint32_t kWDma = kWS / 4096;    // weight loads per wave and step
constexpr uint32_t kDma = kXDma + kWDma;  // all loads per wave and step
// waves along tokens x along rows, and 32 x 32 fragments per wave
constexpr uint32_t kWM = 1, kWN = 4, kFM = kBM / 32 / kWM, kFN = kBN / 32 / kWN;
static_assert(kWS % 4096 == 0 && kXS % 4096 == 0, "whole loads per wave");

// 16 bytes per lane from the buffer (voffset + soffset) into LDS at
// lds + 16 * lane. Written as inline assembly so that the compiler, which
// cannot tell the stages' loads and reads apart, adds no vmcnt(0) before the
// reads of the other stages; the waits are explicit (wait_vm).
__device__ __forceinline__ void dma16(rsrc_t r, const uint8_t *lds, uint32_t voff, uint32_t soff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <uint32_t N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((int)((N & 15u) | ((N >> 4) << 14) | 0x0F70u));
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) { return *(const uint32_t *)p; }

__global__ __launch_bounds__(256) void k_gemm_q8(WeightView wv, const _Float16 *__restrict__ xh,
                                                 float *__restrict__ y, uint32_t tokens, uint32_t row_tiles,
                                                 uint32_t tok_tiles) {
  // three stages, each x (kXS bytes) then W (kWS bytes); separate objects,
  // so that the compiler can tell loads into one stage from reads of another
  __shared__ __align__(16) uint8_t st0[kXS + kWS];
  __shared__ __align__(16) uint8_t st1[kXS + kWS];
  __shared__ __align__(16) uint8_t st2[kXS + kWS];

  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = wave / kWN, wn = wave % kWN;

  // Tiles are dealt so that the workgroups of one XCD (blockIdx % 8) take a
  // contiguous run of tiles, token tiles fastest: they share x and W slices
  // through that XCD's L2.
  const uint32_t ntiles = row_tiles * tok_tiles;
  uint32_t lin = blockIdx.x;
  if (ntiles % 8u == 0u) lin = (blockIdx.x % 8u) * (ntiles / 8u) + blockIdx.x / 8u;
  const uint32_t n0 = (lin / tok_tiles) * kBN, tt = lin % tok_tiles, t0 = tt * kBM;
  const uint32_t rows = wv.rows, k = wv.k;
  const uint32_t steps = (k + kBK - 1u) / kBK, last = steps - 1u;

  // Sources: x run of this token tile, weight rows from the tile's first row.
  const rsrc_t xsrc = make_rsrc(xh + (uint64_t)tt * steps * (kBM * kBK), (uint64_t)steps * kXS);
  const BufSrc src = make_src(wv, (uint64_t)n0 * wv.bpr);
  const uint32_t rb = (uint32_t)wv.row_bytes;
  const uint32_t rmax = rows - 1u - n0;  // last valid row of the tile (rows past it repeat it)

  // Per-lane load offsets. x: load j of wave w fills chunk slots
  // 64 (8 w + j) + lane = 8 t + p of the stage, token t, stored chunk p,
  // holding x chunk c = p ^ (t & 7) (t & 7 = lane >> 3 here).
  const uint32_t xl = (lane >> 3) * 128u + (((lane & 7u) ^ (lane >> 3)) << 4);
  // W: chunk q = 64 (5 w + j) + lane is chunk q % 5 of row q / 5.
  uint32_t wl[kWDma];
#pragma unroll
  for (uint32_t j = 0; j < kWDma; ++j) {
    const uint32_t q = 64u * (kWDma * wave + j) + lane, r = q / 5u;
    wl[j] = min(r, rmax) * rb + 16u * (q - 5u * r);
  }
  // The loads of one step, in four groups (issued one per k slot, so that
  // the texture unit, shared by the CU's waves, is busy all step long).
  auto issue_group = [&](int g, uint32_t s, const uint8_t *xs, const uint8_t *ws) {
#pragma unroll
    for (uint32_t i = 0; i < kDma; ++i) {
      if ((int)(i % 4u) != g) continue;
      if (i < kXDma) {
        const uint32_t slot = kXDma * wave + i;
        dma16(xsrc, xs + 1024u * slot, xl + 1024u * slot, s * kXS);
      } else {
        const uint32_t j = i - kXDma;
        dma16(src.q, ws + 1024u * (kWDma * wave + j), wl[j], s * 68u);
      }
    }
  };
  auto issue = [&](uint32_t s, const uint8_t *xs, const uint8_t *ws) {
#pragma unroll
    for (int g = 0; g < 4; ++g) issue_group(g, s, xs, ws);
  };

  // Fragment geometry. A: token 128 wm + 32 fi + n, chunk (2 m + h) stored
  // at ((2 m + h) ^ (n & 7)); B: row 128 wn + 32 fj + n.
  const uint32_t n = lane & 31u, h = lane >> 5;
  const uint32_t abase = (kFM * 32u * wm + n) * 128u;
  uint32_t acol[4];
#pragma unroll
  for (uint32_t m = 0; m < 4; ++m) acol[m] = ((2u * m + h) ^ (n & 7u)) << 4;
  const uint32_t bbase = (kFN * 32u * wn + n) * kRB + 8u * h;

  float16v acc[kFM][kFN];
#pragma unroll
  for (int i = 0; i < (int)kFM; ++i)
#pragma unroll
    for (int j = 0; j < (int)kFN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  const half2v off = {(_Float16)-1152.0f, (_Float16)-1152.0f};

  // Operands of k slot m: A fragments from the x stage, B fragments decoded
  // from the raw weights (quants of block m / 2 at bytes 34 (m/2) + 2 +
  // 16 (m&1) + 8 h of the row: 2 past a multiple of 8 for block 0, re-aligned
  // with v_alignbyte, which shifts by 0..3 bytes; on a 4-byte boundary for
  // block 1).
  auto load_a = [&](const uint8_t *xs, int m, half8 *a) {
#pragma unroll
    for (int fi = 0; fi < (int)kFM; ++fi) a[fi] = *(const half8 *)(xs + abase + fi * 4096u + acol[m]);
  };
  auto load_b = [&](const uint8_t *ws, int m, uint32_t (*q)[2]) {
    const uint32_t c0 = 34u * (uint32_t)(m >> 1) + 2u + 16u * (uint32_t)(m & 1);
#pragma unroll
    for (int fj = 0; fj < (int)kFN; ++fj) {
      const uint8_t *rp = ws + bbase + fj * (32u * kRB);
      if ((m >> 1) == 0) {
        const uint2 lo = *(const uint2 *)(rp + (c0 & ~7u));
        const uint32_t hi = lds_u32(rp + (c0 & ~7u) + 8u);
        q[fj][0] = __builtin_amdgcn_alignbyte(lo.y, lo.x, c0 & 3u);
        q[fj][1] = __builtin_amdgcn_alignbyte(hi, lo.y, c0 & 3u);
      } else {
        q[fj][0] = lds_u32(rp + c0);
        q[fj][1] = lds_u32(rp + c0 + 4u);
      }
    }
  };
  auto decode = [&](const uint32_t (*q)[2], const half2v *d, half8 *b) {
#pragma unroll
    for (int fj = 0; fj < (int)kFN; ++fj) {
      const uint32_t q0 = q[fj][0] ^ 0x80808080u, q1 = q[fj][1] ^ 0x80808080u;
      const half2v e0 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q0, 0x04010400u));
      const half2v e1 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q0, 0x04030402u));
      const half2v e2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q1, 0x04010400u));
      const half2v e3 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, q1, 0x04030402u));
      const half2v v0 = (e0 + off) * d[fj], v1 = (e1 + off) * d[fj], v2 = (e2 + off) * d[fj],
                   v3 = (e3 + off) * d[fj];
      b[fj] = half8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
    }
  };

  // One step from stage (xs, ws), with the loads of a later step going to
  // (xn, wn_) in four groups; `full` is false on a last step holding one
  // block only (k % 64 == 32): the second block's weights are zero. The
  // operands of slot m + 1 are read and decoded while the 16 MFMAs of slot m
  // run.
  auto compute = [&](const uint8_t *xs, const uint8_t *ws, bool full, uint32_t sn, const uint8_t *xn,
                     const uint8_t *wn_) {
    // block scales of the lane's 4 rows: byte 0 (block 0), byte 34 (block 1)
    half2v d0[kFN], d1[kFN];
#pragma unroll
    for (int fj = 0; fj < (int)kFN; ++fj) {
      const uint8_t *rp = ws + bbase - 8u * h + fj * (32u * kRB);
      const uint32_t w0 = lds_u32(rp), w1 = lds_u32(rp + 32);
      const _Float16 s0 = __builtin_bit_cast(_Float16, (uint16_t)(w0 & 0xFFFFu));
      const _Float16 s1 = full ? __builtin_bit_cast(_Float16, (uint16_t)(w1 >> 16)) : (_Float16)0.0f;
      d0[fj] = half2v{s0, s0};
      d1[fj] = half2v{s1, s1};
    }
    half8 a[2][kFM], b[2][kFN];
    uint32_t q[kFN][2];
    load_a(xs, 0, a[0]);
    load_b(ws, 0, q);
    decode(q, d0, b[0]);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      issue_group(m, sn, xn, wn_);
      if (m < 3) {
        load_a(xs, m + 1, a[(m + 1) & 1]);
        load_b(ws, m + 1, q);
        decode(q, (m + 1) >= 2 ? d1 : d0, b[(m + 1) & 1]);
      }
#pragma unroll
      for (int fi = 0; fi < (int)kFM; ++fi)
#pragma unroll
        for (int fj = 0; fj < (int)kFN; ++fj)
          acc[fi][fj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[m & 1][fi], b[m & 1][fj], acc[fi][fj], 0, 0, 0);
      // schedule: the next slot's LDS reads first, three MFMAs while they
      // land, then its decode interleaved with the remaining MFMAs
      if (m < 3) {
        __builtin_amdgcn_sched_group_barrier(0x100, kFM + 2 * kFN, 0);  // LDS reads
        __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);               // 3 MFMA
#pragma unroll
        for (int i = 0; i < (int)(kFM * kFN) - 3; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x002, (16 * kFN + kFM * kFN - 4) / (kFM * kFN - 3), 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                            // 1 MFMA
        }
      }
    }
  };

  const bool tail_half = (k % kBK) != 0u;  // the last step holds one block
  // Step s: its loads (issued during step s - 2) are complete once at most
  // the next step's kDma loads are outstanding; the barrier makes every
  // wave's loads visible and frees the stage the loads of step s + 2 go to
  // (read in step s - 1).
  auto step = [&](uint32_t s, const uint8_t *xs, const uint8_t *ws, const uint8_t *xn, const uint8_t *wn_) {
    wait_vm<kDma>();
    __builtin_amdgcn_s_barrier();
    compute(xs, ws, !(tail_half && s == last), min(s + 2u, last), xn, wn_);
  };

  issue(0, st0, st0 + kXS);
  issue(min(1u, last), st1, st1 + kXS);
  // three steps per iteration, so that the stages are fixed objects; the
  // last one or two steps after the loop (no branch inside the loop: the
  // accumulators stay in place)
  uint32_t s = 0;
  for (; s + 3u <= steps; s += 3u) {
    step(s, st0, st0 + kXS, st2, st2 + kXS);
    step(s + 1u, st1, st1 + kXS, st0, st0 + kXS);
    step(s + 2u, st2, st2 + kXS, st1, st1 + kXS);
  }
  if (s < steps) step(s, st0, st0 + kXS, st2, st2 + kXS);
  if (s + 1u < steps) step(s + 1u, st1, st1 + kXS, st0, st0 + kXS);
  wait_vm<0>();

  // D[tok][row]: lane holds row (column) n of each fragment and tokens
  // 8 (v / 4) + 4 h + v % 4.
#pragma unroll
  for (int fj = 0; fj < (int)kFN; ++fj) {
    const uint32_t row = n0 + kFN * 32u * wn + 32u * fj + n;
    if (row >= rows) continue;
#pragma unroll
    for (int fi = 0; fi < (int)kFM; ++fi)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t tok = t0 + kFM * 32u * wm + 32u * fi + 8u * (v >> 2) + 4u * h + (v & 3);
        if (tok < tokens) y[(uint64_t)tok * rows + row] = acc[fi][fj][v];
      }
  }
}

}  // namespace

bool gemm_big_applies(int type, uint32_t tokens, uint32_t k) {
  return type == Q8_0 && tokens >= 1024 && k % 32u == 0;
}

hipError_t launch_gemm_big(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, hipStream_t s) {
  const uint32_t tok_tiles = (tokens + kBM - 1) / kBM, row_tiles = (wv.rows + kBN - 1) / kBN;
  hipLaunchKernelGGL(k_gemm_q8, dim3(row_tiles * tok_tiles), dim3(256), 0, s, wv, xh, y, tokens, row_tiles,
                     tok_tiles);
  return hipGetLastError();
}

}  // namespace eff
