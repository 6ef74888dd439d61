// The reference CPU path's arithmetic for Q8_0 on the GPU: the product
// cpu-kernels.js forms (cpu.js:350-381, driven over row chunks by
// cpu-trabajo.js:27-72), as the oracle restates it:
//  * each token's x is cut into blocks of 32 values (cuantiza_filas; 40-byte
//    blocks, BACT = 40, cpu.js:24-27): d = max|x| / 127, q = round(x / d)
//    with ties away from zero (x times the rounded 1 / d), s = d * sum q;
//  * per row and token, y = (((0 + t_0) + t_1) + ... + t_(nb-1)) with
//    t_b = f32(isum_b) * (d_w,b * d_x,b) and isum_b the exact int32 dot of the
//    block's quants, every operation rounded on its own (no fused
//    multiply-add). A row's chunk does not change its bits.
// From 16 tokens the block dots run on the matrix cores (k_cpu_rows_q8_mfma),
// with the same terms added in the same order.
// The default router keeps f32 accuracy instead (these 8-bit activations put
// the CPU path about 5e-3 relative L2 from the exact product); this product
// gives the CPU path's own bits, for callers that need the two backends to
// agree.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/elffuss_amd.h"
#include "eff_device.h"
#include "eff_formats.h"
#include "eff_kernels.h"

namespace eff {

namespace {

constexpr uint32_t kTermWaves = 4;   // rows per workgroup (a wave each)

// One lane per (token, block of 32 x values): the 40-byte activation block.
__global__ __launch_bounds__(256) void k_cpu_acts(const float *__restrict__ x, uint32_t n_blocks,
                                                  uint32_t *__restrict__ act) {
#pragma clang fp contract(off)
  const uint32_t b = blockIdx.x * 256u + threadIdx.x;
  if (b >= n_blocks) return;
  const float4 *v4 = (const float4 *)(x + 32ull * b);
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 t = v4[i];
    v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) a = fmaxf(a, fabsf(v[i]));
  const float d = a / 127.f;
  const float id = d != 0.f ? 1.f / d : 0.f;
  int sum = 0;
  uint32_t qw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = (int)roundf(v[4 * i + j] * id);
      sum += q;
      w |= (uint32_t)(uint8_t)(int8_t)q << (8 * j);
    }
    qw[i] = w;
  }
  const float s = d * (float)sum;
  uint32_t *o = act + 10ull * b;
  o[0] = __float_as_uint(d);
  o[1] = __float_as_uint(s);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[2 + i] = qw[i];
}

// A wave per row. Per chunk of 64 blocks, lane j holds the quants and scale
// of block c + j and forms every token's term for it into LDS; then lane t
// adds token t's terms in block order onto its running sum. Term (t, j) sits
// at column j ^ t of row t, so that both the writes (one t, every j) and the
// reads (every t, one j) fall in 64 different banks. Waves past the last row
// take part in the barriers only. LDS: 256 bytes per wave and token of a
// chunk (at most 64), so that one token takes 1 KB per workgroup.
__global__ __launch_bounds__(kTermWaves * 64) void k_cpu_rows_q8(WeightView wv, const uint32_t *__restrict__ act,
                                                                 float *__restrict__ y, uint32_t tokens) {
#pragma clang fp contract(off)
  extern __shared__ float terms[];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * kTermWaves + wave, rows = wv.rows;
  const bool live = row < rows;
  const uint32_t nb = wv.k / 32u;
  const rsrc_t src = make_rsrc(wv.w, wv.w_bytes);
  float(*tm)[64] = (float(*)[64])(terms + wave * min(tokens, 64u) * 64u);
  for (uint32_t t0 = 0; t0 < tokens; t0 += 64u) {
    const uint32_t tn = min(64u, tokens - t0);
    float s = 0.f;   // lane t: token t0 + t
    for (uint32_t c0 = 0; c0 < nb; c0 += 64u) {
      const uint32_t bn = min(64u, nb - c0), b = c0 + lane;
      const bool mine = live && lane < bn;
      // the block's 34 bytes from their 4-byte aligned floor (sh = 0 or 2)
      uint32_t wq[8];
      float dw = 0.f;
      if (mine) {
        const uint64_t o = (uint64_t)row * wv.row_bytes + 34ull * b;
        const uint32_t sh = (uint32_t)(o & 3u), base = (uint32_t)(o - sh);
        uint32_t r[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) r[i] = __builtin_amdgcn_raw_buffer_load_b32(src, (int)(base + 4u * i), 0, 0);
        dw = h2f(sh ? r[0] >> 16 : r[0] & 0xFFFFu);
#pragma unroll
        for (int i = 0; i < 8; ++i) wq[i] = sh ? r[i + 1] : __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);
      }
      for (uint32_t t = 0; t < tn; ++t) {
        float term = 0.f;
        if (mine) {
          const uint32_t *ab = act + ((uint64_t)(t0 + t) * nb + b) * 10u;
          const float dx = __uint_as_float(ab[0]);
          int isum = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) isum = __builtin_amdgcn_sdot4((int)wq[i], (int)ab[2 + i], isum, false);
          term = (float)isum * (dw * dx);
        }
        tm[t][lane ^ t] = term;
      }
      __syncthreads();
      if (lane < tn) {
#pragma unroll 16
        for (uint32_t j = 0; j < bn; ++j) s = s + tm[lane][j ^ lane];
      }
      __syncthreads();
    }
    if (live && lane < tn) y[(uint64_t)(t0 + lane) * rows + row] = s;
  }
}

// From 16 tokens: the block dots on the matrix cores. v_mfma_i32_16x16x32_i8
// takes exactly one block (32 k): A = the 8-bit x of 16 tokens, B = the
// quants of 16 rows, D = the exact int32 block dots, lane l holding tokens
// 4 (l / 16) .. + 3 of row l % 16. A workgroup of 4 waves takes 64 tokens x
// 64 rows, a wave 16 tokens x the 64 rows (four instructions per block), and
// walks the blocks in order, each lane adding its 16 outputs' terms
// (f32(isum) (dw dx), rounded as above) one block after the other: the bits
// of the one-wave-per-row kernel. The blocks come in chunks of kMfCb staged
// in LDS by coalesced loads: per row the chunk's bytes from their 4-byte
// aligned floor (kMfWs dwords, an odd stride), per token its 40-byte x blocks
// (kMfXs dwords, odd too), so that the lanes' reads of 16 rows or tokens fall
// in different banks.
constexpr uint32_t kMfRows = 64, kMfTok = 16, kMfWaves = 4, kMfCb = 8;
constexpr uint32_t kMfWs = (kMfCb * 34u + 2u + 3u) / 4u | 1u;   // 69 dwords per staged row
constexpr uint32_t kMfXs = kMfCb * 10u + 1u;                    // 81 dwords per staged token
typedef int int4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kMfWaves * 64) void k_cpu_rows_q8_mfma(WeightView wv, const uint32_t *__restrict__ act,
                                                                     float *__restrict__ y, uint32_t tokens) {
#pragma clang fp contract(off)
  __shared__ uint32_t ws[kMfRows * kMfWs];
  __shared__ uint32_t xs[kMfWaves * kMfTok * kMfXs];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t tw = blockIdx.y * kMfWaves * kMfTok, t0 = tw + wave * kMfTok, r0 = blockIdx.x * kMfRows;
  const uint32_t rows = wv.rows, nb = wv.k / 32u, n = lane & 15u, g = lane >> 4;
  const uint32_t rb = (uint32_t)wv.row_bytes;
  const rsrc_t src = make_rsrc(wv.w, wv.w_bytes);
  const bool live = t0 < tokens;   // waves past the tokens take part in the staging and barriers only
  float acc[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rt][i] = 0.f;
  for (uint32_t b0 = 0; b0 < nb; b0 += kMfCb) {
    const uint32_t cb = min(kMfCb, nb - b0);
    __syncthreads();   // the previous chunk is consumed
    // the rows' bytes (loads past the tensor read zeros)
    for (uint32_t i = tid; i < kMfRows * kMfWs; i += kMfWaves * 64u) {
      const uint32_t r = i / kMfWs, d = i - r * kMfWs;
      const uint32_t base = (min(r0 + r, rows - 1u) * rb + 34u * b0) & ~3u;
      ws[i] = __builtin_amdgcn_raw_buffer_load_b32(src, (int)(base + 4u * d), 0, 0);
    }
    // the tokens' x blocks of the chunk
    for (uint32_t i = tid; i < kMfWaves * kMfTok * kMfXs; i += kMfWaves * 64u) {
      const uint32_t t = i / kMfXs, d = i - t * kMfXs;
      xs[i] = d < cb * 10u ? act[((uint64_t)min(tw + t, tokens - 1u) * nb + b0) * 10u + d] : 0u;
    }
    __syncthreads();
    if (live) {
      const uint32_t *xa = xs + (wave * kMfTok + n) * kMfXs + 2u + 2u * g;   // A: token t0 + n
      const uint32_t *xd = xs + (wave * kMfTok + 4u * g) * kMfXs;           // dx: tokens t0 + 4 g + i
      for (uint32_t j = 0; j < cb; ++j) {
        const long a = (long)(((uint64_t)xa[10u * j + 1u] << 32) | xa[10u * j]);
        float dx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) dx[i] = __uint_as_float(xd[i * kMfXs + 10u * j]);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          const uint32_t r = 16u * (uint32_t)rt + n;
          // block j of the row starts sh + 34 j bytes into its staged dwords
          // (sh = 0 or 2): the scale there, the lane's 8 quants 2 + 8 g after
          const uint32_t sh = (min(r0 + r, rows - 1u) * rb + 34u * b0) & 3u, at = sh + 34u * j;
          const uint32_t *wr = ws + r * kMfWs;
          const uint32_t w0 = wr[at >> 2];
          const float dw = h2f((at & 3u) ? w0 >> 16 : w0 & 0xFFFFu);
          const uint32_t qa = at + 2u + 8u * g, qd = qa >> 2;
          const uint32_t q0 = wr[qd], q1 = wr[qd + 1u], q2 = wr[qd + 2u];
          const uint32_t lo = (qa & 3u) ? __builtin_amdgcn_alignbyte(q1, q0, 2) : q0;
          const uint32_t hi = (qa & 3u) ? __builtin_amdgcn_alignbyte(q2, q1, 2) : q1;
          const long bq = (long)(((uint64_t)hi << 32) | lo);
          const int4v d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq, int4v{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[rt][i] = acc[rt][i] + (float)d[i] * (dw * dx[i]);
        }
      }
    }
  }
  if (!live) return;
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const uint32_t row = r0 + 16u * (uint32_t)rt + n;
    if (row >= rows) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = t0 + 4u * g + (uint32_t)i;
      if (t < tokens) y[(uint64_t)t * rows + row] = acc[rt][i];
    }
  }
}

}  // namespace

size_t cpu_path_act_bytes(uint32_t tokens, uint32_t k) { return (size_t)tokens * (k / 32u) * 40u; }

hipError_t launch_cpu_path(const WeightView &wv, const float *x, float *y, uint32_t tokens, void *act,
                           hipStream_t s) {
  // (32-bit byte offsets into the weights)
  if (wv.type != Q8_0 || wv.k % 32u || wv.w_bytes >= (1ull << 32)) return hipErrorInvalidValue;
  const uint32_t nblk = tokens * (wv.k / 32u);   // the caller keeps it below 2^31
  hipLaunchKernelGGL(k_cpu_acts, dim3((nblk + 255u) / 256u), dim3(256), 0, s, x, nblk, (uint32_t *)act);
  if (tokens >= kMfTok) {
    hipLaunchKernelGGL(k_cpu_rows_q8_mfma, dim3((wv.rows + kMfRows - 1u) / kMfRows,
                                                (tokens + kMfWaves * kMfTok - 1u) / (kMfWaves * kMfTok)),
                       dim3(kMfWaves * 64), 0, s, wv, (const uint32_t *)act, y, tokens);
    return hipGetLastError();
  }
  const uint32_t lds = kTermWaves * (tokens < 64u ? tokens : 64u) * 64u * 4u;
  hipLaunchKernelGGL(k_cpu_rows_q8, dim3((wv.rows + kTermWaves - 1u) / kTermWaves), dim3(kTermWaves * 64), lds, s,
                     wv, (const uint32_t *)act, y, tokens);
  return hipGetLastError();
}

}  // namespace eff
