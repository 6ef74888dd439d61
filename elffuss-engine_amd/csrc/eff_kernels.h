// Internal launch interface between the C ABI (eff_api.hip) and the kernels
// (eff_kernels.hip). All launches are asynchronous on `stream`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace eff {

// Raises the dynamic-LDS limit of kernel `fn` to `bytes` once per device: `done`
// (one per kernel) holds a bit per device whose limit is set. Safe to call
// from several threads (a second setter repeats the same idempotent call).
inline hipError_t lds_limit_once(const void *fn, int bytes, std::atomic<uint64_t> &done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? 1ull << dev : 0ull;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

// One quantized matrix W (rows x k) and its addressing.
struct WeightView {
  const uint8_t *w;       // device pointer to the tensor's first byte
  int type;               // eff::Type
  uint32_t rows, k, bpr;  // bpr = k / block_elems
  uint64_t row_bytes;     // bpr * block_bytes (GGUF layouts)
  uint64_t scales_off;    // Q8_0R: byte offset of the scale region (32 * N of the tensor)
  uint64_t w_bytes;       // readable bytes from w (loads past it return 0)
};

// GEMV shape chosen by the host (see plan_gemv).
struct GemvPlan {
  int rows_per_wave;  // R
  int ksplit;         // S: waves of a workgroup splitting k (1, 2, 4); the tile has waves/S * R rows
  int waves;          // waves per workgroup (4, or 8 for the matrix-core GEMV)
  uint32_t kc;        // k elements per slice
  uint32_t tiles;     // row tiles
  uint32_t grid;      // workgroups
  size_t lds_bytes;   // dynamic LDS (unused)
};

GemvPlan plan_gemv(const WeightView &wv, uint32_t tokens);

hipError_t launch_gemv(const WeightView &wv, const float *x, float *y, uint32_t tokens,
                       const GemvPlan &p, hipStream_t stream);

// Matrix-core GEMV (int8 MFMA over x digit planes, eff_gemv_mx.hip). Needs
// k % 64 == 0, 1..8 tokens and the x digits of one workgroup within kMxMaxLds;
// returns false (and the f32 kernel is used) otherwise.
constexpr size_t kMxMaxLds = 160 * 1024;
bool gemv_mx_plan(const WeightView &wv, uint32_t tokens, GemvPlan &p);
// Tuning hook: restrict the plan to (waves, k slices); (0, 0) restores the automatic choice.
void gemv_mx_override(int waves, int ksplit);
hipError_t launch_gemv_mx(const WeightView &wv, const float *x, float *y, uint32_t tokens,
                          const GemvPlan &p, hipStream_t stream);
// Fused matrix-core GEMV over n (1..4) matrices of one type and k that share
// x, for 1..3 tokens: mode 1 sections (ys[i] = W_i x), mode 2 gate + up
// (n = 2, equal rows, ys[0] = silu(W_0 x) * (W_1 x)). Each row is summed as
// its one-matrix launch sums it when the plans agree (always for gate + up).
bool gemv_mx_multi_applies(const WeightView &wv0, uint32_t tokens, int mode);
hipError_t launch_gemv_mx_multi(int mode, uint32_t n, const WeightView *wvs, const float *x, float *const *ys,
                                uint32_t tokens, hipStream_t stream);
// One-token GEMV for Q6_K matrices of >= 32768 rows (the output projection):
// a lane per half row-block, x digits as LDS broadcasts (eff_gemv_rows.hip).
bool gemv_rows_applies(const WeightView &wv, uint32_t tokens);
uint32_t gemv_rows_groups(const WeightView &wv);
hipError_t launch_gemv_rows(const WeightView &wv, const float *x, float *y, hipStream_t stream);
// The same GEMV with the top-m of its logits (the decode head): every
// workgroup of the GEMV also writes the top-k record of its rows (G =
// gemv_rows_groups(wv) workgroups, each over 2 to 5 tiles of 32 rows spread
// over the matrix) to rec (G <= kRowsTopkGroupsMax records), and one more
// launch selects from them into out.
constexpr uint32_t kRowsTopkGroupsMax = 1024;
hipError_t launch_gemv_rows_topk(const WeightView &wv, const float *x, float *y, uint8_t *rec, uint32_t m,
                                 const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, uint32_t *out,
                                 hipStream_t stream);
// Multi-token matrix-core GEMV (16 rows x 4 tokens per MFMA): 4..16 tokens
// per launch, Q8_0/Q4_K/Q6_K/Q2_K/IQ2_XXS, k % 256 == 0.
bool gemv_mt_plan(const WeightView &wv, uint32_t tokens, GemvPlan &p);
hipError_t launch_gemv_mt(const WeightView &wv, const float *x, float *y, uint32_t tokens,
                          const GemvPlan &p, hipStream_t stream);

// x is first rounded to fp16 into `xh_scratch`, gemm_x_bytes(...) bytes laid
// out as [token tile][k step][token][k] (zero past the tokens and past k).
// The kernel configuration is the one chosen for `plan` tokens (plan >=
// tokens); a run over fewer tokens gives those rows the bits they get in a
// run over `plan` tokens.
// cfg: the Q8_0 tile configuration (EFF_OPT_GEMM_CONFIG; 0 automatic).
size_t gemm_x_bytes(int type, uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg);
// An id of that layout: equal ids, one prepared x serves both products.
uint32_t gemm_x_layout(int type, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg);
// k-slice scratch (the Q8_0 GEMM's and the split-x product's): a counter per
// output tile (at most 2^16 tiles), then the slices' sums.
constexpr uint32_t kSliceCntBytes = 1u << 18;
// The k-slice scratch of the product (0 bytes: none): the Q8_0 GEMM cuts k
// into slices over workgroups where the tiles alone leave CUs idle.
// ksl_opt: forced slice count (EFF_OPT_GEMM_SPLIT; 0 automatic). The scratch
// starts with counters that must be zero before the first launch; each
// launch leaves them zero.
size_t gemm_sk_bytes(int type, uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg,
                     uint32_t ksl_opt);
hipError_t launch_gemm(const WeightView &wv, const float *x, float *y, uint32_t tokens, uint32_t plan,
                       uint32_t cfg, uint32_t ksl_opt, void *xh_scratch, void *sk_scratch, hipStream_t stream);
// The two halves of launch_gemm: x into its fp16 layout, and the product from it.
hipError_t launch_gemm_x(int type, const float *x, uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows,
                         uint32_t cfg, void *xh, hipStream_t stream);
hipError_t launch_gemm_prepared(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, uint32_t plan,
                                uint32_t cfg, uint32_t ksl_opt, void *sk_scratch, hipStream_t stream);
// Q8_0 / Q8_0R GEMM with direct-to-LDS staging (> 128 tokens, and below 6144
// rows from the GEMM's threshold); x in the
// [token tile][k step][2^gemm_big_tile_log2 tokens][64] layout.
bool gemm_big_applies(int type, uint32_t tokens, uint32_t k, uint32_t rows);
uint32_t gemm_big_tile_log2(uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg);
size_t gemm_big_scratch_bytes(uint32_t tokens, uint32_t plan, uint32_t k, uint32_t rows, uint32_t cfg,
                              uint32_t ksl_opt);
hipError_t launch_gemm_big(const WeightView &wv, const _Float16 *xh, float *y, uint32_t tokens, uint32_t plan,
                           uint32_t cfg, uint32_t ksl_opt, void *scratch, hipStream_t stream);

// Split-x matrix-core product (eff_gemm_sx.hip): Q2_K, Q4_K, IQ2_XXS, Q8_0,
// Q6_K from 2 tokens, k % 256 == 0, f32-accurate. `scratch` holds
// sx_x_bytes(...) bytes (x as fp16 hi/lo parts and the block scales). cfg: 0
// automatic, 1: 32 rows x 8 waves per workgroup, 2: 64 rows x 4 waves, 3: as 2
// with k in two slices. ksl_opt: forced k slices (0 automatic); `sk` holds
// the k-slice scratch, sx_sk_bytes(...) bytes (none: 0), with the same
// counters as the GEMM's (gemm_sk_bytes).
bool sx_applies(const WeightView &wv, uint32_t tokens);
size_t sx_x_bytes(int type, uint32_t tokens, uint32_t k);
size_t sx_sk_bytes(const WeightView &wv, uint32_t tokens, int cfg, uint32_t ksl_opt);
hipError_t launch_sx(const WeightView &wv, const float *x, float *y, uint32_t tokens, void *scratch, int cfg,
                     uint32_t ksl_opt, void *sk, hipStream_t stream);
// The same product in two halves, so that one preparation of x serves every
// product of that x: sx_x_layout is the layout the product reads (0: none,
// the one-launch product up to 8 tokens reads x itself; kSxLayout for IQ2_XXS,
// Q8_0 and Q6_K, | 1 with the group sums of Q2_K, | 2 with those of Q4_K);
// launch_sx_prepare writes x in it (sx_prepared_bytes), launch_sx_prepared
// runs the product from it (the same bits as launch_sx).
constexpr uint32_t kSxLayout = 0x100u;
uint32_t sx_x_layout(const WeightView &wv, uint32_t tokens, int cfg, uint32_t ksl_opt);
size_t sx_prepared_bytes(uint32_t layout, uint32_t tokens, uint32_t k);
hipError_t launch_sx_prepare(uint32_t layout, const float *x, uint32_t tokens, uint32_t k, void *xprep,
                             hipStream_t stream);
hipError_t launch_sx_prepared(const WeightView &wv, const void *xprep, float *y, uint32_t tokens, int cfg,
                              uint32_t ksl_opt, void *sk, hipStream_t stream);

// The reference CPU path's arithmetic for Q8_0 (eff_cpu_path.hip): x into
// 40-byte 8-bit blocks in `act` (cpu_path_act_bytes(...)), then per row and
// token the block terms added in block order; the bits of or_cpu_matmul.
size_t cpu_path_act_bytes(uint32_t tokens, uint32_t k);
hipError_t launch_cpu_path(const WeightView &wv, const float *x, float *y, uint32_t tokens, void *act,
                           hipStream_t stream);

// Embedding gather: out[t] = dequantized row ids[t] (bit-identical to dequant);
// with the norm, also nrm[t] = x[t] / sqrt(mean(x[t]^2) + eps) * wn, dim <= kGatherNormMaxDim.
constexpr uint32_t kGatherNormMaxDim = 32768;
hipError_t launch_gather(const WeightView &wv, const uint32_t *ids, uint32_t tokens, float *out, hipStream_t stream);
hipError_t launch_gather_norm(const WeightView &wv, const uint32_t *ids, uint32_t tokens, const float *wn, float eps,
                              float *x, float *nrm, hipStream_t stream);

hipError_t launch_dequant(const WeightView &wv, uint32_t n_blocks, float *out, hipStream_t stream);

// Streaming read of `bytes` bytes of src by `workgroups` workgroups of 256
// threads, `unroll` (1, 2, 4) 16-byte loads in flight per lane; sink holds one
// word per workgroup (written only in the unlikely event that a workgroup's XOR
// of its bytes equals a fixed constant).
hipError_t launch_read_floor(const uint8_t *src, uint64_t bytes, uint32_t workgroups, uint32_t unroll, uint32_t *sink,
                             hipStream_t stream);

// Top-k (eff_topk.hip). The logits are cut into G <= kTopkGroupsMax groups
// of 256 * ceil(vocab / 65536) consecutive logits; the first kernel writes
// one kTopkRecordBytes record per group (its 4 largest elements) and, in an
// array after the G records, each group's largest composite (8 bytes); the
// second selects from them. The scratch is G x kTopkGroupBytes, at most
// 18 KiB for any vocabulary.
constexpr uint32_t kTopkGroupsMax = 256;
constexpr uint32_t kTopkRecordBytes = 64;
constexpr uint32_t kTopkGroupBytes = kTopkRecordBytes + 8u;
constexpr uint32_t kTopkRecordChunk = 4096;   // the reference's logits per chunk (header field `chunks`)
constexpr uint32_t topk_group_size(uint32_t vocab) { return 256u * ((vocab + 65535u) / 65536u); }
constexpr uint32_t topk_groups(uint32_t vocab) {
  return (vocab + topk_group_size(vocab) - 1u) / topk_group_size(vocab);
}
constexpr size_t topk_scratch_bytes_for(uint32_t vocab) { return (size_t)topk_groups(vocab) * kTopkGroupBytes; }
constexpr size_t kTopkScratchMax = (size_t)kTopkGroupsMax * kTopkGroupBytes;
size_t topk_scratch_bytes(uint32_t vocab);

hipError_t launch_topk(const uint32_t *logits, uint32_t base, uint32_t vocab, uint32_t m,
                       const uint32_t *penal_ids_dev, uint32_t n_penal, uint32_t serial,
                       uint32_t *scratch, uint32_t *out, hipStream_t stream);

}  // namespace eff
