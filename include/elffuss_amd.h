/*
 * elffuss_amd.h — C ABI of the MI355X (gfx950) quantized matrix-product path.
 *
 * This is the drop-in boundary for Elffuss Engine's quantized GEMV/GEMM hot
 * path. A host binding (N-API addon for the JavaScript engine, ctypes for
 * Python) calls these functions with plain pointers and sizes. Device memory
 * is held in opaque buffers; every launch is enqueued on the context's HIP
 * stream and returns without waiting, as the reference records dispatches into
 * an open compute pass and returns (ops.js:667-710). Only eff_buf_read,
 * eff_read_end and eff_sync wait for the device (device.js:165-200, readback).
 *
 * Return codes follow the reference's error conventions:
 *   EFF_OK              success;
 *   EFF_NOT_APPLICABLE  "this fast path does not apply, caller falls back",
 *                       the reference's `null` (ops.gemv.js:13-21, ops.gemm2.js:5-8);
 *   negative            contract violation or device failure, the reference's
 *                       thrown Error; eff_last_error() gives the message.
 *
 * Types are ggml type codes (gguf.js:51-64) plus the internal repacked type
 * Q8_0R (kernels.bloques.wgsl.js:86-89), which never appears in a GGUF file.
 */
#ifndef ELFFUSS_AMD_H
#define ELFFUSS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define EFF_OK              0
#define EFF_NOT_APPLICABLE  1
#define EFF_E_INVALID      (-1)  /* bad argument (null pointer, zero size, ...) */
#define EFF_E_TYPE         (-2)  /* unknown or unsupported type (ops.js:767-771) */
#define EFF_E_SHAPE        (-3)  /* k not a multiple of the block (ops.js:850-852) */
#define EFF_E_MARK         (-4)  /* repacked buffer unmarked, wrong type or call beyond the tensor (repack.js:268-286) */
#define EFF_E_BOUNDS       (-5)  /* a buffer is too small for the call */
#define EFF_E_DEVICE       (-6)  /* HIP runtime error */
#define EFF_E_NOMEM        (-7)  /* device allocation failed */

/* ---- types (ggml codes; gguf.js:51-64) ---------------------------------- */
#define EFF_TYPE_Q8_0      8
#define EFF_TYPE_Q2_K      10
#define EFF_TYPE_Q4_K      12
#define EFF_TYPE_Q6_K      14
#define EFF_TYPE_IQ2_XXS   16
#define EFF_TYPE_Q8_0R     264   /* Q8_0 repacked at load (kernels.bloques.wgsl.js:19-35) */

/* ---- options (the reference's globalThis.__ELFFUSS_* switches, ops.js:827-1101) */
#define EFF_OPT_GEMV_MAX_TOKENS  1  /* tokens <= this go to the GEMV kernels (default 8) */
#define EFF_OPT_GEMM_MIN_TOKENS  2  /* tokens >= this go to the fp16 MFMA GEMM (default 64; __ELFFUSS_DRIFT_DESDE) */
#define EFF_OPT_GEMV_KERNEL      3  /* 0: int8 matrix-core GEMV where it applies (default), 1: f32 vector GEMV */
#define EFF_OPT_SPLIT_CONFIG     4  /* split-x product workgroups (tuning): 0 automatic (default), 1: 32 rows x
                                       8 waves, 2: 64 rows x 4 waves, 3: 64 rows x 4 waves with k in two slices
                                       (EFF_OPT_SPLIT_SLICES) */
#define EFF_OPT_SPLIT_MIN_TOKENS 5  /* Q2_K, Q4_K, IQ2_XXS, Q8_0, Q6_K: tokens >= this run the split-x product, fewer
                                       the int8 matrix-core GEMVs (0: automatic, 5 for Q2_K and IQ2_XXS, 9 for the
                                       others, 7 where k > 4096 and for Q4_K and Q6_K where k = 4096 from 5120
                                       rows (default); else >= 4).
                                       Q8_0 only below EFF_OPT_GEMM_MIN_TOKENS */
#define EFF_OPT_GEMM_CONFIG      6  /* Q8_0 GEMM from the GEMM's threshold (below 6144 rows at every count),
                                       tiles (tuning; tokens x rows, waves along tokens x rows, LDS stages):
                                       0 automatic (default), 1: 256x256 1x4 3, 2: 128x128 1x4 3,
                                       3: 128x128 1x4 6, 4: 64x128 1x4 4, 5: 128x256 1x4 4, 6: 256x128 2x2 3; every
                                       configuration sums each output in the same order (the same bits) */
#define EFF_OPT_GEMM_SPLIT       7  /* the same Q8_0 GEMM, k slices over workgroups (tuning): 0 automatic
                                       (default: where the tiles leave CUs idle, about 256 workgroups in all,
                                       slices of 512 k at least), else that many (1: none; 256 x 256 tiles
                                       take none); the slices' sums are added in slice order, so each count
                                       gives fixed bits */
#define EFF_OPT_SPLIT_SLICES     8  /* split-x product, k slices over workgroups (tuning): 0 automatic (default),
                                       else that many (1: none); the slices' sums are added in slice order */

/* ---- fused GEMV modes (gemv2Shader `modo`, kernels.gemv.wgsl.js:370-375) -- */
#define EFF_GEMV_SECTIONS  1  /* 'secciones': ys[i] = W_i x for 2..4 matrices */
#define EFF_GEMV_SWIGLU    2  /* 'swiglu': ys[0] = silu(W_gate x) * (W_up x) */

/* ---- top-k output layout (kernels.topk.wgsl.js:40-60) ------------------- */
#define EFF_TOPK_M_MAX     192   /* largest M = K' + |S| accepted (TOPK_M_MAX) */
#define EFF_TOPK_P_MAX     128   /* penalised ids (TOPK_P_MAX) */
#define EFF_TOPK_CAP       256   /* candidate pairs in the output (TOPK_CAP) */
#define EFF_TOPK_HEADER    8     /* u32 header words (TOPK_CABECERA) */
#define EFF_TOPK_N_MAX     (1u << 24)  /* vocabulary limit (TOPK_N_MAX) */

typedef struct eff_ctx eff_ctx;
typedef struct eff_buf eff_buf;
typedef struct eff_read eff_read;
typedef struct eff_graph eff_graph;

/* Dispatch counters: lets a caller assert that a fast path really ran
 * (ops.gemv.js:92-95 `hechos`, ops.topk.js:36-40 `estadisticasTopK`). */
typedef struct eff_stats {
  uint64_t gemv;        /* GEMV launches (tokens <= GEMV max) */
  uint64_t gemm;        /* fp16 MFMA GEMM launches */
  uint64_t skinny;      /* GEMV launches over token groups (GEMV max < tokens < GEMM min) */
  uint64_t dequant;     /* dequant launches */
  uint64_t topk;        /* top-k calls (records + selection; eff_topk, eff_topk_noalloc, eff_qgemv_topk) */
  uint64_t not_applicable;  /* calls answered EFF_NOT_APPLICABLE */
  uint64_t split;       /* split-x matrix-core launches (Q2_K, Q4_K, IQ2_XXS, Q8_0, Q8_0R, Q6_K from
                           EFF_OPT_SPLIT_MIN_TOKENS) */
  uint64_t fused;       /* fused GEMV launches (eff_qgemv_multi) */
  uint64_t gather;      /* gather launches (eff_gather, eff_gather_norm) */
  uint64_t gemm_x;      /* conversions of x to fp16 for the GEMM (one per eff_qgemm / eff_qgemm_planned /
                           router GEMM call, one per eff_gemm_prepare_x, one per eff_qmatmul_prepare_x
                           for the GEMM) */
  uint64_t split_x;     /* preparations of x for the split-x product in a launch of their own (one per
                           split-x router call but those of Q2_K and IQ2_XXS up to 8 tokens under the
                           automatic configuration, which prepare x inside the product; one per
                           eff_qmatmul_prepare_x for it) */
  uint64_t cpu_path;    /* products with the reference CPU path's arithmetic (eff_qmatmul_cpu_path) */
} eff_stats;

/* ---- types and geometry -------------------------------------------------- */

/* Type code for a ggml type name ("Q8_0", "Q8_0R", "Q4_K", "Q6_K", "Q2_K",
 * "IQ2_XXS"); EFF_E_TYPE otherwise. Replaces quantInfo/QUANT_TYPES
 * (kernels.wgsl.js:886-895). */
int eff_type_from_name(const char *name);

/* Name of a type code, or NULL. */
const char *eff_type_name(int type);

/* Elements and bytes per block (gguf.js:51-64; kernels.wgsl.js QUANT_TYPES).
 * For Q8_0R block_bytes is the average 34, not a stride (kernels.wgsl.js:846-850). */
int eff_type_geometry(int type, uint32_t *block_elems, uint32_t *block_bytes);

/* ---- context -------------------------------------------------------------- */

/* Open a context on HIP device `device` with its own stream (default priority).
 * Replaces requestDevice + createOps (device.js:66-139, ops.js:1604-1633). */
int eff_init(int device, eff_ctx **out);

/* Release the context, its stream (if owned) and its scratch memory, after
 * the work on its stream has ended. Read tickets still open (eff_read_begin)
 * stay valid: they may be ended and released afterwards. */
int eff_shutdown(eff_ctx *ctx);

/* Message of the last error on this context ("" if none). */
const char *eff_last_error(const eff_ctx *ctx);

/* The hipStream_t launches are enqueued on. */
void *eff_stream(eff_ctx *ctx);

/* Enqueue on a caller-owned hipStream_t from now on (NULL: back to the
 * context's own stream). The caller keeps ownership. The calls enqueued from
 * now on wait for those already enqueued on the previous stream (they share
 * the context's scratch buffers): the new stream waits for an event recorded
 * on the previous one, unless it is being recorded into a graph (the caller
 * orders the replays). EFF_E_INVALID while the previous stream is recorded
 * into a graph. */
int eff_set_stream(eff_ctx *ctx, void *hip_stream);

/* Wait for everything enqueued on the context's stream. */
int eff_sync(eff_ctx *ctx);

/* Set an option (EFF_OPT_*). Mirrors the __ELFFUSS_* switches read per call. */
int eff_set_option(eff_ctx *ctx, int option, int64_t value);

/* Dispatch counters since eff_init. */
int eff_get_stats(const eff_ctx *ctx, eff_stats *out);

/* ---- recorded launches (the MI355X form of ctx.batch / ctx.corta) -------- */

/* The reference records a layer's (or a token's) dispatches into one compute
 * pass and submits them together (ctx.batch, ops.js:311-332; ctx.corta,
 * ops.js:342-348). Here the launches enqueued on the context's stream between
 * eff_graph_begin and eff_graph_end are recorded, not run, into a HIP graph;
 * eff_graph_launch replays them, in order, on the context's stream without
 * waiting, any number of times, with the same buffers and shapes (new inputs
 * are written into the same buffers between replays). While recording, the
 * calls that wait, allocate or move host data (eff_sync, eff_buf_alloc,
 * eff_buf_free, eff_buf_retire, eff_buf_write, eff_buf_write_r, eff_buf_read,
 * eff_read_begin, and an op whose scratch would have to grow) return
 * EFF_E_INVALID and leave the recording open. An op's scratch is grown by
 * its first call of a shape outside a recording. */
int eff_graph_begin(eff_ctx *ctx);
int eff_graph_end(eff_ctx *ctx, eff_graph **out);
int eff_graph_launch(eff_ctx *ctx, eff_graph *g);
/* Launches (graph nodes) a recording holds. */
size_t eff_graph_nodes(const eff_graph *g);
int eff_graph_destroy(eff_graph *g);

/* ---- device buffers ------------------------------------------------------ */

/* Allocate `bytes` of device memory (plus hidden read slack; the reference's
 * loader leaves 4 bytes after every tensor, model.js:248-254) from the
 * device's stream-ordered memory pool. Contents are zero for every later
 * operation on the context's stream: the clear is enqueued there and the host
 * does not wait. Refused (EFF_E_INVALID) while the stream is under graph
 * capture. Replaces device.createBuffer behind the ctx.alloc pool
 * (ops.js:233-281), which the JS host keeps. */
int eff_buf_alloc(eff_ctx *ctx, size_t bytes, eff_buf **out);

/* Wrap caller-owned device memory of `bytes` bytes (not freed by
 * eff_buf_free). The caller must leave at least 16 readable bytes after it. */
int eff_buf_wrap(eff_ctx *ctx, void *device_ptr, size_t bytes, eff_buf **out);

/* Free a buffer after the work of every stream of the device has ended
 * (a device wait). */
int eff_buf_free(eff_ctx *ctx, eff_buf *buf);

/* Free a buffer in stream order, without waiting: the memory goes back to
 * the pool once the work enqueued before this call on the context's stream
 * has run, and the handle is invalid on return. The caller guarantees that
 * no work on another stream still reads the buffer. Replaces
 * GPUBuffer.destroy(), which is safe with work already submitted (the pool's
 * destruction of unused size classes, ops.js:264-279). Refused
 * (EFF_E_INVALID) while the stream is under graph capture. */
int eff_buf_retire(eff_ctx *ctx, eff_buf *buf);
size_t eff_buf_size(const eff_buf *buf);
void *eff_buf_device_ptr(const eff_buf *buf);

/* Host -> device, enqueued on the stream (queue.writeBuffer). `src` may be
 * reused on return: up to 4 MiB it is copied into a pinned staging ring and
 * the call does not wait for the device (it waits only when the ring range it
 * needs is still being copied); larger writes wait for their copy. Refused
 * (EFF_E_INVALID) on a stream under graph capture. */
int eff_buf_write(eff_ctx *ctx, eff_buf *buf, size_t offset, const void *src, size_t n);

/* Device -> host; waits for prior work (readback, device.js:165-200). */
int eff_buf_read(eff_ctx *ctx, eff_buf *buf, size_t offset, void *dst, size_t n);

/* The readback split in two (device.js:165-200, mapAsync): eff_read_begin
 * enqueues the copy of n bytes into pinned host memory on the context's
 * stream, now, so the snapshot holds exactly the work enqueued before it;
 * eff_read_end (any thread) waits for that copy and copies the bytes to dst;
 * eff_read_release frees the ticket. The buffer may be reused by later
 * operations on the stream right after eff_read_begin. eff_read_end's errors
 * are described by eff_read_error (the context's message is not touched). */
int eff_read_begin(eff_ctx *ctx, eff_buf *buf, size_t offset, size_t n, eff_read **out);
int eff_read_end(eff_read *r, void *dst);
/* Without waiting: 1 once the ticket's copy has completed (eff_read_end
 * then returns at once), 0 while it is in flight, negative on a device error
 * (described by eff_read_error). Lets a host poll from its own loop instead
 * of blocking a thread. */
int eff_read_poll(eff_read *r);
const char *eff_read_error(const eff_read *r);
int eff_read_release(eff_read *r);

/* Device -> device copy, enqueued. */
int eff_buf_copy(eff_ctx *ctx, eff_buf *dst, size_t dst_offset, eff_buf *src,
                 size_t src_offset, size_t n);

/* ---- repacked layout (Q8_0R) -------------------------------------------- */

/* Bytes of the Q8_0R format of n blocks: 34n rounded up to 4
 * (bytesReordenado, kernels.bloques.wgsl.js:111-113). */
size_t eff_bytes_reordered(int type_r, uint32_t n_blocks);

/* Bytes of a Q8_0R buffer for n blocks: 34n rounded up to 16
 * (bytesBufferR, kernels.bloques.wgsl.js:115-120). */
size_t eff_bytes_buffer_r(int type_r, uint32_t n_blocks);

/* Blocks a Q8_0R buffer of `bytes` bytes holds: floor(2L/17), L = bytes/4
 * (bloquesDeBuffer, kernels.bloques.wgsl.js:128-135). */
uint32_t eff_blocks_from_buffer(int type_r, size_t bytes);

/* First u32 word of the scale region of a tensor of n blocks: 8n
 * (escalasDesde, kernels.bloques.wgsl.js:122-125). */
uint32_t eff_scales_from(int type_r, uint32_t n_blocks);

/* Mark `buf` as holding a Q8_0R tensor of n blocks; its size must equal
 * eff_bytes_buffer_r (marcaBufferR, repack.js:241-251). */
int eff_buf_mark_r(eff_buf *buf, int type_r, uint32_t n_blocks);

/* Blocks recorded by the mark, EFF_E_MARK if unmarked (bloquesR, repack.js:256-259). */
int eff_buf_blocks_r(const eff_buf *buf, uint32_t *n_blocks);

/* Host repack of n GGUF Q8_0 blocks into Q8_0R (reordena, repack.js:187-199).
 * `dst_bytes` >= eff_bytes_reordered; bytes after the scales are zeroed. */
int eff_repack(int type_r, const void *src, uint32_t n_blocks, void *dst, size_t dst_bytes);

/* Inverse: Q8_0R back to GGUF blocks, 34n bytes (vuelveAlGGUF, repack.js:204-219). */
int eff_unrepack(int type_r, const void *src, size_t src_bytes, uint32_t n_blocks, void *dst);

/* Upload a chunk of a tensor into its repacked buffer: n_blocks GGUF Q8_0
 * blocks (34 bytes each, host memory) that are blocks first_block.. of the
 * tensor, repacked and written to their two regions of `buf` (quants at
 * 32 first_block, scales at 32 N + 2 first_block, N from the buffer's mark).
 * Synchronous with respect to `src`. Replaces one chunk of
 * subeReordenadoPorTrozos (repack.js:318-345). EFF_E_MARK for an unmarked
 * buffer, EFF_E_BOUNDS for blocks past the tensor. */
int eff_buf_write_r(eff_ctx *ctx, eff_buf *buf, int type_r, uint32_t first_block, const void *src,
                    uint32_t n_blocks);

/* ---- host data preparation ---------------------------------------------- */

/* Quantize n floats (n a multiple of the block) into GGUF blocks. Q8_0 follows
 * the reference's quantizer (cpu.js:273-287, aF16 cpu.js:84-99). Q4_K, Q6_K,
 * Q2_K and IQ2_XXS have no quantizer in the reference (it only reads them);
 * these are this library's own, producing valid blocks of the GGUF layout.
 * Uses all host threads. */
int eff_quantize(int type, const float *src, size_t n, void *dst, size_t dst_bytes);

/* Deterministic N(0, sigma) floats: uniforms from the mulberry32 hash of
 * sample.js:36-41 at counters seed+2i, seed+2i+1, Box-Muller in double,
 * rounded to float. Element i depends only on (seed, i). */
int eff_fill_normal(uint32_t seed, float sigma, float *dst, size_t n);

/* ---- operations (enqueued on the context's stream) ---------------------- */

/* Y[tokens][rows] = W (rows x k, quantized) . X[tokens][k]; X and Y are f32.
 * Router of quant.matmul (ops.js:827-1101): tokens <= GEMV max -> GEMV;
 * Q8_0/Q8_0R at tokens >= GEMM min -> fp16 MFMA GEMM (the reference's
 * DRIFT/GEMM2 types, kernels.drift.wgsl.js:33); Q2_K, Q4_K, IQ2_XXS, Q6_K and
 * Q8_0/Q8_0R below GEMM min, from EFF_OPT_SPLIT_MIN_TOKENS (5 for Q2_K and
 * IQ2_XXS, 9 for the others) -> split-x product (f32-accurate; fewer tokens
 * run the int8 matrix-core GEMVs, as accurate, and the split-x product from 2
 * tokens where those cannot hold x's digits in LDS at this k); otherwise (k
 * not a multiple of 256) -> GEMV over token groups, f32-accurate. Where few
 * rows leave CUs idle the GEMM and the split-x product cut k into slices over
 * workgroups (fixed bits for a shape). Q8_0R gives the bits of the Q8_0
 * tensor it was repacked from on every path.
 * EFF_E_SHAPE if k % block_elems != 0. */
int eff_qmatmul(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y,
                uint32_t rows, uint32_t k, uint32_t tokens);

/* eff_qmatmul with x prepared once for several products. The router's
 * split-x product and fp16 GEMM read x in a prepared form (fp16 hi/lo parts
 * with block scales; fp16 tiles); the matmuls of one activation (q, k and v;
 * gate and up) can share it, as the reference shares its fp16 x across the
 * GEMMs of one activation (aF16, ops.gemm2.js:151-196). An extension of
 * quant.matmul (ops.js:827-1101), which has no such step; the outputs are its
 * bits all the same:
 *  - eff_qmatmul_x_layout: the bytes of the prepared x the router's path for
 *    this call reads, and an id of its layout: calls whose ids, tokens and k
 *    agree can share one prepared x (the split-x layouts are shared across
 *    IQ2_XXS, Q8_0 and Q6_K, and across any rows). EFF_NOT_APPLICABLE where
 *    the path reads x itself (the GEMVs, including the one-launch split-x
 *    product up to 8 tokens, and the token groups): run eff_qmatmul.
 *  - eff_qmatmul_prepare_x: x (tokens x k f32) into xp in that layout.
 *  - eff_qmatmul_prepared: the product from xp; the same bits as eff_qmatmul
 *    over the x xp was prepared from (with the same tokens, k and a type of
 *    the same layout). EFF_NOT_APPLICABLE as eff_qmatmul_x_layout. */
int eff_qmatmul_x_layout(eff_ctx *ctx, int type, uint32_t rows, uint32_t k, uint32_t tokens, size_t *bytes,
                         uint32_t *layout);
int eff_qmatmul_prepare_x(eff_ctx *ctx, int type, eff_buf *x, eff_buf *xp, uint32_t rows, uint32_t k,
                          uint32_t tokens);
int eff_qmatmul_prepared(eff_ctx *ctx, int type, eff_buf *w, eff_buf *xp, eff_buf *y, uint32_t rows, uint32_t k,
                         uint32_t tokens);

/* Y = W . X for Q8_0 with the reference CPU path's arithmetic (cpu-kernels.js
 * matvec_q8_0 / matmul_q8_0 via mm, cpu.js:350-381, over the row chunks of
 * cpu-trabajo.js:27-72), on the GPU: each token's x in 8-bit blocks of 32
 * (d = max|x| / 127, q = round(x / d) ties away from zero; BACT = 40,
 * cpu.js:24-27), per block the exact int32 dot of the quants, per row the
 * terms f32(isum) * (d_w * d_x) added in block order, each operation rounded
 * on its own. The outputs are the bits of that path as restated and pinned
 * (or_cpu_matmul); they differ from eff_qmatmul's f32-accurate ones by the
 * 8-bit activations (about 5e-3 relative L2). EFF_NOT_APPLICABLE for other
 * types (the CPU path's kernels are Q8_0 and Q4_0, cpu-trabajo.js:31);
 * EFF_E_SHAPE if k % 32 != 0; EFF_E_INVALID for tokens * k / 32 >= 2^31. */
int eff_qmatmul_cpu_path(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y,
                         uint32_t rows, uint32_t k, uint32_t tokens);

/* The decode GEMV alone (quant.gemv.matmul, ops.gemv.js:148-164): f32
 * accumulation, 1..GEMV max tokens. EFF_NOT_APPLICABLE outside that range. */
int eff_qgemv(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y,
              uint32_t rows, uint32_t k, uint32_t tokens);

/* Fused decode GEMV over matrices of one type and k that share x, 1..3
 * tokens, one launch with x prepared once. Replaces quant.gemv.secciones
 * (ops.gemv.js:192-215; mode EFF_GEMV_SECTIONS, n = 2..4, ys[i] = W_i x with
 * rows[i] rows) and quant.gemv.gateUp (ops.gemv.js:166-190; mode
 * EFF_GEMV_SWIGLU, n = 2, rows[0] == rows[1], ys[0] = silu(W_0 x) * (W_1 x),
 * silu(v) = v / (1 + exp(-v))). Every output equals the one-matrix GEMV's
 * bits when the planner gives both the same k split (always for gate + up).
 * EFF_NOT_APPLICABLE (the reference's null) for other n or tokens, or when the
 * f32 vector GEMV is selected; EFF_E_SHAPE for gate and up of unequal rows. */
int eff_qgemv_multi(eff_ctx *ctx, int type, int mode, uint32_t n, eff_buf *const *ws, eff_buf *x,
                    eff_buf *const *ys, const uint32_t *rows, uint32_t k, uint32_t tokens);

/* The prefill GEMM alone (quant.gemm2.matmul, ops.gemm2.js:266-280): x and
 * the dequantized weights rounded to fp16, MFMA with fp32 accumulation.
 * EFF_NOT_APPLICABLE when tokens < GEMM min (planGemm2 returning null). */
int eff_qgemm(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y,
              uint32_t rows, uint32_t k, uint32_t tokens);

/* The prefill GEMM over `tokens` rows of x with the kernel configuration
 * eff_qgemm chooses for `plan_tokens` tokens (tokens <= plan_tokens). A row's
 * output depends only on its x row and W, summed in that configuration's
 * order, so tokens = 1 with the last x row of a batch gives the bits of the
 * batch's last output row: gemm2.cola (ops.gemm2.js:282-303).
 * EFF_NOT_APPLICABLE when plan_tokens < GEMM min. */
int eff_qgemm_planned(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y,
                      uint32_t rows, uint32_t k, uint32_t tokens, uint32_t plan_tokens);

/* x prepared once for several GEMMs: the reference converts x to fp16 once
 * per activation and reuses it across the matmuls that read it (aF16, a memo
 * keyed on the pool's allocation mark, ops.gemm2.js:151-196; cleared by
 * olvida(), ops.gemm2.js:266). The JS host keeps that memo; the library
 * provides the three steps:
 *  - eff_gemm_x_layout: the bytes of x prepared for a GEMM of `tokens` rows
 *    under the plan of `plan_tokens` (the configuration eff_qgemm_planned
 *    would run), and an id of the layout: products whose ids, tokens and k
 *    agree can share one prepared x. NOT_APPLICABLE where the GEMM is not.
 *  - eff_gemm_prepare_x: x rounded to fp16 (RNE; f32AF16Shader,
 *    kernels.drift.wgsl.js:34-63) into xh, in that layout.
 *  - eff_qgemm_prepared: the GEMM from the prepared x: the same bits as
 *    eff_qgemm_planned over x. */
int eff_gemm_x_layout(eff_ctx *ctx, int type, uint32_t rows, uint32_t k, uint32_t tokens, uint32_t plan_tokens,
                      size_t *bytes, uint32_t *layout);
int eff_gemm_prepare_x(eff_ctx *ctx, int type, eff_buf *x, eff_buf *xh, uint32_t rows, uint32_t k, uint32_t tokens,
                       uint32_t plan_tokens);
int eff_qgemm_prepared(eff_ctx *ctx, int type, eff_buf *w, eff_buf *xh, eff_buf *y, uint32_t rows, uint32_t k,
                       uint32_t tokens, uint32_t plan_tokens);

/* Dequantize n_blocks blocks to f32, bit-exact with the reference decoders
 * (quant.dequant, ops.js:813-823; dequantShader, kernels.wgsl.js:903-922). */
int eff_dequant(eff_ctx *ctx, int type, eff_buf *w, eff_buf *out, uint32_t n_blocks);

/* Rows of a quantized table as f32, the embedding lookup: out[t][0..dim) is
 * the dequantized row ids[t] of w for t < tokens (ids: u32 in a device buffer;
 * an id past the table reads zeros). Bit-identical to eff_dequant of that row.
 * Replaces quant.gather (ops.js:1104-1118). EFF_E_SHAPE if dim % block_elems. */
int eff_gather(eff_ctx *ctx, int type, eff_buf *w, eff_buf *ids, eff_buf *out, uint32_t dim, uint32_t tokens);

/* The gather fused with the first layer's RMS norm (fusion.gatherNorma,
 * ops.fusion.js:154-170; kernels.fusion.wgsl.js:164-206): x as eff_gather, and
 * nrm[t][c] = x[t][c] * (1 / sqrt(sum_c x[t][c]^2 / dim + eps)) * wn[c].
 * dim <= 32768. EFF_E_TYPE for IQ2_XXS (the reference's closed list,
 * kernels.fusion.wgsl.js:159-161). */
int eff_gather_norm(eff_ctx *ctx, int type, eff_buf *w, eff_buf *ids, eff_buf *wn, float eps, eff_buf *x,
                    eff_buf *nrm, uint32_t dim, uint32_t tokens);

/* Exact top-m of logits[base .. base+vocab) ordered by (f32 value desc with
 * -0 == +0, index asc), plus the raw logits of the penalised ids. Writes the
 * reference's output record into `out` (kernels.topk.wgsl.js:50-59):
 *   u32[0] candidates, [1] flags (2 = NaN seen, 1|4 = overflow), [2] n_penal,
 *   [3] chunks, [4] serial, [5..7] 0, then EFF_TOPK_P_MAX penalised-logit bit
 *   patterns, then EFF_TOPK_CAP (id, bits) pairs.
 * Pairs are written sorted by (value desc, index asc). Replaces
 * createTopKGPU().candidatos (ops.topk.js:99-165). */
int eff_topk(eff_ctx *ctx, eff_buf *logits, uint32_t base, uint32_t vocab, uint32_t m,
             const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, eff_buf *out);

/* The decode head: y[0 .. rows) = W x for one token (as eff_qmatmul with
 * tokens = 1), then the exact top-m of y written to `out` exactly as
 * eff_topk(y, 0, rows, m, penal_ids, n_penal, serial, out) writes it. This is
 * the output projection fused with top-k = 40 of north_star's configuration
 * 4; the reference runs the two as separate passes (model.js:1145-1177, then
 * createTopKGPU().candidatos, ops.topk.js:99-165). For Q6_K matrices of
 * 32768 .. 131072 rows every workgroup of the GEMV also writes the top-k
 * record of its rows (128 on average), and one more launch selects from the
 * records; other
 * shapes run the GEMV and eff_topk. The same NOT_APPLICABLE cases as
 * eff_topk, checked before anything is enqueued. */
int eff_qgemv_topk(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k,
                   uint32_t m, const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, eff_buf *out);

/* eff_topk without any device allocation. No counterpart in the reference:
 * it is for callers that cannot allocate (code under HIP graph capture,
 * serving loops that forbid hipMalloc). The top-k's group records go to a
 * fixed device array of the library (18 KiB, one per GPU, held until the
 * process ends) instead of the context's scratch; it holds the records of
 * every vocabulary eff_topk accepts (vocab < EFF_TOPK_N_MAX), and a call that
 * would need more is refused with EFF_E_BOUNDS. Same output and
 * NOT_APPLICABLE cases as eff_topk. Calls that overlap on one GPU (several
 * streams or contexts at once) share the array and race. */
#define EFF_TOPK_NOALLOC_SCRATCH_BYTES 18432u
int eff_topk_noalloc(eff_ctx *ctx, eff_buf *logits, uint32_t base, uint32_t vocab, uint32_t m,
                     const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, eff_buf *out);

/* Size in bytes of the top-k output record (topkBytesSalida). */
size_t eff_topk_out_bytes(void);

/* ---- measurement --------------------------------------------------------- */

/* No counterpart in the reference: a streaming read of the first `bytes` bytes
 * of `src`, on the context's stream, by `workgroups` (1..65535) workgroups of
 * 256 threads, each reading one contiguous chunk with 16-byte loads, `unroll`
 * (1, 2 or 4) in flight per lane. It computes nothing visible (`sink`, at least
 * 4 * workgroups bytes, is written only if a workgroup's XOR of its bytes equals
 * a fixed constant). The time of the same bytes read this way is the floor the
 * benchmark holds each GEMV against, beside the HBM roofline. */
int eff_read_floor(eff_ctx *ctx, eff_buf *src, size_t bytes, uint32_t workgroups, uint32_t unroll, eff_buf *sink);

#ifdef __cplusplus
}
#endif

#endif /* ELFFUSS_AMD_H */
