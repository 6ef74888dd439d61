// C ABI of the quantized matrix-product path: contexts, device buffers,
// repack marks, the matmul router and the op entry points. Declarations and
// the reference interfaces they replace are in include/elffuss_amd.h.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/elffuss_amd.h"
#include "eff_formats.h"
#include "eff_kernels.h"

using namespace eff;

// Scratch of eff_topk_noalloc: the top-k group records of one call, in a
// fixed device array of 18 KiB (the records of the largest vocabulary the
// top-k accepts). Every GPU the library runs on holds its own copy until the
// process ends. Host code never uses the array's name as an address: eff_init
// looks up each device's copy once, with that device current
// (hipGetSymbolAddress), and the entry point passes that pointer. The first
// kernel writes every record the second reads, so no call needs the array
// cleared; calls that overlap on one GPU share it and race.
static constexpr size_t kNoAllocBytes = eff::kTopkScratchMax;
static_assert(eff::topk_scratch_bytes_for(EFF_TOPK_N_MAX - 1u) <= kNoAllocBytes, "no-alloc scratch too small");
static_assert(kNoAllocBytes == EFF_TOPK_NOALLOC_SCRATCH_BYTES, "no-alloc scratch size differs from the header's");
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];        // per device: the address of its `scratch`
hipError_t g_scratch_err[kMaxDevices];   // per device: the lookup's result, once done
bool g_scratch_done[kMaxDevices];
}  // namespace

// Bytes allocated past every eff_buf_alloc request. Kernels read at most 4
// bytes past a block (the reference's loader slack, model.js:248-254).
static constexpr size_t kSlack = 256;

// How long eff_read_end polls a read's completion before a blocking wait.
static constexpr int64_t kReadSpinNs = 2000000;

// Pinned blocks of finished reads (eff_read_begin / eff_read_end), reused.
// Shared by a context and its live read tickets; the last owner frees them.
struct ReadPool {
  std::mutex mu;
  std::vector<std::pair<void *, size_t>> blocks;
  std::vector<hipEvent_t> events;   // completed tickets' events, for reuse
  ~ReadPool() {
    for (auto &b : blocks) (void)hipHostFree(b.first);
    for (hipEvent_t ev : events) (void)hipEventDestroy(ev);
  }
};

struct eff_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  std::string error;
  int64_t gemv_max_tokens = 8;
  int64_t gemm_min_tokens = 64;
  int64_t gemv_kernel = 0;
  eff_stats stats{};
  void *topk_scratch = nullptr;
  size_t topk_scratch_bytes = 0;
  void *xh_scratch = nullptr;       // fp16 copy of the GEMM activations
  size_t xh_scratch_bytes = 0;
  void *sx_scratch = nullptr;       // x as fp16 hi/lo parts for the split-x product
  size_t sx_scratch_bytes = 0;
  int64_t sx_config = 0;
  int64_t gemm_config = 0;
  int64_t gemm_split = 0;           // Q8_0 GEMM k slices (0: automatic)
  int64_t sx_split = 0;             // split-x k slices (0: automatic)
  void *sk_scratch = nullptr;       // k-slice counters and sums (GEMM and split-x)
  size_t sk_scratch_bytes = 0;
  hipEvent_t order_ev = nullptr;    // orders a newly set stream after the previous one
  int64_t sx_min_tokens = 0;        // 0: the measured default (sx_routes)
  void *act_scratch = nullptr;      // x in the CPU path's 8-bit blocks (eff_qmatmul_cpu_path)
  size_t act_scratch_bytes = 0;
  // Pinned staging ring of eff_buf_write: the source bytes are copied here on
  // the calling thread and the device copy is enqueued from here, so a write
  // returns without waiting for the device. `pend` holds the ring ranges whose
  // copies may still be in flight, oldest first, with the event after each.
  struct Pend {
    size_t a, b;
    hipEvent_t ev;
  };
  uint8_t *stage = nullptr;
  size_t stage_head = 0;
  std::deque<Pend> stage_pend;
  std::vector<hipEvent_t> events;   // recorded and completed, ready for reuse
  std::shared_ptr<ReadPool> reads = std::make_shared<ReadPool>();
};

// An enqueued device -> host read (eff_read_begin). The ticket keeps the
// device number and a reference to its context's pool of pinned blocks, never
// the context itself: it may be waited for and released after eff_shutdown.
struct eff_read {
  int device = 0;
  std::shared_ptr<ReadPool> pool;
  void *host = nullptr;   // pinned block of `cap` bytes
  size_t cap = 0, n = 0;
  hipEvent_t ev = nullptr;
  int rc = EFF_OK;
  std::string error;
};

struct eff_buf {
  void *ptr = nullptr;
  size_t size = 0;
  bool owned = false;
  int mark_type = 0;        // EFF_TYPE_Q8_0R when marked
  uint32_t mark_blocks = 0; // N of the tensor
};

// The launches of one recording (eff_graph_begin .. eff_graph_end), ready to
// be replayed on a context's stream.
struct eff_graph {
  int device = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  size_t nodes = 0;
};

namespace {

int fail(eff_ctx *ctx, int code, const char *fmt, ...) {
  if (ctx) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    ctx->error = buf;
  }
  return code;
}

int hip_fail(eff_ctx *ctx, hipError_t e, const char *what) {
  return fail(ctx, EFF_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define EFF_HIP(ctx, call)                              \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
  } while (0)

// Select the context's device for the calling thread.
int use_device(eff_ctx *ctx) {
  EFF_HIP(ctx, hipSetDevice(ctx->device));
  return EFF_OK;
}

// An output buffer of at least `bytes` bytes, 16-byte aligned.
int check_out(eff_ctx *ctx, eff_buf *b, uint64_t bytes, const char *who) {
  if (!b) return fail(ctx, EFF_E_INVALID, "%s: null buffer", who);
  if (bytes > b->size)
    return fail(ctx, EFF_E_BOUNDS, "%s: needs %llu bytes and the buffer has %zu", who, (unsigned long long)bytes,
                b->size);
  if ((uintptr_t)b->ptr & 15) return fail(ctx, EFF_E_INVALID, "%s: device buffers must be 16-byte aligned", who);
  return EFF_OK;
}

// EFF_E_INVALID when the context's stream is being recorded into a graph:
// for the calls that wait for the device, allocate or move host data, none
// of which a replay could repeat.
int refuse_capture(eff_ctx *ctx, const char *who) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  EFF_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return fail(ctx, EFF_E_INVALID, "%s: not allowed while the stream is recorded into a graph", who);
  return EFF_OK;
}

// Validate a matmul-shaped call and build the weight view. Mirrors the checks
// of quant.matmul (ops.js:846-870): known type, k a multiple of the block,
// repacked buffers marked with the tensor's N and not read beyond it.
int weight_view(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k,
                uint32_t tokens, WeightView &wv, const char *who) {
  if (!ctx) return EFF_E_INVALID;
  if (!w || !x || !y) return fail(ctx, EFF_E_INVALID, "%s: null buffer", who);
  if (!type_known(type)) return fail(ctx, EFF_E_TYPE, "%s: unsupported quantization type %d", who, type);
  if (rows == 0 || k == 0 || tokens == 0) return fail(ctx, EFF_E_INVALID, "%s: empty shape rows=%u k=%u tokens=%u", who, rows, k, tokens);
  Geometry g = geometry(type);
  if (k % g.elems) return fail(ctx, EFF_E_SHAPE, "%s %s: k=%u is not a multiple of %u", who, eff_type_name(type), k, g.elems);
  const uint32_t bpr = k / g.elems;
  const uint64_t nblocks = (uint64_t)rows * bpr;
  wv.w = (const uint8_t *)w->ptr;
  wv.type = type;
  wv.rows = rows;
  wv.k = k;
  wv.bpr = bpr;
  wv.row_bytes = (uint64_t)bpr * g.bytes;
  wv.scales_off = 0;
  wv.w_bytes = w->size + (w->owned ? kSlack : 16);  // wrapped buffers guarantee 16 readable bytes
  if (type == EFF_TYPE_Q8_0R) {
    if (w->mark_type != EFF_TYPE_Q8_0R)
      return fail(ctx, EFF_E_MARK, "%s Q8_0R: the buffer does not carry the mark of a repacked tensor "
                  "(eff_buf_mark_r); the scale region is located from the tensor's block count", who);
    if (nblocks > w->mark_blocks)
      return fail(ctx, EFF_E_MARK, "%s Q8_0R: the call reads %llu blocks and the tensor has %u", who,
                  (unsigned long long)nblocks, w->mark_blocks);
    wv.scales_off = (uint64_t)32 * w->mark_blocks;
  } else if (nblocks * g.bytes > w->size) {
    return fail(ctx, EFF_E_BOUNDS, "%s %s: W needs %llu bytes and the buffer has %zu", who, eff_type_name(type),
                (unsigned long long)(nblocks * g.bytes), w->size);
  }
  if ((uint64_t)tokens * k * 4 > x->size)
    return fail(ctx, EFF_E_BOUNDS, "%s: x needs %llu bytes and the buffer has %zu", who,
                (unsigned long long)tokens * k * 4, x->size);
  if ((uint64_t)tokens * rows * 4 > y->size)
    return fail(ctx, EFF_E_BOUNDS, "%s: y needs %llu bytes and the buffer has %zu", who,
                (unsigned long long)tokens * rows * 4, y->size);
  if (((uintptr_t)x->ptr | (uintptr_t)y->ptr | (uintptr_t)w->ptr) & 15)
    return fail(ctx, EFF_E_INVALID, "%s: device buffers must be 16-byte aligned", who);
  return EFF_OK;
}

int run_sx(eff_ctx *ctx, const WeightView &wv, const float *x, float *y, uint32_t tokens);

// Types whose prefill the router sends to the fp16 GEMM: those the
// reference's fp16 GEMMs accept (GEMM2_TIPOS, kernels.gemm2.wgsl.js:51).
bool router_gemm_type(int type) { return type == EFF_TYPE_Q8_0 || type == EFF_TYPE_Q8_0R; }

// The 16-row GEMV computes tokens in groups of 4: at 5 and 6 tokens it pays
// for 8, and the 4-row GEMV (which scales with the token count) is faster
// (µs, 5 / 6 tokens, 16-row against 4-row: Q8_0 8192 x 2048 9.00 / 9.24
// against 8.21 / 8.70, 4096 x 4096 10.63 / 10.98 against 9.59 / 10.63; Q4_K
// 8192 x 2048 7.46 / 7.73 against 6.69 / 7.18; Q6_K 4096 x 4096 11.80 /
// 12.17 against 11.10 / 12.07); at 4, 7 and 8 tokens the 16-row GEMV is as
// fast or faster.
bool mt_routes(uint32_t tokens) { return tokens != 5u && tokens != 6u; }

// The split-x product from 5 tokens (Q4_K: 9); below, the int8 matrix-core
// GEMVs, which are as accurate and faster at 4 tokens (C5 shapes: 5.75 / 6.72
// us against 7.32 / 7.33 for Q2_K / IQ2_XXS); from 5 tokens split-x is as fast
// or faster for those two types (5: 7.42 / 7.42 against 7.49 / 8.62; 7: 7.52 /
// 7.56 against 7.75 / 8.90), for Q4_K from 9 (8: 8.66 against 7.90).
// Q8_0, Q8_0R and Q6_K take it from 9 tokens, where the GEMV would run over
// token groups; Q8_0 and Q8_0R only below the fp16 GEMM's threshold (from
// there the reference's DRIFT path, whose fp16 roundings the GEMM keeps).
// Below that, from 2 tokens, also where no int8 matrix-core GEMV fits its x
// digits into LDS at this k (about 43 K token x k values: 4096 x 14336 from 3
// tokens, 2048 x 8192 from 6), which would leave the f32 vector GEMV a pass
// over the weights per token group (Q8_0 4096 x 14336, 8 tokens: 102.9 us).
bool sx_routes(const eff_ctx *ctx, const WeightView &wv, uint32_t tokens) {
  const int64_t lo = ctx->sx_min_tokens ? ctx->sx_min_tokens
                                        : (wv.type == Q2_K || wv.type == IQ2_XXS ? 5 : 9);
  if (router_gemm_type(wv.type) && (int64_t)tokens >= ctx->gemm_min_tokens) return false;
  if (ctx->gemv_kernel != 0 || !sx_applies(wv, tokens)) return false;
  if ((int64_t)tokens >= lo) return true;
  // From 7 tokens where k > 4096, every type: the 16-row GEMV then holds the
  // x digits of 7-8 tokens in 97 KB of LDS or more, one workgroup per CU (us,
  // 7 / 8 tokens, the GEMV against the split-x product: Q8_0 4096 x 4608 20.2 /
  // 20.8 against 14.5, 5120 x 5120 31.9 / 33.0 against 23.6, 13824 x 5120 45.2 /
  // 46.8 against 34.8; Q4_K 4096 x 4608 19.1 / 19.6 against 11.6; Q6_K 20.5 /
  // 20.9 against 16.6 at 4096 x 5120). Where k = 4096, Q4_K and Q6_K from 5120
  // rows (Q4_K 6144 x 4096 17.3 / 17.9 against 12.7, 14336 x 4096 23.1 / 23.7
  // against 19.4 / 19.6, 32000 x 4096 34.5 / 37.3 against 30.0 / 30.2; Q6_K
  // 6144 x 4096 22.3 / 22.9 against 16.6 / 16.7, 14336 x 4096 32.7 / 32.9 against
  // 29.4; where the GEMV's row tiles fill the CUs evenly it is faster: Q6_K
  // 16384 x 4096 26.2 / 27.1 against 30.0), not Q8_0 (14336 x 4096 27.6 / 27.9
  // against 29.1) nor at 4096 rows (Q4_K 10.0 / 10.3 against 10.6). At 5 and 6
  // tokens the 4-row GEMV stays (Q8_0 5120 x 5120 at 5: 20.8 against 23.6;
  // 13824 x 5120 at 6: 27.1 against 34.7; Q4_K at 6 would gain 4-15%, Q6_K
  // -2 to 8%).
  if (!ctx->sx_min_tokens && tokens >= 7u &&
      (wv.k > 4096u || (wv.k == 4096u && (wv.type == Q4_K || wv.type == Q6_K) && wv.rows >= 5120u)))
    return true;
  GemvPlan p;
  return !gemv_rows_applies(wv, tokens) && !(mt_routes(tokens) && gemv_mt_plan(wv, tokens, p)) &&
         !gemv_mx_plan(wv, tokens, p);
}


int run_gemv(eff_ctx *ctx, const WeightView &wv, const float *x, float *y, uint32_t tokens) {
  if (sx_routes(ctx, wv, tokens)) return run_sx(ctx, wv, x, y, tokens);
  GemvPlan p;
  hipError_t e;
  if (ctx->gemv_kernel == 0 && gemv_rows_applies(wv, tokens)) {
    e = launch_gemv_rows(wv, x, y, ctx->stream);
  } else if (ctx->gemv_kernel == 0 && mt_routes(tokens) && gemv_mt_plan(wv, tokens, p)) {
    e = launch_gemv_mt(wv, x, y, tokens, p, ctx->stream);
  } else if (ctx->gemv_kernel == 0 && gemv_mx_plan(wv, tokens, p)) {
    e = launch_gemv_mx(wv, x, y, tokens, p, ctx->stream);
  } else {
    p = plan_gemv(wv, tokens);
    e = launch_gemv(wv, x, y, tokens, p, ctx->stream);
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "gemv launch");
  return EFF_OK;
}

// Grow a context-owned scratch buffer (outside of any graph capture: the
// first call of a shape must be eager).
int grow(eff_ctx *ctx, void **p, size_t *have, size_t need, const char *what) {
  if (need <= *have) return EFF_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  EFF_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return fail(ctx, EFF_E_INVALID, "%s scratch of %zu bytes: it cannot grow while the stream is recorded into a "
                "graph; run the largest call of this shape once before the recording", what, need);
  if (*p) {
    EFF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    (void)hipFree(*p);
    *p = nullptr;
    *have = 0;
  }
  if (hipMalloc(p, need) != hipSuccess) return fail(ctx, EFF_E_NOMEM, "%s scratch of %zu bytes", what, need);
  *have = need;
  return EFF_OK;
}

// The k-slice scratch of a call, `need` bytes (null where the call takes no
// k slices). A new allocation gets its counters zeroed (outside of any graph
// capture: grow allocates eagerly only); every launch leaves them zero.
int sk_get(eff_ctx *ctx, size_t need, void **out) {
  *out = nullptr;
  if (!need) return EFF_OK;
  const size_t before = ctx->sk_scratch_bytes;
  const int rc = grow(ctx, &ctx->sk_scratch, &ctx->sk_scratch_bytes, need, "k-slice");
  if (rc) return rc;
  if (ctx->sk_scratch_bytes != before) EFF_HIP(ctx, hipMemsetAsync(ctx->sk_scratch, 0, ctx->sk_scratch_bytes, ctx->stream));
  *out = ctx->sk_scratch;
  return EFF_OK;
}

// The GEMM's k-slice scratch.
int sk_scratch(eff_ctx *ctx, const WeightView &wv, uint32_t tokens, uint32_t plan, void **out) {
  return sk_get(ctx, gemm_sk_bytes(wv.type, tokens, plan, wv.k, wv.rows, (uint32_t)ctx->gemm_config,
                                   (uint32_t)ctx->gemm_split), out);
}

// Split-x matrix-core product (Q2_K, Q4_K, IQ2_XXS, Q8_0, Q8_0R, Q6_K from 2
// tokens, f32-accurate).
int run_sx(eff_ctx *ctx, const WeightView &wv, const float *x, float *y, uint32_t tokens) {
  int rc = grow(ctx, &ctx->sx_scratch, &ctx->sx_scratch_bytes, sx_x_bytes(wv.type, tokens, wv.k), "split-x");
  if (rc) return rc;
  const uint32_t ks = (uint32_t)ctx->sx_split;
  void *sk;
  if ((rc = sk_get(ctx, sx_sk_bytes(wv, tokens, (int)ctx->sx_config, ks), &sk))) return rc;
  hipError_t e = launch_sx(wv, x, y, tokens, ctx->sx_scratch, (int)ctx->sx_config, ks, sk, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "split-x launch");
  ++ctx->stats.split;
  if (sx_x_layout(wv, tokens, (int)ctx->sx_config, ks)) ++ctx->stats.split_x;
  return EFF_OK;
}

// The prepared x the router's path for a call reads (eff_qmatmul_x_layout):
// a split-x layout, the fp16 GEMM's, or 0 where the path reads x itself. The
// same decisions, in the same order, as eff_qmatmul.
uint32_t route_layout(const eff_ctx *ctx, const WeightView &wv, uint32_t tokens, size_t *bytes) {
  *bytes = 0;
  if (sx_routes(ctx, wv, tokens)) {
    const uint32_t l = sx_x_layout(wv, tokens, (int)ctx->sx_config, (uint32_t)ctx->sx_split);
    if (l) *bytes = sx_prepared_bytes(l, tokens, wv.k);
    return l;
  }
  const bool gemv = (int64_t)tokens <= ctx->gemv_max_tokens && tokens <= 8;
  if (!gemv && (int64_t)tokens >= ctx->gemm_min_tokens && router_gemm_type(wv.type)) {
    const uint32_t cfg = (uint32_t)ctx->gemm_config;
    *bytes = gemm_x_bytes(wv.type, tokens, tokens, wv.k, wv.rows, cfg);
    return gemm_x_layout(wv.type, tokens, wv.k, wv.rows, cfg);
  }
  return 0u;
}

// The shape checks of the prepared-x router entry points, and the routing
// view of the call (type, rows, k; no buffers).
int matmul_prepared_view(eff_ctx *ctx, int type, uint32_t rows, uint32_t k, uint32_t tokens, WeightView &wv,
                         const char *who) {
  if (!type_known(type)) return fail(ctx, EFF_E_TYPE, "%s: unsupported quantization type %d", who, type);
  if (rows == 0 || k == 0 || tokens == 0)
    return fail(ctx, EFF_E_INVALID, "%s: empty shape rows=%u k=%u tokens=%u", who, rows, k, tokens);
  const Geometry g = geometry(type);
  if (k % g.elems) return fail(ctx, EFF_E_SHAPE, "%s %s: k=%u is not a multiple of %u", who, eff_type_name(type), k, g.elems);
  wv = WeightView{};
  wv.type = type;
  wv.rows = rows;
  wv.k = k;
  wv.bpr = k / g.elems;
  return EFF_OK;
}

int run_gemm(eff_ctx *ctx, const WeightView &wv, const float *x, float *y, uint32_t tokens, uint32_t plan) {
  const uint32_t cfg = (uint32_t)ctx->gemm_config;
  int rc = grow(ctx, &ctx->xh_scratch, &ctx->xh_scratch_bytes,
                gemm_x_bytes(wv.type, tokens, plan, wv.k, wv.rows, cfg), "gemm x");
  if (rc) return rc;
  void *sk;
  if ((rc = sk_scratch(ctx, wv, tokens, plan, &sk))) return rc;
  hipError_t e = launch_gemm(wv, x, y, tokens, plan, cfg, (uint32_t)ctx->gemm_split, ctx->xh_scratch, sk,
                             ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "gemm launch");
  ++ctx->stats.gemm_x;
  return EFF_OK;
}

// The checks shared by the prepared-x GEMM entry points: the GEMM applies
// (NOT_APPLICABLE otherwise, as eff_qgemm_planned), tokens under the plan.
int gemm_prepared_check(eff_ctx *ctx, int type, uint32_t rows, uint32_t k, uint32_t tokens, uint32_t plan,
                        const char *who) {
  if (!type_known(type)) return fail(ctx, EFF_E_TYPE, "%s: unsupported quantization type %d", who, type);
  if (rows == 0 || k == 0 || tokens == 0)
    return fail(ctx, EFF_E_INVALID, "%s: empty shape rows=%u k=%u tokens=%u", who, rows, k, tokens);
  const Geometry g = geometry(type);
  if (k % g.elems) return fail(ctx, EFF_E_SHAPE, "%s %s: k=%u is not a multiple of %u", who, eff_type_name(type), k, g.elems);
  if (plan == 0 || (int64_t)plan < ctx->gemm_min_tokens) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  if (tokens > plan) return fail(ctx, EFF_E_INVALID, "%s: %u tokens under the plan of %u", who, tokens, plan);
  return EFF_OK;
}

// Writes of at most this many bytes go through the staging ring and return
// without waiting; the ring holds twice as much.
constexpr size_t kStageMaxWrite = (size_t)4 << 20;
constexpr size_t kStageBytes = 2 * kStageMaxWrite;

int take_event(eff_ctx *ctx, hipEvent_t *ev) {
  if (!ctx->events.empty()) {
    *ev = ctx->events.back();
    ctx->events.pop_back();
    return EFF_OK;
  }
  EFF_HIP(ctx, hipEventCreateWithFlags(ev, hipEventDisableTiming));
  return EFF_OK;
}

// A range of `n` bytes of the staging ring whose earlier copies have ended.
int stage_reserve(eff_ctx *ctx, size_t n, uint8_t **out) {
  if (!ctx->stage) {
    void *p = nullptr;
    if (hipHostMalloc(&p, kStageBytes, hipHostMallocDefault) != hipSuccess)
      return fail(ctx, EFF_E_NOMEM, "pinned staging of %zu bytes", kStageBytes);
    ctx->stage = (uint8_t *)p;
    ctx->stage_head = 0;
  }
  // retire the copies that have ended (oldest first)
  while (!ctx->stage_pend.empty() && hipEventQuery(ctx->stage_pend.front().ev) == hipSuccess) {
    ctx->events.push_back(ctx->stage_pend.front().ev);
    ctx->stage_pend.pop_front();
  }
  size_t a = ctx->stage_head;
  if (a + n > kStageBytes) a = 0;
  const size_t b = a + n;
  for (auto it = ctx->stage_pend.begin(); it != ctx->stage_pend.end();) {
    if (it->a < b && a < it->b) {
      EFF_HIP(ctx, hipEventSynchronize(it->ev));
      ctx->events.push_back(it->ev);
      it = ctx->stage_pend.erase(it);
    } else {
      ++it;
    }
  }
  ctx->stage_head = b;
  *out = ctx->stage + a;
  return EFF_OK;
}

// Record the end of the copy just enqueued from stage[a, a + n).
int stage_commit(eff_ctx *ctx, size_t a, size_t n) {
  hipEvent_t ev;
  int rc = take_event(ctx, &ev);
  if (rc) return rc;
  EFF_HIP(ctx, hipEventRecord(ev, ctx->stream));
  ctx->stage_pend.push_back({a, a + n, ev});
  return EFF_OK;
}

}  // namespace

extern "C" {

int eff_init(int device, eff_ctx **out) {
  if (!out) return EFF_E_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return EFF_E_DEVICE;
  eff_ctx *ctx = new eff_ctx();
  ctx->device = device;
  if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking) != hipSuccess) {
    delete ctx;
    return EFF_E_DEVICE;
  }
  ctx->stream = ctx->own;
  if (device < kMaxDevices) {
    // once per device, with the device current: the address of its copy of
    // the no-alloc scratch (a lookup, not an allocation)
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_done[device]) {
      void *p = nullptr;
      g_scratch_err[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      g_scratch_ptr[device] = g_scratch_err[device] == hipSuccess ? p : nullptr;
      g_scratch_done[device] = true;
    }
  }
  *out = ctx;
  return EFF_OK;
}

int eff_shutdown(eff_ctx *ctx) {
  if (!ctx) return EFF_E_INVALID;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->topk_scratch) (void)hipFree(ctx->topk_scratch);
  if (ctx->xh_scratch) (void)hipFree(ctx->xh_scratch);
  if (ctx->sx_scratch) (void)hipFree(ctx->sx_scratch);
  if (ctx->act_scratch) (void)hipFree(ctx->act_scratch);
  if (ctx->sk_scratch) (void)hipFree(ctx->sk_scratch);
  if (ctx->order_ev) (void)hipEventDestroy(ctx->order_ev);
  for (auto &p : ctx->stage_pend) (void)hipEventDestroy(p.ev);
  for (hipEvent_t ev : ctx->events) (void)hipEventDestroy(ev);
  if (ctx->stage) (void)hipHostFree(ctx->stage);
  ctx->reads.reset();   // the pinned blocks go with the last live read ticket
  if (ctx->own) (void)hipStreamDestroy(ctx->own);
  delete ctx;
  return EFF_OK;
}

const char *eff_last_error(const eff_ctx *ctx) { return ctx ? ctx->error.c_str() : "no context"; }

void *eff_stream(eff_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

// The context's scratch buffers (and the k-slice counters, which must be
// zero when a launch starts) are reused by every call, so a call on the new
// stream must not overlap one still queued on the previous stream: the new
// stream waits for an event recorded on the previous one. A stream being
// recorded into a graph takes no such wait (its launches run when the graph
// is replayed, which the caller orders); switching away from a stream being
// recorded is refused (the recording would lose the calls that follow).
int eff_set_stream(eff_ctx *ctx, void *hip_stream) {
  if (!ctx) return EFF_E_INVALID;
  const hipStream_t next = hip_stream ? (hipStream_t)hip_stream : ctx->own;
  if (next == ctx->stream) return EFF_OK;
  int rc = use_device(ctx);
  if (rc || (rc = refuse_capture(ctx, "set stream"))) return rc;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  EFF_HIP(ctx, hipStreamIsCapturing(next, &cs));
  if (cs == hipStreamCaptureStatusNone) {
    if (!ctx->order_ev) EFF_HIP(ctx, hipEventCreateWithFlags(&ctx->order_ev, hipEventDisableTiming));
    EFF_HIP(ctx, hipEventRecord(ctx->order_ev, ctx->stream));
    EFF_HIP(ctx, hipStreamWaitEvent(next, ctx->order_ev, 0));
  }
  ctx->stream = next;
  return EFF_OK;
}

int eff_sync(eff_ctx *ctx) {
  if (!ctx) return EFF_E_INVALID;
  int rc = use_device(ctx);
  if (rc || (rc = refuse_capture(ctx, "sync"))) return rc;
  EFF_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return EFF_OK;
}

int eff_set_option(eff_ctx *ctx, int option, int64_t value) {
  if (!ctx) return EFF_E_INVALID;
  switch (option) {
    case EFF_OPT_GEMV_MAX_TOKENS:
      if (value < 0 || value > 8) return fail(ctx, EFF_E_INVALID, "GEMV max tokens must be in 0..8, got %lld", (long long)value);
      ctx->gemv_max_tokens = value;
      return EFF_OK;
    case EFF_OPT_GEMM_MIN_TOKENS:
      if (value < 1) return fail(ctx, EFF_E_INVALID, "GEMM min tokens must be >= 1, got %lld", (long long)value);
      ctx->gemm_min_tokens = value;
      return EFF_OK;
    case EFF_OPT_GEMV_KERNEL:
      if (value < 0 || value > 1) return fail(ctx, EFF_E_INVALID, "GEMV kernel must be 0 or 1, got %lld", (long long)value);
      ctx->gemv_kernel = value;
      return EFF_OK;
    case EFF_OPT_SPLIT_CONFIG:
      if (value < 0 || value > 3) return fail(ctx, EFF_E_INVALID, "split-x configuration must be 0..3, got %lld", (long long)value);
      ctx->sx_config = value;
      return EFF_OK;
    case EFF_OPT_SPLIT_MIN_TOKENS:
      if (value != 0 && value < 4)
        return fail(ctx, EFF_E_INVALID, "split-x min tokens must be 0 or >= 4, got %lld", (long long)value);
      ctx->sx_min_tokens = value;
      return EFF_OK;
    case EFF_OPT_GEMM_CONFIG:
      if (value < 0 || value > 6) return fail(ctx, EFF_E_INVALID, "GEMM configuration must be 0..6, got %lld", (long long)value);
      ctx->gemm_config = value;
      return EFF_OK;
    case EFF_OPT_GEMM_SPLIT:
      if (value < 0 || value > 64) return fail(ctx, EFF_E_INVALID, "GEMM k slices must be 0..64, got %lld", (long long)value);
      ctx->gemm_split = value;
      return EFF_OK;
    case EFF_OPT_SPLIT_SLICES:
      if (value < 0 || value > 64)
        return fail(ctx, EFF_E_INVALID, "split-x k slices must be 0..64, got %lld", (long long)value);
      ctx->sx_split = value;
      return EFF_OK;
    default: return fail(ctx, EFF_E_INVALID, "unknown option %d", option);
  }
}

int eff_get_stats(const eff_ctx *ctx, eff_stats *out) {
  if (!ctx || !out) return EFF_E_INVALID;
  *out = ctx->stats;
  return EFF_OK;
}

int eff_buf_alloc(eff_ctx *ctx, size_t bytes, eff_buf **out) {
  if (!ctx || !out) return EFF_E_INVALID;
  *out = nullptr;
  if (bytes == 0) return fail(ctx, EFF_E_INVALID, "buffer of 0 bytes");
  int rc = use_device(ctx);
  if (rc) return rc;
  // A clear recorded into a graph would be replayed with it (and memset nodes
  // are avoided in captured graphs): buffers are made outside a recording.
  if ((rc = refuse_capture(ctx, "alloc"))) return rc;
  // Stream-ordered allocation from the device's memory pool, so that a
  // buffer can also be given back in stream order (eff_buf_retire).
  void *p = nullptr;
  if (hipMallocAsync(&p, bytes + kSlack, ctx->stream) != hipSuccess)
    return fail(ctx, EFF_E_NOMEM, "allocation of %zu bytes failed", bytes + kSlack);
  // The clear is ordered on the context's stream: every later operation on
  // that stream sees zeros, and the host does not wait.
  if (hipMemsetAsync(p, 0, bytes + kSlack, ctx->stream) != hipSuccess) {
    (void)hipFreeAsync(p, ctx->stream);
    return fail(ctx, EFF_E_DEVICE, "clearing a new buffer failed");
  }
  eff_buf *b = new eff_buf();
  b->ptr = p;
  b->size = bytes;
  b->owned = true;
  *out = b;
  return EFF_OK;
}

int eff_buf_wrap(eff_ctx *ctx, void *device_ptr, size_t bytes, eff_buf **out) {
  if (!ctx || !out || !device_ptr || bytes == 0) return EFF_E_INVALID;
  eff_buf *b = new eff_buf();
  b->ptr = device_ptr;
  b->size = bytes;
  b->owned = false;
  *out = b;
  return EFF_OK;
}

int eff_buf_free(eff_ctx *ctx, eff_buf *buf) {
  if (!ctx || !buf) return EFF_E_INVALID;
  if (buf->owned) {
    // the work of every stream of the device ends first, so nothing still
    // reads the memory when the pool may hand it out again
    int rc = use_device(ctx);
    if (rc || (rc = refuse_capture(ctx, "free"))) return rc;
    (void)hipDeviceSynchronize();
    (void)hipFreeAsync(buf->ptr, ctx->stream);
  }
  delete buf;
  return EFF_OK;
}

int eff_buf_retire(eff_ctx *ctx, eff_buf *buf) {
  if (!ctx || !buf) return EFF_E_INVALID;
  if (buf->owned) {
    int rc = use_device(ctx);
    if (rc || (rc = refuse_capture(ctx, "retire"))) return rc;
    // given back in stream order: the pool reuses the memory only after the
    // work enqueued before this call on the context's stream has run
    EFF_HIP(ctx, hipFreeAsync(buf->ptr, ctx->stream));
  }
  delete buf;
  return EFF_OK;
}

size_t eff_buf_size(const eff_buf *buf) { return buf ? buf->size : 0; }
void *eff_buf_device_ptr(const eff_buf *buf) { return buf ? buf->ptr : nullptr; }

int eff_buf_write(eff_ctx *ctx, eff_buf *buf, size_t off, const void *src, size_t n) {
  if (!ctx || !buf || (!src && n)) return EFF_E_INVALID;
  if (off > buf->size || n > buf->size - off) return fail(ctx, EFF_E_BOUNDS, "write of %zu bytes at %zu past a %zu-byte buffer", n, off, buf->size);
  if (!n) return EFF_OK;
  int rc = use_device(ctx);
  if (rc) return rc;
  if ((rc = refuse_capture(ctx, "write"))) return rc;
  char *dst = (char *)buf->ptr + off;
  if (n > kStageMaxWrite) {
    // Large uploads (weights at load time): the copy is waited for, so `src`
    // may be reused on return.
    EFF_HIP(ctx, hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, ctx->stream));
    EFF_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return EFF_OK;
  }
  uint8_t *st = nullptr;
  if ((rc = stage_reserve(ctx, n, &st))) return rc;
  memcpy(st, src, n);
  EFF_HIP(ctx, hipMemcpyAsync(dst, st, n, hipMemcpyHostToDevice, ctx->stream));
  return stage_commit(ctx, (size_t)(st - ctx->stage), n);
}

int eff_buf_read(eff_ctx *ctx, eff_buf *buf, size_t off, void *dst, size_t n) {
  if (!ctx || !buf || (!dst && n)) return EFF_E_INVALID;
  if (off > buf->size || n > buf->size - off) return fail(ctx, EFF_E_BOUNDS, "read of %zu bytes at %zu past a %zu-byte buffer", n, off, buf->size);
  int rc = use_device(ctx);
  if (rc || (rc = refuse_capture(ctx, "read"))) return rc;
  if (n) EFF_HIP(ctx, hipMemcpyAsync(dst, (const char *)buf->ptr + off, n, hipMemcpyDeviceToHost, ctx->stream));
  EFF_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return EFF_OK;
}

int eff_read_begin(eff_ctx *ctx, eff_buf *buf, size_t off, size_t n, eff_read **out) {
  if (!ctx || !buf || !out) return EFF_E_INVALID;
  *out = nullptr;
  if (off > buf->size || n > buf->size - off) return fail(ctx, EFF_E_BOUNDS, "read of %zu bytes at %zu past a %zu-byte buffer", n, off, buf->size);
  int rc = use_device(ctx);
  if (rc || (rc = refuse_capture(ctx, "readback"))) return rc;
  eff_read *r = new eff_read();
  r->device = ctx->device;
  r->pool = ctx->reads;
  r->n = n;
  {
    std::lock_guard<std::mutex> lk(r->pool->mu);
    auto &blocks = r->pool->blocks;
    for (size_t i = 0; i < blocks.size(); ++i) {
      if (blocks[i].second >= n) {
        r->host = blocks[i].first;
        r->cap = blocks[i].second;
        blocks.erase(blocks.begin() + i);
        break;
      }
    }
    if (!r->pool->events.empty()) {
      r->ev = r->pool->events.back();
      r->pool->events.pop_back();
    }
  }
  if (!r->host) {
    r->cap = n < 65536 ? 65536 : n;
    if (hipHostMalloc(&r->host, r->cap, hipHostMallocDefault) != hipSuccess) {
      delete r;
      return fail(ctx, EFF_E_NOMEM, "pinned read block of %zu bytes", n);
    }
  }
  hipError_t e = r->ev ? hipSuccess : hipEventCreateWithFlags(&r->ev, hipEventDisableTiming);
  if (e == hipSuccess && n) e = hipMemcpyAsync(r->host, (const char *)buf->ptr + off, n, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipEventRecord(r->ev, ctx->stream);
  if (e != hipSuccess) {
    eff_read_release(r);
    return hip_fail(ctx, e, "read begin");
  }
  *out = r;
  return EFF_OK;
}

int eff_read_end(eff_read *r, void *dst) {
  if (!r || (!dst && r->n)) return EFF_E_INVALID;
  hipError_t e = hipSetDevice(r->device);
  // A readback in a decode loop usually ends within microseconds of the call:
  // the copy is polled for up to kReadSpinNs before the blocking wait, whose
  // wake-up would otherwise add to every token.
  if (e == hipSuccess) {
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
      e = hipEventQuery(r->ev);
      if (e != hipErrorNotReady) break;
      if (std::chrono::steady_clock::now() - t0 > std::chrono::nanoseconds(kReadSpinNs)) {
        e = hipEventSynchronize(r->ev);
        break;
      }
    }
  }
  if (e != hipSuccess) {
    r->rc = EFF_E_DEVICE;
    r->error = std::string("read: ") + hipGetErrorString(e);
    return r->rc;
  }
  if (r->n) memcpy(dst, r->host, r->n);
  return EFF_OK;
}

int eff_read_poll(eff_read *r) {
  if (!r) return EFF_E_INVALID;
  hipError_t e = hipSetDevice(r->device);
  if (e == hipSuccess) e = hipEventQuery(r->ev);
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  r->rc = EFF_E_DEVICE;
  r->error = std::string("read: ") + hipGetErrorString(e);
  return r->rc;
}

const char *eff_read_error(const eff_read *r) { return r ? r->error.c_str() : "no read"; }

int eff_read_release(eff_read *r) {
  if (!r) return EFF_E_INVALID;
  (void)hipSetDevice(r->device);
  const bool done = !r->ev || hipEventSynchronize(r->ev) == hipSuccess;
  {
    std::lock_guard<std::mutex> lk(r->pool->mu);
    if (r->host) r->pool->blocks.push_back({r->host, r->cap});
    if (r->ev && done) r->pool->events.push_back(r->ev);   // completed: recorded again by a later read
  }
  if (r->ev && !done) (void)hipEventDestroy(r->ev);
  delete r;   // the pool goes with its last owner (context or ticket)
  return EFF_OK;
}

int eff_buf_copy(eff_ctx *ctx, eff_buf *dst, size_t doff, eff_buf *src, size_t soff, size_t n) {
  if (!ctx || !dst || !src) return EFF_E_INVALID;
  if (doff > dst->size || n > dst->size - doff || soff > src->size || n > src->size - soff)
    return fail(ctx, EFF_E_BOUNDS, "copy of %zu bytes out of bounds", n);
  if (!n) return EFF_OK;
  int rc = use_device(ctx);
  if (rc) return rc;
  EFF_HIP(ctx, hipMemcpyAsync((char *)dst->ptr + doff, (const char *)src->ptr + soff, n, hipMemcpyDeviceToDevice, ctx->stream));
  return EFF_OK;
}

int eff_buf_mark_r(eff_buf *buf, int type_r, uint32_t n) {
  if (!buf) return EFF_E_INVALID;
  if (type_r != EFF_TYPE_Q8_0R) return EFF_E_TYPE;
  if (n == 0) return EFF_E_INVALID;
  if (buf->size != eff_bytes_buffer_r(type_r, n)) return EFF_E_MARK;
  buf->mark_type = type_r;
  buf->mark_blocks = n;
  return EFF_OK;
}

int eff_buf_write_r(eff_ctx *ctx, eff_buf *buf, int type_r, uint32_t first_block, const void *src,
                    uint32_t n_blocks) {
  if (!ctx || !buf || (!src && n_blocks)) return EFF_E_INVALID;
  if (type_r != EFF_TYPE_Q8_0R) return fail(ctx, EFF_E_TYPE, "write R: %d is not a repacked type", type_r);
  if (buf->mark_type != EFF_TYPE_Q8_0R)
    return fail(ctx, EFF_E_MARK, "write R: the buffer does not carry the mark of a repacked tensor");
  const uint32_t N = buf->mark_blocks;
  if (first_block > N || n_blocks > N - first_block)
    return fail(ctx, EFF_E_BOUNDS, "write R: blocks %u..%u past a tensor of %u", first_block,
                first_block + n_blocks, N);
  if (!n_blocks) return EFF_OK;
  std::string tmp(eff_bytes_reordered(type_r, n_blocks), '\0');  // 34 n rounded up to a word
  int rc = eff_repack(type_r, src, n_blocks, &tmp[0], tmp.size());
  if (rc) return fail(ctx, rc, "write R: repack failed");
  if ((rc = use_device(ctx)) || (rc = refuse_capture(ctx, "write R"))) return rc;
  char *base = (char *)buf->ptr;
  EFF_HIP(ctx, hipMemcpyAsync(base + (size_t)32 * first_block, tmp.data(), (size_t)32 * n_blocks,
                              hipMemcpyHostToDevice, ctx->stream));
  EFF_HIP(ctx, hipMemcpyAsync(base + (size_t)32 * N + (size_t)2 * first_block, tmp.data() + (size_t)32 * n_blocks,
                              (size_t)2 * n_blocks, hipMemcpyHostToDevice, ctx->stream));
  EFF_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return EFF_OK;
}

int eff_buf_blocks_r(const eff_buf *buf, uint32_t *n) {
  if (!buf || !n) return EFF_E_INVALID;
  if (buf->mark_type != EFF_TYPE_Q8_0R) return EFF_E_MARK;
  *n = buf->mark_blocks;
  return EFF_OK;
}

int eff_qgemv(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k, uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (tokens == 0 || (int64_t)tokens > ctx->gemv_max_tokens || tokens > 8) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  WeightView wv;
  int rc = weight_view(ctx, type, w, x, y, rows, k, tokens, wv, "gemv");
  if (rc) return rc;
  if ((rc = use_device(ctx))) return rc;
  rc = run_gemv(ctx, wv, (const float *)x->ptr, (float *)y->ptr, tokens);
  if (!rc) ++ctx->stats.gemv;
  return rc;
}

int eff_qgemv_multi(eff_ctx *ctx, int type, int mode, uint32_t n, eff_buf *const *ws, eff_buf *x,
                    eff_buf *const *ys, const uint32_t *rows, uint32_t k, uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (mode != EFF_GEMV_SECTIONS && mode != EFF_GEMV_SWIGLU)
    return fail(ctx, EFF_E_INVALID, "gemv multi: unknown mode %d", mode);
  if (!ws || !ys || !rows) return fail(ctx, EFF_E_INVALID, "gemv multi: null array");
  // the reference's gateUp takes two matrices and secciones two to four; 1..3 tokens
  if (n < 2 || n > 4 || (mode == EFF_GEMV_SWIGLU && n != 2) || tokens < 1 || tokens > 3 || ctx->gemv_kernel != 0) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  if (mode == EFF_GEMV_SWIGLU && rows[0] != rows[1])
    return fail(ctx, EFF_E_SHAPE, "gemv gate+up: gate has %u rows and up %u", rows[0], rows[1]);
  WeightView wvs[4];
  float *yp[4] = {nullptr, nullptr, nullptr, nullptr};
  for (uint32_t i = 0; i < n; ++i) {
    eff_buf *yb = mode == EFF_GEMV_SWIGLU ? ys[0] : ys[i];
    int rc = weight_view(ctx, type, ws[i], x, yb, rows[i], k, tokens, wvs[i], "gemv multi");
    if (rc) return rc;
    yp[i] = (float *)yb->ptr;
  }
  int rc = use_device(ctx);
  if (rc) return rc;
  // a matrix whose one-matrix GEMV runs the row kernel would not get that
  // GEMV's bits from a fused launch: not applicable, the caller runs them apart
  bool rows_kernel = false;
  for (uint32_t i = 0; i < n; ++i) rows_kernel = rows_kernel || gemv_rows_applies(wvs[i], tokens);
  if (rows_kernel || !gemv_mx_multi_applies(wvs[0], tokens, mode)) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  hipError_t e = launch_gemv_mx_multi(mode, n, wvs, (const float *)x->ptr, yp, tokens, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "gemv multi launch");
  ++ctx->stats.fused;
  return EFF_OK;
}

int eff_qgemm(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k, uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (tokens == 0 || (int64_t)tokens < ctx->gemm_min_tokens) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  WeightView wv;
  int rc = weight_view(ctx, type, w, x, y, rows, k, tokens, wv, "gemm");
  if (rc) return rc;
  if ((rc = use_device(ctx))) return rc;
  rc = run_gemm(ctx, wv, (const float *)x->ptr, (float *)y->ptr, tokens, tokens);
  if (!rc) ++ctx->stats.gemm;
  return rc;
}

int eff_qgemm_planned(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k,
                      uint32_t tokens, uint32_t plan_tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (plan_tokens == 0 || (int64_t)plan_tokens < ctx->gemm_min_tokens) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  if (tokens > plan_tokens)
    return fail(ctx, EFF_E_INVALID, "gemm planned: %u tokens under the plan of %u", tokens, plan_tokens);
  WeightView wv;
  int rc = weight_view(ctx, type, w, x, y, rows, k, tokens, wv, "gemm planned");
  if (rc) return rc;
  if ((rc = use_device(ctx))) return rc;
  rc = run_gemm(ctx, wv, (const float *)x->ptr, (float *)y->ptr, tokens, plan_tokens);
  if (!rc) ++ctx->stats.gemm;
  return rc;
}

int eff_gemm_x_layout(eff_ctx *ctx, int type, uint32_t rows, uint32_t k, uint32_t tokens, uint32_t plan_tokens,
                      size_t *bytes, uint32_t *layout) {
  if (!ctx || !bytes || !layout) return EFF_E_INVALID;
  const int rc = gemm_prepared_check(ctx, type, rows, k, tokens, plan_tokens, "gemm x layout");
  if (rc) return rc;
  const uint32_t cfg = (uint32_t)ctx->gemm_config;
  *bytes = gemm_x_bytes(type, tokens, plan_tokens, k, rows, cfg);
  *layout = gemm_x_layout(type, plan_tokens, k, rows, cfg);
  return EFF_OK;
}

int eff_gemm_prepare_x(eff_ctx *ctx, int type, eff_buf *x, eff_buf *xh, uint32_t rows, uint32_t k, uint32_t tokens,
                       uint32_t plan_tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (!x || !xh) return fail(ctx, EFF_E_INVALID, "gemm prepare x: null buffer");
  int rc = gemm_prepared_check(ctx, type, rows, k, tokens, plan_tokens, "gemm prepare x");
  if (rc) return rc;
  const uint32_t cfg = (uint32_t)ctx->gemm_config;
  if ((uint64_t)tokens * k * 4 > x->size)
    return fail(ctx, EFF_E_BOUNDS, "gemm prepare x: x needs %llu bytes and the buffer has %zu",
                (unsigned long long)tokens * k * 4, x->size);
  if ((rc = check_out(ctx, xh, gemm_x_bytes(type, tokens, plan_tokens, k, rows, cfg), "gemm prepare x")) ||
      (rc = use_device(ctx)))
    return rc;
  if ((uintptr_t)x->ptr & 15) return fail(ctx, EFF_E_INVALID, "gemm prepare x: device buffers must be 16-byte aligned");
  const hipError_t e = launch_gemm_x(type, (const float *)x->ptr, tokens, plan_tokens, k, rows, cfg, xh->ptr,
                                     ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "gemm prepare x launch");
  ++ctx->stats.gemm_x;
  return EFF_OK;
}

int eff_qgemm_prepared(eff_ctx *ctx, int type, eff_buf *w, eff_buf *xh, eff_buf *y, uint32_t rows, uint32_t k,
                       uint32_t tokens, uint32_t plan_tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (!w || !xh || !y) return fail(ctx, EFF_E_INVALID, "gemm prepared: null buffer");
  int rc = gemm_prepared_check(ctx, type, rows, k, tokens, plan_tokens, "gemm prepared");
  if (rc) return rc;
  const uint32_t cfg = (uint32_t)ctx->gemm_config;
  // the weight view checks against a stand-in x of the call's size (the
  // product reads xh, checked below)
  eff_buf xs{};
  xs.ptr = xh->ptr;
  xs.size = (size_t)tokens * k * 4;
  WeightView wv;
  if ((rc = weight_view(ctx, type, w, &xs, y, rows, k, tokens, wv, "gemm prepared")) ||
      (rc = check_out(ctx, xh, gemm_x_bytes(type, tokens, plan_tokens, k, rows, cfg), "gemm prepared x")) ||
      (rc = use_device(ctx)))
    return rc;
  void *sk;
  if ((rc = sk_scratch(ctx, wv, tokens, plan_tokens, &sk))) return rc;
  const hipError_t e = launch_gemm_prepared(wv, (const _Float16 *)xh->ptr, (float *)y->ptr, tokens, plan_tokens, cfg,
                                            (uint32_t)ctx->gemm_split, sk, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "gemm prepared launch");
  ++ctx->stats.gemm;
  return EFF_OK;
}

int eff_qmatmul(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k, uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  WeightView wv;
  int rc = weight_view(ctx, type, w, x, y, rows, k, tokens, wv, "matmul");
  if (rc) return rc;
  if ((rc = use_device(ctx))) return rc;
  const float *xp = (const float *)x->ptr;
  float *yp = (float *)y->ptr;
  if ((int64_t)tokens <= ctx->gemv_max_tokens && tokens <= 8) {
    rc = run_gemv(ctx, wv, xp, yp, tokens);
    if (!rc) ++ctx->stats.gemv;
    return rc;
  }
  // Q2_K, Q4_K, IQ2_XXS, Q6_K: the reference has no f16 GEMM for these types
  // (DRIFT and GEMM2 read Q8_0/Q4_0 only) and runs its f32 kernel at every
  // token count (ops.js:117-128); so does this router, on the split-x matrix
  // cores, and for Q8_0 below the GEMM's threshold.
  if (sx_routes(ctx, wv, tokens)) return run_sx(ctx, wv, xp, yp, tokens);
  // The fp16 GEMM is the reference's DRIFT/GEMM2 semantics, which exist for
  // Q8_0 (and Q4_0) only (kernels.drift.wgsl.js:33, kernels.gemm2.wgsl.js:51).
  if ((int64_t)tokens >= ctx->gemm_min_tokens && router_gemm_type(type)) {
    rc = run_gemm(ctx, wv, xp, yp, tokens, tokens);
    if (!rc) ++ctx->stats.gemm;
    return rc;
  }
  // Between the two: the GEMV over groups of tokens (16 per launch for the
  // multi-token matrix-core kernel, else 8). Y is token-major, so each group
  // writes a contiguous slice.
  GemvPlan p16;
  const uint32_t grp = ctx->gemv_kernel == 0 && gemv_mt_plan(wv, 16, p16) ? 16u : 8u;
  for (uint32_t t0 = 0; t0 < tokens; t0 += grp) {
    const uint32_t tn = tokens - t0 < grp ? tokens - t0 : grp;
    rc = run_gemv(ctx, wv, xp + (uint64_t)t0 * k, yp + (uint64_t)t0 * rows, tn);
    if (rc) return rc;
    ++ctx->stats.skinny;
  }
  return EFF_OK;
}

int eff_qmatmul_x_layout(eff_ctx *ctx, int type, uint32_t rows, uint32_t k, uint32_t tokens, size_t *bytes,
                         uint32_t *layout) {
  if (!ctx || !bytes || !layout) return EFF_E_INVALID;
  WeightView wv;
  const int rc = matmul_prepared_view(ctx, type, rows, k, tokens, wv, "matmul x layout");
  if (rc) return rc;
  size_t n = 0;
  const uint32_t l = route_layout(ctx, wv, tokens, &n);
  if (!l) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  *bytes = n;
  *layout = l;
  return EFF_OK;
}

int eff_qmatmul_prepare_x(eff_ctx *ctx, int type, eff_buf *x, eff_buf *xp, uint32_t rows, uint32_t k,
                          uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (!x || !xp) return fail(ctx, EFF_E_INVALID, "matmul prepare x: null buffer");
  WeightView wv;
  int rc = matmul_prepared_view(ctx, type, rows, k, tokens, wv, "matmul prepare x");
  if (rc) return rc;
  size_t n = 0;
  const uint32_t l = route_layout(ctx, wv, tokens, &n);
  if (!l) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  if ((uint64_t)tokens * k * 4 > x->size)
    return fail(ctx, EFF_E_BOUNDS, "matmul prepare x: x needs %llu bytes and the buffer has %zu",
                (unsigned long long)tokens * k * 4, x->size);
  if ((uintptr_t)x->ptr & 15) return fail(ctx, EFF_E_INVALID, "matmul prepare x: device buffers must be 16-byte aligned");
  if ((rc = check_out(ctx, xp, n, "matmul prepare x")) || (rc = use_device(ctx))) return rc;
  hipError_t e;
  if (l & kSxLayout) {
    e = launch_sx_prepare(l, (const float *)x->ptr, tokens, k, xp->ptr, ctx->stream);
    ++ctx->stats.split_x;
  } else {
    e = launch_gemm_x(type, (const float *)x->ptr, tokens, tokens, k, rows, (uint32_t)ctx->gemm_config, xp->ptr,
                      ctx->stream);
    ++ctx->stats.gemm_x;
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "matmul prepare x launch");
  return EFF_OK;
}

int eff_qmatmul_prepared(eff_ctx *ctx, int type, eff_buf *w, eff_buf *xp, eff_buf *y, uint32_t rows, uint32_t k,
                         uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (!w || !xp || !y) return fail(ctx, EFF_E_INVALID, "matmul prepared: null buffer");
  WeightView wv;
  int rc = matmul_prepared_view(ctx, type, rows, k, tokens, wv, "matmul prepared");
  if (rc) return rc;
  size_t n = 0;
  const uint32_t l = route_layout(ctx, wv, tokens, &n);
  if (!l) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  // the weight view checks against a stand-in x of the call's size (the
  // product reads xp, checked below)
  eff_buf xs{};
  xs.ptr = xp->ptr;
  xs.size = (size_t)tokens * k * 4;
  if ((rc = weight_view(ctx, type, w, &xs, y, rows, k, tokens, wv, "matmul prepared")) ||
      (rc = check_out(ctx, xp, n, "matmul prepared x")) || (rc = use_device(ctx)))
    return rc;
  hipError_t e;
  if (l & kSxLayout) {
    void *sk;
    if ((rc = sk_get(ctx, sx_sk_bytes(wv, tokens, (int)ctx->sx_config, (uint32_t)ctx->sx_split), &sk))) return rc;
    e = launch_sx_prepared(wv, xp->ptr, (float *)y->ptr, tokens, (int)ctx->sx_config, (uint32_t)ctx->sx_split, sk,
                           ctx->stream);
    ++ctx->stats.split;
  } else {
    void *sk;
    if ((rc = sk_scratch(ctx, wv, tokens, tokens, &sk))) return rc;
    e = launch_gemm_prepared(wv, (const _Float16 *)xp->ptr, (float *)y->ptr, tokens, tokens,
                             (uint32_t)ctx->gemm_config, (uint32_t)ctx->gemm_split, sk, ctx->stream);
    ++ctx->stats.gemm;
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "matmul prepared launch");
  return EFF_OK;
}

int eff_qmatmul_cpu_path(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k,
                         uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  WeightView wv;
  int rc = weight_view(ctx, type, w, x, y, rows, k, tokens, wv, "cpu path");
  if (rc) return rc;
  if (type != EFF_TYPE_Q8_0) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  if ((uint64_t)tokens * (k / 32u) >= (1ull << 31))
    return fail(ctx, EFF_E_INVALID, "cpu path: %u tokens of %u values are too many blocks", tokens, k);
  if ((rc = use_device(ctx)) ||
      (rc = grow(ctx, &ctx->act_scratch, &ctx->act_scratch_bytes, cpu_path_act_bytes(tokens, k), "cpu path x")))
    return rc;
  const hipError_t e = launch_cpu_path(wv, (const float *)x->ptr, (float *)y->ptr, tokens, ctx->act_scratch,
                                       ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "cpu path launch");
  ++ctx->stats.cpu_path;
  return EFF_OK;
}

int eff_read_floor(eff_ctx *ctx, eff_buf *src, size_t bytes, uint32_t workgroups, uint32_t unroll, eff_buf *sink) {
  if (!ctx) return EFF_E_INVALID;
  if (!src || !sink) return fail(ctx, EFF_E_INVALID, "read floor: null buffer");
  if (bytes == 0 || workgroups == 0 || workgroups > 65535u || (unroll != 1u && unroll != 2u && unroll != 4u))
    return fail(ctx, EFF_E_INVALID, "read floor: %zu bytes, %u workgroups, unroll %u (bytes > 0, 1..65535 workgroups, "
                "unroll 1, 2 or 4)", bytes, workgroups, unroll);
  if (bytes > src->size) return fail(ctx, EFF_E_BOUNDS, "read floor: %zu bytes from a buffer of %zu", bytes, src->size);
  if ((uint64_t)workgroups * 4u > sink->size)
    return fail(ctx, EFF_E_BOUNDS, "read floor: the sink needs %llu bytes and has %zu",
                (unsigned long long)workgroups * 4u, sink->size);
  int rc = use_device(ctx);
  if (rc) return rc;
  const hipError_t e = launch_read_floor((const uint8_t *)src->ptr, bytes, workgroups, unroll, (uint32_t *)sink->ptr,
                                         ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "read floor launch");
  return EFF_OK;
}

int eff_dequant(eff_ctx *ctx, int type, eff_buf *w, eff_buf *out, uint32_t n_blocks) {
  if (!ctx) return EFF_E_INVALID;
  if (!w || !out) return fail(ctx, EFF_E_INVALID, "dequant: null buffer");
  if (!type_known(type)) return fail(ctx, EFF_E_TYPE, "dequant: unsupported quantization type %d", type);
  if (n_blocks == 0) return EFF_OK;
  Geometry g = geometry(type);
  uint64_t scales_off = 0;
  if (type == EFF_TYPE_Q8_0R) {
    if (w->mark_type != EFF_TYPE_Q8_0R) return fail(ctx, EFF_E_MARK, "dequant Q8_0R: buffer without the repack mark");
    if (n_blocks > w->mark_blocks) return fail(ctx, EFF_E_MARK, "dequant Q8_0R: %u blocks requested, tensor has %u", n_blocks, w->mark_blocks);
    scales_off = (uint64_t)32 * w->mark_blocks;
  } else if ((uint64_t)n_blocks * g.bytes > w->size) {
    return fail(ctx, EFF_E_BOUNDS, "dequant: %u blocks need %llu bytes, buffer has %zu", n_blocks,
                (unsigned long long)n_blocks * g.bytes, w->size);
  }
  if ((uint64_t)n_blocks * g.elems * 4 > out->size) return fail(ctx, EFF_E_BOUNDS, "dequant: output buffer too small");
  int rc = use_device(ctx);
  if (rc) return rc;
  WeightView wv{};
  wv.w = (const uint8_t *)w->ptr;
  wv.type = type;
  wv.scales_off = scales_off;
  wv.w_bytes = w->size + (w->owned ? kSlack : 16);  // wrapped buffers guarantee 16 readable bytes
  hipError_t e = launch_dequant(wv, n_blocks, (float *)out->ptr, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "dequant launch");
  ++ctx->stats.dequant;
  return EFF_OK;
}

}  // extern "C"

namespace {

// Shared checks of the gather entry points (quant.gather, ops.js:1104-1110).
int gather_view(eff_ctx *ctx, int type, eff_buf *w, eff_buf *ids, uint32_t dim, uint32_t tokens, WeightView &wv,
                const char *who) {
  if (!w || !ids) return fail(ctx, EFF_E_INVALID, "%s: null buffer", who);
  if (!type_known(type)) return fail(ctx, EFF_E_TYPE, "%s: unsupported quantization type %d", who, type);
  const Geometry g = geometry(type);
  if (dim == 0 || dim % g.elems)
    return fail(ctx, EFF_E_SHAPE, "%s %s: dim=%u is not a multiple of %u", who, eff_type_name(type), dim, g.elems);
  if ((uint64_t)tokens * 4 > ids->size)
    return fail(ctx, EFF_E_BOUNDS, "%s: %u ids need %llu bytes and the buffer has %zu", who, tokens,
                (unsigned long long)tokens * 4, ids->size);
  wv = WeightView{};
  wv.w = (const uint8_t *)w->ptr;
  wv.type = type;
  wv.k = dim;
  wv.bpr = dim / g.elems;
  wv.row_bytes = (uint64_t)wv.bpr * g.bytes;
  wv.w_bytes = w->size + (w->owned ? kSlack : 16);
  if (type == EFF_TYPE_Q8_0R) {
    if (w->mark_type != EFF_TYPE_Q8_0R)
      return fail(ctx, EFF_E_MARK, "%s Q8_0R: the buffer does not carry the mark of a repacked tensor", who);
    if (w->mark_blocks < wv.bpr)
      return fail(ctx, EFF_E_MARK, "%s Q8_0R: a row of %u blocks and a tensor of %u", who, wv.bpr, w->mark_blocks);
    wv.scales_off = (uint64_t)32 * w->mark_blocks;
  } else if (wv.row_bytes > w->size) {
    return fail(ctx, EFF_E_BOUNDS, "%s %s: a row needs %llu bytes and the table has %zu", who, eff_type_name(type),
                (unsigned long long)wv.row_bytes, w->size);
  }
  return EFF_OK;
}

// The checks of the top-k entry points (createTopKGPU().candidatos,
// ops.topk.js:99-165): outside the limits the reference falls back to a full
// readback (ops.topk.js:104-105, topk.js:114-117), i.e. NOT_APPLICABLE here.
int topk_check(eff_ctx *ctx, eff_buf *logits, uint32_t base, uint32_t vocab, uint32_t m, const uint32_t *penal_ids,
               uint32_t n_penal, eff_buf *out, const char *who) {
  if (!logits || !out) return fail(ctx, EFF_E_INVALID, "%s: null buffer", who);
  if (n_penal && !penal_ids) return fail(ctx, EFF_E_INVALID, "%s: null penalised ids", who);
  if (vocab == 0 || vocab >= EFF_TOPK_N_MAX || m == 0 || m > EFF_TOPK_M_MAX || n_penal > EFF_TOPK_P_MAX) {
    ++ctx->stats.not_applicable;
    return EFF_NOT_APPLICABLE;
  }
  if (((uint64_t)base + vocab) * 4 > logits->size) return fail(ctx, EFF_E_BOUNDS, "%s: logits buffer too small", who);
  if (out->size < eff_topk_out_bytes())
    return fail(ctx, EFF_E_BOUNDS, "%s: output buffer needs %zu bytes", who, eff_topk_out_bytes());
  return EFF_OK;
}


}  // namespace

extern "C" {

int eff_gather(eff_ctx *ctx, int type, eff_buf *w, eff_buf *ids, eff_buf *out, uint32_t dim, uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  WeightView wv;
  int rc = gather_view(ctx, type, w, ids, dim, tokens, wv, "gather");
  if (rc || (rc = check_out(ctx, out, (uint64_t)tokens * dim * 4, "gather"))) return rc;
  if (tokens == 0) return EFF_OK;
  if ((rc = use_device(ctx))) return rc;
  hipError_t e = launch_gather(wv, (const uint32_t *)ids->ptr, tokens, (float *)out->ptr, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "gather launch");
  ++ctx->stats.gather;
  return EFF_OK;
}

int eff_gather_norm(eff_ctx *ctx, int type, eff_buf *w, eff_buf *ids, eff_buf *wn, float eps, eff_buf *x,
                    eff_buf *nrm, uint32_t dim, uint32_t tokens) {
  if (!ctx) return EFF_E_INVALID;
  if (type == EFF_TYPE_IQ2_XXS)
    return fail(ctx, EFF_E_TYPE, "gather+norm: IQ2_XXS has no block reader here (its grid is not bound)");
  WeightView wv;
  int rc = gather_view(ctx, type, w, ids, dim, tokens, wv, "gather+norm");
  if (rc) return rc;
  if (dim > kGatherNormMaxDim) return fail(ctx, EFF_E_SHAPE, "gather+norm: dim=%u above %u", dim, kGatherNormMaxDim);
  if ((rc = check_out(ctx, x, (uint64_t)tokens * dim * 4, "gather+norm x")) ||
      (rc = check_out(ctx, nrm, (uint64_t)tokens * dim * 4, "gather+norm nrm")) ||
      (rc = check_out(ctx, wn, (uint64_t)dim * 4, "gather+norm weights")))
    return rc;
  if (tokens == 0) return EFF_OK;
  if ((rc = use_device(ctx))) return rc;
  hipError_t e = launch_gather_norm(wv, (const uint32_t *)ids->ptr, tokens, (const float *)wn->ptr, eps,
                                    (float *)x->ptr, (float *)nrm->ptr, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "gather+norm launch");
  ++ctx->stats.gather;
  return EFF_OK;
}

size_t eff_topk_out_bytes(void) { return sizeof(uint32_t) * (EFF_TOPK_HEADER + EFF_TOPK_P_MAX + 2 * EFF_TOPK_CAP); }

int eff_topk(eff_ctx *ctx, eff_buf *logits, uint32_t base, uint32_t vocab, uint32_t m, const uint32_t *penal_ids,
             uint32_t n_penal, uint32_t serial, eff_buf *out) {
  if (!ctx) return EFF_E_INVALID;
  int rc = topk_check(ctx, logits, base, vocab, m, penal_ids, n_penal, out, "topk");
  if (rc) return rc;
  if ((rc = use_device(ctx))) return rc;
  if ((rc = grow(ctx, &ctx->topk_scratch, &ctx->topk_scratch_bytes, topk_scratch_bytes(vocab), "topk"))) return rc;
  hipError_t e = launch_topk((const uint32_t *)logits->ptr, base, vocab, m, penal_ids, n_penal, serial,
                             (uint32_t *)ctx->topk_scratch, (uint32_t *)out->ptr, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "topk launch");
  ++ctx->stats.topk;
  return EFF_OK;
}

int eff_qgemv_topk(eff_ctx *ctx, int type, eff_buf *w, eff_buf *x, eff_buf *y, uint32_t rows, uint32_t k, uint32_t m,
                   const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, eff_buf *out) {
  if (!ctx) return EFF_E_INVALID;
  // the top-k's limits first, so that a NOT_APPLICABLE call enqueues nothing
  int rc = topk_check(ctx, y, 0, rows, m, penal_ids, n_penal, out, "gemv+topk");
  if (rc) return rc;
  WeightView wv;
  if ((rc = weight_view(ctx, type, w, x, y, rows, k, 1, wv, "gemv+topk"))) return rc;
  if ((rc = use_device(ctx))) return rc;
  const float *xp = (const float *)x->ptr;
  float *yp = (float *)y->ptr;
  if (ctx->gemv_kernel == 0 && gemv_rows_applies(wv, 1) && gemv_rows_groups(wv) <= kRowsTopkGroupsMax) {
    // the GEMV writes the top-k's group records; one launch selects from them
    const uint32_t groups = gemv_rows_groups(wv);
    if ((rc = grow(ctx, &ctx->topk_scratch, &ctx->topk_scratch_bytes, (size_t)groups * kTopkGroupBytes, "topk")))
      return rc;
    hipError_t e = launch_gemv_rows_topk(wv, xp, yp, (uint8_t *)ctx->topk_scratch, m, penal_ids, n_penal, serial,
                                         (uint32_t *)out->ptr, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "gemv+topk launch");
  } else {
    if ((rc = run_gemv(ctx, wv, xp, yp, 1))) return rc;
    if ((rc = grow(ctx, &ctx->topk_scratch, &ctx->topk_scratch_bytes, topk_scratch_bytes(rows), "topk"))) return rc;
    hipError_t e = launch_topk((const uint32_t *)yp, 0, rows, m, penal_ids, n_penal, serial,
                               (uint32_t *)ctx->topk_scratch, (uint32_t *)out->ptr, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "topk launch");
  }
  ++ctx->stats.gemv;
  ++ctx->stats.topk;
  return EFF_OK;
}

int eff_graph_begin(eff_ctx *ctx) {
  if (!ctx) return EFF_E_INVALID;
  int rc = use_device(ctx);
  if (rc || (rc = refuse_capture(ctx, "graph begin"))) return rc;
  // thread-local: only calls from this thread that could not be recorded
  // (waits, allocations) are refused while recording
  EFF_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  return EFF_OK;
}

int eff_graph_end(eff_ctx *ctx, eff_graph **out) {
  if (!ctx || !out) return EFF_E_INVALID;
  *out = nullptr;
  int rc = use_device(ctx);
  if (rc) return rc;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  EFF_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cs));
  if (cs == hipStreamCaptureStatusNone) return fail(ctx, EFF_E_INVALID, "graph end: no recording is open");
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &g);
  if (e != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return hip_fail(ctx, e, "graph end (a call made during the recording invalidated it)");
  }
  eff_graph *gr = new eff_graph();
  gr->device = ctx->device;
  gr->graph = g;
  e = hipGraphGetNodes(g, nullptr, &gr->nodes);
  if (e == hipSuccess) e = hipGraphInstantiate(&gr->exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    eff_graph_destroy(gr);
    return hip_fail(ctx, e, "graph instantiate");
  }
  *out = gr;
  return EFF_OK;
}

int eff_graph_launch(eff_ctx *ctx, eff_graph *g) {
  if (!ctx || !g) return EFF_E_INVALID;
  if (g->device != ctx->device)
    return fail(ctx, EFF_E_INVALID, "graph launch: recorded on device %d, the context is on %d", g->device, ctx->device);
  int rc = use_device(ctx);
  if (rc) return rc;
  EFF_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
  return EFF_OK;
}

size_t eff_graph_nodes(const eff_graph *g) { return g ? g->nodes : 0; }

int eff_graph_destroy(eff_graph *g) {
  if (!g) return EFF_E_INVALID;
  (void)hipSetDevice(g->device);
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
  return EFF_OK;
}

int eff_topk_noalloc(eff_ctx *ctx, eff_buf *logits, uint32_t base, uint32_t vocab, uint32_t m,
                     const uint32_t *penal_ids, uint32_t n_penal, uint32_t serial, eff_buf *out) {
  if (!ctx) return EFF_E_INVALID;
  int rc = topk_check(ctx, logits, base, vocab, m, penal_ids, n_penal, out, "topk noalloc");
  if (rc) return rc;
  if (topk_scratch_bytes(vocab) > kNoAllocBytes)
    return fail(ctx, EFF_E_BOUNDS, "topk noalloc: a vocabulary of %u logits needs %zu scratch bytes and the fixed "
                "scratch holds %zu", vocab, topk_scratch_bytes(vocab), kNoAllocBytes);
  if (ctx->device >= kMaxDevices || !g_scratch_done[ctx->device])
    return fail(ctx, EFF_E_DEVICE, "topk noalloc: the fixed scratch of device %d was not looked up", ctx->device);
  if (!g_scratch_ptr[ctx->device])
    return hip_fail(ctx, g_scratch_err[ctx->device], "topk noalloc: hipGetSymbolAddress of the fixed scratch");
  if ((rc = use_device(ctx))) return rc;
  hipError_t e = launch_topk((const uint32_t *)logits->ptr, base, vocab, m, penal_ids, n_penal, serial,
                             (uint32_t *)g_scratch_ptr[ctx->device], (uint32_t *)out->ptr, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "topk noalloc launch");
  ++ctx->stats.topk;
  return EFF_OK;
}

}  // extern "C"
