// N-API addon over the C ABI (include/elffuss_amd.h): the native half of the
// JavaScript host. Device contexts and buffers travel as napi externals.
// Conventions kept from the reference's JS operators: a negative status
// throws an Error carrying the library's message and `code`;
// EFF_NOT_APPLICABLE returns null (the caller falls back, ops.gemv.js:13-21).
#include <node_api.h>
#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

#include "elffuss_amd.h"

namespace {

#define NAPI_OK(call)                                   \
  do {                                                  \
    if ((call) != napi_ok) return throw_msg(env, "napi call failed: " #call); \
  } while (0)

napi_value throw_msg(napi_env env, const std::string &msg, int code = EFF_E_INVALID) {
  napi_value err, m, c;
  napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
  napi_create_error(env, nullptr, m, &err);
  napi_create_int32(env, code, &c);
  napi_set_named_property(env, err, "code", c);
  napi_throw(env, err);
  return nullptr;
}

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value null_value(napi_env env) {
  napi_value u;
  napi_get_null(env, &u);
  return u;
}

napi_value make_int(napi_env env, int64_t v) {
  napi_value r;
  napi_create_int64(env, v, &r);
  return r;
}

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  for (size_t i = argc; i < want; ++i) argv[i] = undefined(env);
  return true;
}

template <class T>
T *external(napi_env env, napi_value v) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok) return nullptr;
  return (T *)p;
}

int64_t i64(napi_env env, napi_value v, int64_t dflt = 0) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_number) return dflt;
  int64_t r = dflt;
  napi_get_value_int64(env, v, &r);
  return r;
}

double f64(napi_env env, napi_value v, double dflt = 0) {
  double r = dflt;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_number) napi_get_value_double(env, v, &r);
  return r;
}

// Bytes of an ArrayBuffer, typed array or DataView.
bool bytes_of(napi_env env, napi_value v, void **data, size_t *len) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  if (is) {
    napi_typedarray_type tt;
    size_t n, off;
    napi_value ab;
    void *p;
    if (napi_get_typedarray_info(env, v, &tt, &n, &p, &ab, &off) != napi_ok) return false;
    size_t el = 1;
    switch (tt) {
      case napi_int16_array: case napi_uint16_array: el = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
      case napi_float64_array: el = 8; break;
      default: el = 1;
    }
    *data = p;
    *len = n * el;
    return true;
  }
  napi_is_arraybuffer(env, v, &is);
  if (is) return napi_get_arraybuffer_info(env, v, data, len) == napi_ok;
  napi_is_dataview(env, v, &is);
  if (is) {
    napi_value ab;
    size_t off;
    return napi_get_dataview_info(env, v, len, data, &ab, &off) == napi_ok;
  }
  return false;
}

napi_value status(napi_env env, eff_ctx *ctx, int rc) {
  if (rc == EFF_OK) return make_int(env, 0);
  if (rc == EFF_NOT_APPLICABLE) return null_value(env);
  return throw_msg(env, ctx ? eff_last_error(ctx) : "elffuss_amd error", rc);
}

// ---- types and host helpers ------------------------------------------------

napi_value TypeFromName(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  char buf[32] = {0};
  size_t n = 0;
  napi_get_value_string_utf8(env, a[0], buf, sizeof buf, &n);
  return make_int(env, eff_type_from_name(buf));
}

napi_value Geometry(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  uint32_t e = 0, b = 0;
  if (eff_type_geometry((int)i64(env, a[0]), &e, &b)) return null_value(env);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "blockElems", make_int(env, e));
  napi_set_named_property(env, o, "blockBytes", make_int(env, b));
  return o;
}

napi_value BufferMath(napi_env env, napi_callback_info info) {
  // (which, type, n): 0 bytesReordered, 1 bytesBufferR, 2 blocksFromBuffer, 3 scalesFrom
  napi_value a[3];
  get_args(env, info, 3, a);
  int which = (int)i64(env, a[0]), t = (int)i64(env, a[1]);
  int64_t n = i64(env, a[2]);
  switch (which) {
    case 0: return make_int(env, (int64_t)eff_bytes_reordered(t, (uint32_t)n));
    case 1: return make_int(env, (int64_t)eff_bytes_buffer_r(t, (uint32_t)n));
    case 2: return make_int(env, (int64_t)eff_blocks_from_buffer(t, (size_t)n));
    default: return make_int(env, (int64_t)eff_scales_from(t, (uint32_t)n));
  }
}

napi_value NewBytes(napi_env env, size_t n, void **data) {
  napi_value ab, arr;
  napi_create_arraybuffer(env, n, data, &ab);
  napi_create_typedarray(env, napi_uint8_array, n, ab, 0, &arr);
  return arr;
}

// repack(typeR, src, nBlocks, dstBytes) -> Uint8Array
napi_value Repack(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  void *src;
  size_t len;
  if (!bytes_of(env, a[1], &src, &len)) return throw_msg(env, "repack: source must be bytes");
  int t = (int)i64(env, a[0]);
  uint32_t n = (uint32_t)i64(env, a[2]);
  size_t dst_bytes = (size_t)i64(env, a[3], (int64_t)eff_bytes_buffer_r(t, n));
  if (len < (size_t)34 * n) return throw_msg(env, "repack: fewer source bytes than blocks", EFF_E_BOUNDS);
  void *dst;
  napi_value out = NewBytes(env, dst_bytes, &dst);
  int rc = eff_repack(t, src, n, dst, dst_bytes);
  if (rc) return throw_msg(env, "repack failed", rc);
  return out;
}

napi_value Unrepack(napi_env env, napi_callback_info info) {
  napi_value a[3];
  get_args(env, info, 3, a);
  void *src;
  size_t len;
  if (!bytes_of(env, a[1], &src, &len)) return throw_msg(env, "unrepack: source must be bytes");
  uint32_t n = (uint32_t)i64(env, a[2]);
  void *dst;
  napi_value out = NewBytes(env, (size_t)34 * n, &dst);
  int rc = eff_unrepack((int)i64(env, a[0]), src, len, n, dst);
  if (rc) return throw_msg(env, "unrepack failed", rc);
  return out;
}

napi_value Quantize(napi_env env, napi_callback_info info) {
  napi_value a[2];
  get_args(env, info, 2, a);
  void *src;
  size_t len;
  if (!bytes_of(env, a[1], &src, &len)) return throw_msg(env, "quantize: source must be a Float32Array");
  int t = (int)i64(env, a[0]);
  uint32_t e = 0, b = 0;
  if (eff_type_geometry(t, &e, &b)) return throw_msg(env, "quantize: unknown type", EFF_E_TYPE);
  size_t n = len / 4;
  void *dst;
  napi_value out = NewBytes(env, n / e * b, &dst);
  int rc = eff_quantize(t, (const float *)src, n, dst, n / e * b);
  if (rc) return throw_msg(env, "quantize failed", rc);
  return out;
}

napi_value FillNormal(napi_env env, napi_callback_info info) {
  napi_value a[3];
  get_args(env, info, 3, a);
  size_t n = (size_t)i64(env, a[2]);
  napi_value ab, arr;
  void *data;
  napi_create_arraybuffer(env, n * 4, &data, &ab);
  napi_create_typedarray(env, napi_float32_array, n, ab, 0, &arr);
  eff_fill_normal((uint32_t)i64(env, a[0]), (float)f64(env, a[1], 1.0), (float *)data, n);
  return arr;
}

// ---- context and buffers ----------------------------------------------------

napi_value Init(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  eff_ctx *ctx = nullptr;
  int rc = eff_init((int)i64(env, a[0]), &ctx);
  if (rc) return throw_msg(env, "eff_init: no usable HIP device", rc);
  napi_value ext;
  napi_create_external(env, ctx, nullptr, nullptr, &ext);
  return ext;
}

napi_value Shutdown(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  if (ctx) eff_shutdown(ctx);
  return undefined(env);
}

napi_value Sync(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  return status(env, ctx, eff_sync(ctx));
}

napi_value SetOption(napi_env env, napi_callback_info info) {
  napi_value a[3];
  get_args(env, info, 3, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  return status(env, ctx, eff_set_option(ctx, (int)i64(env, a[1]), i64(env, a[2])));
}

napi_value Stats(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  eff_stats s{};
  eff_get_stats(external<eff_ctx>(env, a[0]), &s);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "gemv", make_int(env, (int64_t)s.gemv));
  napi_set_named_property(env, o, "gemm", make_int(env, (int64_t)s.gemm));
  napi_set_named_property(env, o, "skinny", make_int(env, (int64_t)s.skinny));
  napi_set_named_property(env, o, "dequant", make_int(env, (int64_t)s.dequant));
  napi_set_named_property(env, o, "topk", make_int(env, (int64_t)s.topk));
  napi_set_named_property(env, o, "notApplicable", make_int(env, (int64_t)s.not_applicable));
  napi_set_named_property(env, o, "split", make_int(env, (int64_t)s.split));
  napi_set_named_property(env, o, "fused", make_int(env, (int64_t)s.fused));
  napi_set_named_property(env, o, "gather", make_int(env, (int64_t)s.gather));
  napi_set_named_property(env, o, "gemmX", make_int(env, (int64_t)s.gemm_x));
  napi_set_named_property(env, o, "splitX", make_int(env, (int64_t)s.split_x));
  napi_set_named_property(env, o, "cpuPath", make_int(env, (int64_t)s.cpu_path));
  return o;
}

napi_value BufAlloc(napi_env env, napi_callback_info info) {
  napi_value a[2];
  get_args(env, info, 2, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  eff_buf *b = nullptr;
  int rc = eff_buf_alloc(ctx, (size_t)i64(env, a[1]), &b);
  if (rc) return throw_msg(env, ctx ? eff_last_error(ctx) : "alloc", rc);
  napi_value ext;
  napi_create_external(env, b, nullptr, nullptr, &ext);
  return ext;
}

napi_value BufFree(napi_env env, napi_callback_info info) {
  napi_value a[2];
  get_args(env, info, 2, a);
  eff_buf_free(external<eff_ctx>(env, a[0]), external<eff_buf>(env, a[1]));
  return undefined(env);
}

// GPUBuffer.destroy(): given back in stream order, no wait (eff_buf_retire).
napi_value BufRetire(napi_env env, napi_callback_info info) {
  napi_value a[2];
  get_args(env, info, 2, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = eff_buf_retire(ctx, external<eff_buf>(env, a[1]));
  if (rc) return throw_msg(env, ctx ? eff_last_error(ctx) : "retire", rc);
  return undefined(env);
}

// Recorded launches (eff_graph_*): graphBegin(ctx); graphEnd(ctx) -> external;
// graphLaunch(ctx, g); graphNodes(g) -> number; graphDestroy(g).
napi_value GraphBegin(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  return status(env, ctx, eff_graph_begin(ctx));
}

napi_value GraphEnd(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  eff_graph *g = nullptr;
  int rc = eff_graph_end(ctx, &g);
  if (rc) return throw_msg(env, ctx ? eff_last_error(ctx) : "graph end", rc);
  napi_value ext;
  napi_create_external(env, g, nullptr, nullptr, &ext);
  return ext;
}

napi_value GraphLaunch(napi_env env, napi_callback_info info) {
  napi_value a[2];
  get_args(env, info, 2, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  return status(env, ctx, eff_graph_launch(ctx, external<eff_graph>(env, a[1])));
}

napi_value GraphNodes(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  return make_int(env, (int64_t)eff_graph_nodes(external<eff_graph>(env, a[0])));
}

napi_value GraphDestroy(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  eff_graph_destroy(external<eff_graph>(env, a[0]));
  return undefined(env);
}

napi_value BufWrite(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  void *src;
  size_t len;
  if (!bytes_of(env, a[3], &src, &len)) return throw_msg(env, "writeBuffer: data must be an ArrayBuffer or view");
  return status(env, ctx, eff_buf_write(ctx, external<eff_buf>(env, a[1]), (size_t)i64(env, a[2]), src, len));
}

napi_value BufRead(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  size_t n = (size_t)i64(env, a[3]);
  napi_value ab;
  void *dst;
  napi_create_arraybuffer(env, n, &dst, &ab);
  int rc = eff_buf_read(ctx, external<eff_buf>(env, a[1]), (size_t)i64(env, a[2]), dst, n);
  if (rc) return throw_msg(env, eff_last_error(ctx), rc);
  return ab;
}

// Asynchronous read (the readback of device.js:165-200): the device -> host
// copy is enqueued on the calling thread, so the snapshot holds exactly the
// work recorded before readback(); a libuv worker only waits for that copy;
// the Promise resolves with an ArrayBuffer. The ticket owns its pinned
// memory, and its error message is its own (the context's is not touched
// from the worker).
struct ReadWork {
  napi_async_work work;
  napi_deferred deferred;
  eff_read *ticket;
  size_t n;
  std::vector<uint8_t> data;
  int rc;
  std::string err;
};

void read_execute(napi_env, void *p) {
  ReadWork *w = (ReadWork *)p;
  w->data.resize(w->n);
  w->rc = eff_read_end(w->ticket, w->data.data());
  if (w->rc) w->err = eff_read_error(w->ticket);
}

void read_complete(napi_env env, napi_status, void *p) {
  ReadWork *w = (ReadWork *)p;
  eff_read_release(w->ticket);
  if (w->rc) {
    napi_value m, e, c;
    napi_create_string_utf8(env, w->err.c_str(), w->err.size(), &m);
    napi_create_error(env, nullptr, m, &e);
    napi_create_int32(env, w->rc, &c);
    napi_set_named_property(env, e, "code", c);
    napi_reject_deferred(env, w->deferred, e);
  } else {
    void *dst;
    napi_value ab;
    napi_create_arraybuffer(env, w->n, &dst, &ab);
    if (w->n) memcpy(dst, w->data.data(), w->n);
    napi_resolve_deferred(env, w->deferred, ab);
  }
  napi_delete_async_work(env, w->work);
  delete w;
}

napi_value BufReadAsync(napi_env env, napi_callback_info info) {
  napi_value a[4];
  get_args(env, info, 4, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  const size_t n = (size_t)i64(env, a[3]);
  eff_read *ticket = nullptr;
  int rc = eff_read_begin(ctx, external<eff_buf>(env, a[1]), (size_t)i64(env, a[2]), n, &ticket);
  if (rc) return throw_msg(env, ctx ? eff_last_error(ctx) : "readback", rc);
  ReadWork *w = new ReadWork();
  w->ticket = ticket;
  w->n = n;
  w->rc = 0;
  napi_value promise, name;
  napi_create_promise(env, &w->deferred, &promise);
  napi_create_string_utf8(env, "eff_read_end", NAPI_AUTO_LENGTH, &name);
  napi_create_async_work(env, nullptr, name, read_execute, read_complete, w, &w->work);
  napi_queue_async_work(env, w->work);
  return promise;
}

napi_value BufSize(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  return make_int(env, (int64_t)eff_buf_size(external<eff_buf>(env, a[0])));
}

napi_value BufMarkR(napi_env env, napi_callback_info info) {
  napi_value a[3];
  get_args(env, info, 3, a);
  return make_int(env, eff_buf_mark_r(external<eff_buf>(env, a[0]), (int)i64(env, a[1]), (uint32_t)i64(env, a[2])));
}

// bufWriteR(ctx, buf, typeR, firstBlock, ggufBytes): one chunk of the
// chunked Q8_0R upload (repack.js:318-345), repacked on the host.
napi_value BufWriteR(napi_env env, napi_callback_info info) {
  napi_value a[5];
  get_args(env, info, 5, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  void *src;
  size_t len;
  if (!bytes_of(env, a[4], &src, &len)) return throw_msg(env, "bufWriteR: data must be an ArrayBuffer or view");
  if (len % 34) return throw_msg(env, "bufWriteR: data is not whole 34-byte blocks", EFF_E_INVALID);
  return status(env, ctx, eff_buf_write_r(ctx, external<eff_buf>(env, a[1]), (int)i64(env, a[2]),
                                          (uint32_t)i64(env, a[3]), src, (uint32_t)(len / 34)));
}

napi_value BufBlocksR(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  uint32_t n = 0;
  if (eff_buf_blocks_r(external<eff_buf>(env, a[0]), &n)) return undefined(env);
  return make_int(env, n);
}

// ---- operations -------------------------------------------------------------

typedef int (*MatFn)(eff_ctx *, int, eff_buf *, eff_buf *, eff_buf *, uint32_t, uint32_t, uint32_t);

napi_value MatCall(napi_env env, napi_callback_info info, MatFn fn) {
  napi_value a[8];
  get_args(env, info, 8, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = fn(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
              external<eff_buf>(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6]),
              (uint32_t)i64(env, a[7], 1));
  return status(env, ctx, rc);
}

napi_value QMatmul(napi_env env, napi_callback_info info) { return MatCall(env, info, eff_qmatmul); }
napi_value QGemv(napi_env env, napi_callback_info info) { return MatCall(env, info, eff_qgemv); }
napi_value QGemm(napi_env env, napi_callback_info info) { return MatCall(env, info, eff_qgemm); }

// qgemmPlanned(ctx, type, w, x, y, rows, k, tokens, planTokens)
napi_value QGemmPlanned(napi_env env, napi_callback_info info) {
  napi_value a[9];
  get_args(env, info, 9, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = eff_qgemm_planned(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
                             external<eff_buf>(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6]),
                             (uint32_t)i64(env, a[7], 1), (uint32_t)i64(env, a[8], 1));
  return status(env, ctx, rc);
}

// gemmXLayout(ctx, type, rows, k, tokens, plan) -> {bytes, layout} | null
napi_value GemmXLayout(napi_env env, napi_callback_info info) {
  napi_value a[6];
  get_args(env, info, 6, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  size_t bytes = 0;
  uint32_t layout = 0;
  int rc = eff_gemm_x_layout(ctx, (int)i64(env, a[1]), (uint32_t)i64(env, a[2]), (uint32_t)i64(env, a[3]),
                             (uint32_t)i64(env, a[4], 1), (uint32_t)i64(env, a[5], 1), &bytes, &layout);
  if (rc) return status(env, ctx, rc);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "bytes", make_int(env, (int64_t)bytes));
  napi_set_named_property(env, o, "layout", make_int(env, (int64_t)layout));
  return o;
}

// gemmPrepareX(ctx, type, x, xh, rows, k, tokens, plan)
napi_value GemmPrepareX(napi_env env, napi_callback_info info) {
  napi_value a[8];
  get_args(env, info, 8, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = eff_gemm_prepare_x(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
                              (uint32_t)i64(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6], 1),
                              (uint32_t)i64(env, a[7], 1));
  return status(env, ctx, rc);
}

// qgemmPrepared(ctx, type, w, xh, y, rows, k, tokens, plan)
napi_value QGemmPrepared(napi_env env, napi_callback_info info) {
  napi_value a[9];
  get_args(env, info, 9, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = eff_qgemm_prepared(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
                              external<eff_buf>(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6]),
                              (uint32_t)i64(env, a[7], 1), (uint32_t)i64(env, a[8], 1));
  return status(env, ctx, rc);
}

// qmatmulCpuPath(ctx, type, w, x, y, rows, k, tokens) -> 0 | null
napi_value QMatmulCpuPath(napi_env env, napi_callback_info info) {
  napi_value a[8];
  get_args(env, info, 8, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = eff_qmatmul_cpu_path(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
                                external<eff_buf>(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6]),
                                (uint32_t)i64(env, a[7], 1));
  return status(env, ctx, rc);
}

// qmatmulXLayout(ctx, type, rows, k, tokens) -> {bytes, layout} | null
napi_value QMatmulXLayout(napi_env env, napi_callback_info info) {
  napi_value a[5];
  get_args(env, info, 5, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  size_t bytes = 0;
  uint32_t layout = 0;
  int rc = eff_qmatmul_x_layout(ctx, (int)i64(env, a[1]), (uint32_t)i64(env, a[2]), (uint32_t)i64(env, a[3]),
                                (uint32_t)i64(env, a[4], 1), &bytes, &layout);
  if (rc) return status(env, ctx, rc);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "bytes", make_int(env, (int64_t)bytes));
  napi_set_named_property(env, o, "layout", make_int(env, (int64_t)layout));
  return o;
}

// qmatmulPrepareX(ctx, type, x, xp, rows, k, tokens)
napi_value QMatmulPrepareX(napi_env env, napi_callback_info info) {
  napi_value a[7];
  get_args(env, info, 7, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = eff_qmatmul_prepare_x(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
                                 (uint32_t)i64(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6], 1));
  return status(env, ctx, rc);
}

// qmatmulPrepared(ctx, type, w, xp, y, rows, k, tokens)
napi_value QMatmulPrepared(napi_env env, napi_callback_info info) {
  napi_value a[8];
  get_args(env, info, 8, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  int rc = eff_qmatmul_prepared(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
                                external<eff_buf>(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6]),
                                (uint32_t)i64(env, a[7], 1));
  return status(env, ctx, rc);
}

// qgemvMulti(ctx, type, mode, [w...], x, [y...], [rows...], k, tokens)
napi_value QGemvMulti(napi_env env, napi_callback_info info) {
  napi_value a[9];
  get_args(env, info, 9, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  eff_buf *ws[4] = {nullptr, nullptr, nullptr, nullptr}, *ys[4] = {nullptr, nullptr, nullptr, nullptr};
  uint32_t rows[4] = {0, 0, 0, 0}, nw = 0, ny = 0, nr = 0;
  napi_get_array_length(env, a[3], &nw);
  napi_get_array_length(env, a[5], &ny);
  napi_get_array_length(env, a[6], &nr);
  if (nw > 4 || ny > 4 || nr != nw) return throw_msg(env, "gemv multi: 1..4 weights, as many row counts, at most 4 outputs");
  for (uint32_t i = 0; i < nw; ++i) {
    napi_value v;
    napi_get_element(env, a[3], i, &v);
    ws[i] = external<eff_buf>(env, v);
    napi_get_element(env, a[6], i, &v);
    rows[i] = (uint32_t)i64(env, v);
  }
  for (uint32_t i = 0; i < ny; ++i) {
    napi_value v;
    napi_get_element(env, a[5], i, &v);
    ys[i] = external<eff_buf>(env, v);
  }
  return status(env, ctx, eff_qgemv_multi(ctx, (int)i64(env, a[1]), (int)i64(env, a[2]), nw, ws,
                                          external<eff_buf>(env, a[4]), ys, rows, (uint32_t)i64(env, a[7]),
                                          (uint32_t)i64(env, a[8], 1)));
}

napi_value Dequant(napi_env env, napi_callback_info info) {
  napi_value a[5];
  get_args(env, info, 5, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  return status(env, ctx, eff_dequant(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]),
                                      external<eff_buf>(env, a[3]), (uint32_t)i64(env, a[4])));
}

// gather(ctx, type, w, ids, out, dim, tokens)
napi_value Gather(napi_env env, napi_callback_info info) {
  napi_value a[7];
  get_args(env, info, 7, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  return status(env, ctx, eff_gather(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]), external<eff_buf>(env, a[3]),
                                     external<eff_buf>(env, a[4]), (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6])));
}

// gatherNorm(ctx, type, w, ids, wn, eps, x, nrm, dim, tokens)
napi_value GatherNorm(napi_env env, napi_callback_info info) {
  napi_value a[10];
  get_args(env, info, 10, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  double eps = 0;
  napi_get_value_double(env, a[5], &eps);
  return status(env, ctx, eff_gather_norm(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]),
                                          external<eff_buf>(env, a[3]), external<eff_buf>(env, a[4]), (float)eps,
                                          external<eff_buf>(env, a[6]), external<eff_buf>(env, a[7]),
                                          (uint32_t)i64(env, a[8]), (uint32_t)i64(env, a[9])));
}

// topk(ctx, logits, base, vocab, m, penalIds (Uint32Array|null), serial, out)
napi_value TopK(napi_env env, napi_callback_info info) {
  napi_value a[8];
  get_args(env, info, 8, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  void *ids = nullptr;
  size_t len = 0;
  napi_valuetype t;
  napi_typeof(env, a[5], &t);
  if (t != napi_null && t != napi_undefined && !bytes_of(env, a[5], &ids, &len))
    return throw_msg(env, "topk: penalised ids must be a Uint32Array");
  return status(env, ctx, eff_topk(ctx, external<eff_buf>(env, a[1]), (uint32_t)i64(env, a[2]),
                                   (uint32_t)i64(env, a[3]), (uint32_t)i64(env, a[4]), (const uint32_t *)ids,
                                   (uint32_t)(len / 4), (uint32_t)i64(env, a[6]), external<eff_buf>(env, a[7])));
}

// qgemvTopk(ctx, type, w, x, y, rows, k, m, penalIds (Uint32Array|null), serial, out)
napi_value QGemvTopK(napi_env env, napi_callback_info info) {
  napi_value a[11];
  get_args(env, info, 11, a);
  eff_ctx *ctx = external<eff_ctx>(env, a[0]);
  void *ids = nullptr;
  size_t len = 0;
  napi_valuetype t;
  napi_typeof(env, a[8], &t);
  if (t != napi_null && t != napi_undefined && !bytes_of(env, a[8], &ids, &len))
    return throw_msg(env, "qgemvTopk: penalised ids must be a Uint32Array");
  return status(env, ctx, eff_qgemv_topk(ctx, (int)i64(env, a[1]), external<eff_buf>(env, a[2]),
                                         external<eff_buf>(env, a[3]), external<eff_buf>(env, a[4]),
                                         (uint32_t)i64(env, a[5]), (uint32_t)i64(env, a[6]), (uint32_t)i64(env, a[7]),
                                         (const uint32_t *)ids, (uint32_t)(len / 4), (uint32_t)i64(env, a[9]),
                                         external<eff_buf>(env, a[10])));
}

napi_value TopKOutBytes(napi_env env, napi_callback_info) { return make_int(env, (int64_t)eff_topk_out_bytes()); }

napi_value Register(napi_env env, napi_value exports) {
  struct { const char *name; napi_callback fn; } fns[] = {
      {"typeFromName", TypeFromName}, {"geometry", Geometry}, {"bufferMath", BufferMath},
      {"repack", Repack}, {"unrepack", Unrepack}, {"quantize", Quantize}, {"fillNormal", FillNormal},
      {"init", Init}, {"shutdown", Shutdown}, {"sync", Sync}, {"setOption", SetOption}, {"stats", Stats},
      {"bufAlloc", BufAlloc}, {"bufFree", BufFree}, {"bufWrite", BufWrite}, {"bufRead", BufRead},
      {"bufReadAsync", BufReadAsync}, {"bufSize", BufSize}, {"bufMarkR", BufMarkR}, {"bufBlocksR", BufBlocksR}, {"bufWriteR", BufWriteR},
      {"qmatmul", QMatmul}, {"qgemv", QGemv}, {"qgemvMulti", QGemvMulti}, {"qgemm", QGemm}, {"qgemmPlanned", QGemmPlanned}, {"dequant", Dequant}, {"gather", Gather}, {"gatherNorm", GatherNorm}, {"topk", TopK}, {"qgemvTopk", QGemvTopK},
      {"topkOutBytes", TopKOutBytes}, {"bufRetire", BufRetire}, {"graphBegin", GraphBegin},
      {"graphEnd", GraphEnd}, {"graphLaunch", GraphLaunch}, {"graphNodes", GraphNodes},
      {"graphDestroy", GraphDestroy}, {"gemmXLayout", GemmXLayout}, {"gemmPrepareX", GemmPrepareX},
      {"qgemmPrepared", QGemmPrepared}, {"qmatmulXLayout", QMatmulXLayout},
      {"qmatmulPrepareX", QMatmulPrepareX}, {"qmatmulPrepared", QMatmulPrepared},
      {"qmatmulCpuPath", QMatmulCpuPath},
  };
  for (auto &f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Register)
