"""Python binding of libelffuss_amd.so (the C ABI in include/elffuss_amd.h).

The binding is a thin ctypes layer: device buffers stay opaque `Buffer`
objects, every operation is enqueued on the context's HIP stream, and errors
come back as exceptions carrying the library's message. `NotApplicable` is the
reference's `null` ("this fast path does not apply", ops.gemv.js:13-21).

There is no fallback: if the shared library is missing or no GPU is present,
loading or opening a context raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libelffuss_amd.so")

OK, NOT_APPLICABLE = 0, 1
E_INVALID, E_TYPE, E_SHAPE, E_MARK, E_BOUNDS, E_DEVICE, E_NOMEM = -1, -2, -3, -4, -5, -6, -7
Q8_0, Q2_K, Q4_K, Q6_K, IQ2_XXS, Q8_0R = 8, 10, 12, 14, 16, 264
TYPES = {"Q8_0": Q8_0, "Q2_K": Q2_K, "Q4_K": Q4_K, "Q6_K": Q6_K, "IQ2_XXS": IQ2_XXS, "Q8_0R": Q8_0R}
OPT_GEMV_MAX_TOKENS, OPT_GEMM_MIN_TOKENS, OPT_GEMV_KERNEL, OPT_SPLIT_CONFIG, OPT_SPLIT_MIN_TOKENS = 1, 2, 3, 4, 5
OPT_GEMM_CONFIG, OPT_GEMM_SPLIT, OPT_SPLIT_SLICES = 6, 7, 8
GEMV_SECTIONS, GEMV_SWIGLU = 1, 2
TOPK_HEADER, TOPK_P_MAX, TOPK_CAP, TOPK_M_MAX = 8, 128, 256, 192
TOPK_NOALLOC_SCRATCH_BYTES = 18432

ERRORS = {E_INVALID: "invalid argument", E_TYPE: "unsupported type", E_SHAPE: "shape",
          E_MARK: "repack mark", E_BOUNDS: "bounds", E_DEVICE: "device", E_NOMEM: "out of memory"}


class EffError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{ERRORS.get(code, code)}] {msg}")
        self.code = code


class NotApplicable(Exception):
    """The requested fast path does not apply (the reference returns null)."""


class Stats(ctypes.Structure):
    _fields_ = [("gemv", ctypes.c_uint64), ("gemm", ctypes.c_uint64), ("skinny", ctypes.c_uint64),
                ("dequant", ctypes.c_uint64), ("topk", ctypes.c_uint64), ("not_applicable", ctypes.c_uint64),
                ("split", ctypes.c_uint64), ("fused", ctypes.c_uint64), ("gather", ctypes.c_uint64),
                ("gemm_x", ctypes.c_uint64), ("split_x", ctypes.c_uint64), ("cpu_path", ctypes.c_uint64)]


_lib = None


def lib():
    """Load the shared library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `make -C elffuss-engine_amd` (or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    p, u32, u64, i32, i64, sz = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int,
                                 ctypes.c_int64, ctypes.c_size_t)
    sig = {
        "eff_type_from_name": ([ctypes.c_char_p], i32),
        "eff_type_name": ([i32], ctypes.c_char_p),
        "eff_type_geometry": ([i32, ctypes.POINTER(u32), ctypes.POINTER(u32)], i32),
        "eff_init": ([i32, ctypes.POINTER(p)], i32),
        "eff_shutdown": ([p], i32),
        "eff_last_error": ([p], ctypes.c_char_p),
        "eff_stream": ([p], p),
        "eff_set_stream": ([p, p], i32),
        "eff_sync": ([p], i32),
        "eff_set_option": ([p, i32, i64], i32),
        "eff_get_stats": ([p, ctypes.POINTER(Stats)], i32),
        "eff_buf_alloc": ([p, sz, ctypes.POINTER(p)], i32),
        "eff_buf_wrap": ([p, p, sz, ctypes.POINTER(p)], i32),
        "eff_buf_free": ([p, p], i32),
        "eff_buf_retire": ([p, p], i32),
        "eff_graph_begin": ([p], i32),
        "eff_graph_end": ([p, ctypes.POINTER(p)], i32),
        "eff_graph_launch": ([p, p], i32),
        "eff_graph_nodes": ([p], sz),
        "eff_graph_destroy": ([p], i32),
        "eff_buf_size": ([p], sz),
        "eff_buf_device_ptr": ([p], p),
        "eff_buf_write": ([p, p, sz, p, sz], i32),
        "eff_buf_read": ([p, p, sz, p, sz], i32),
        "eff_buf_copy": ([p, p, sz, p, sz, sz], i32),
        "eff_read_begin": ([p, p, sz, sz, ctypes.POINTER(p)], i32),
        "eff_read_end": ([p, p], i32),
        "eff_read_poll": ([p], i32),
        "eff_read_error": ([p], ctypes.c_char_p),
        "eff_read_release": ([p], i32),
        "eff_bytes_reordered": ([i32, u32], sz),
        "eff_bytes_buffer_r": ([i32, u32], sz),
        "eff_blocks_from_buffer": ([i32, sz], u32),
        "eff_scales_from": ([i32, u32], u32),
        "eff_buf_mark_r": ([p, i32, u32], i32),
        "eff_buf_blocks_r": ([p, ctypes.POINTER(u32)], i32),
        "eff_buf_write_r": ([p, p, i32, u32, p, u32], i32),
        "eff_repack": ([i32, p, u32, p, sz], i32),
        "eff_unrepack": ([i32, p, sz, u32, p], i32),
        "eff_quantize": ([i32, p, sz, p, sz], i32),
        "eff_fill_normal": ([u32, ctypes.c_float, p, sz], i32),
        "eff_qmatmul": ([p, i32, p, p, p, u32, u32, u32], i32),
        "eff_qgemv": ([p, i32, p, p, p, u32, u32, u32], i32),
        "eff_qgemm": ([p, i32, p, p, p, u32, u32, u32], i32),
        "eff_qgemm_planned": ([p, i32, p, p, p, u32, u32, u32, u32], i32),
        "eff_gemm_x_layout": ([p, i32, u32, u32, u32, u32, ctypes.POINTER(sz), ctypes.POINTER(u32)], i32),
        "eff_gemm_prepare_x": ([p, i32, p, p, u32, u32, u32, u32], i32),
        "eff_qgemm_prepared": ([p, i32, p, p, p, u32, u32, u32, u32], i32),
        "eff_qmatmul_cpu_path": ([p, i32, p, p, p, u32, u32, u32], i32),
        "eff_qmatmul_x_layout": ([p, i32, u32, u32, u32, ctypes.POINTER(sz), ctypes.POINTER(u32)], i32),
        "eff_qmatmul_prepare_x": ([p, i32, p, p, u32, u32, u32], i32),
        "eff_qmatmul_prepared": ([p, i32, p, p, p, u32, u32, u32], i32),
        "eff_qgemv_multi": ([p, i32, i32, u32, ctypes.POINTER(p), p, ctypes.POINTER(p), ctypes.POINTER(u32), u32, u32],
                            i32),
        "eff_dequant": ([p, i32, p, p, u32], i32),
        "eff_gather": ([p, i32, p, p, p, u32, u32], i32),
        "eff_gather_norm": ([p, i32, p, p, p, ctypes.c_float, p, p, u32, u32], i32),
        "eff_topk": ([p, p, u32, u32, u32, p, u32, u32, p], i32),
        "eff_topk_noalloc": ([p, p, u32, u32, u32, p, u32, u32, p], i32),
        "eff_read_floor": ([p, p, ctypes.c_size_t, u32, u32, p], i32),
        "eff_qgemv_topk": ([p, i32, p, p, p, u32, u32, u32, p, u32, u32, p], i32),
        "eff_topk_out_bytes": ([], sz),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


EXPORTED = ("eff_type_from_name eff_type_name eff_type_geometry eff_init eff_shutdown eff_last_error "
            "eff_stream eff_set_stream eff_sync eff_set_option eff_get_stats eff_buf_alloc eff_buf_wrap "
            "eff_buf_free eff_buf_retire eff_graph_begin eff_graph_end eff_graph_launch eff_graph_nodes "
            "eff_graph_destroy eff_buf_size eff_buf_device_ptr eff_buf_write eff_buf_read eff_buf_copy "
            "eff_read_begin eff_read_end eff_read_poll eff_read_error eff_read_release "
            "eff_bytes_reordered eff_bytes_buffer_r eff_blocks_from_buffer eff_scales_from eff_buf_mark_r "
            "eff_buf_blocks_r eff_buf_write_r eff_repack eff_unrepack eff_quantize eff_fill_normal eff_qmatmul eff_qgemv "
            "eff_qgemm eff_qgemm_planned eff_gemm_x_layout eff_gemm_prepare_x eff_qgemm_prepared eff_qmatmul_x_layout eff_qmatmul_prepare_x eff_qmatmul_prepared eff_qmatmul_cpu_path eff_qgemv_multi eff_dequant eff_gather eff_gather_norm eff_topk eff_topk_noalloc eff_qgemv_topk eff_topk_out_bytes eff_read_floor").split()


def type_code(t):
    if isinstance(t, str):
        if t not in TYPES:
            raise EffError(E_TYPE, f"unsupported quantization type «{t}»")
        return TYPES[t]
    return int(t)


def geometry(t):
    e, b = ctypes.c_uint32(), ctypes.c_uint32()
    rc = lib().eff_type_geometry(type_code(t), ctypes.byref(e), ctypes.byref(b))
    if rc:
        raise EffError(rc, f"unknown type {t}")
    return e.value, b.value


# ---- host data preparation (no device needed) ------------------------------

def fill_normal(seed, sigma, n):
    out = np.empty(n, dtype=np.float32)
    rc = lib().eff_fill_normal(seed & 0xFFFFFFFF, sigma, out.ctypes.data, n)
    if rc:
        raise EffError(rc, "fill_normal")
    return out


def quantize(t, x):
    t = type_code(t)
    xs = np.ascontiguousarray(x, dtype=np.float32).ravel()
    e, b = geometry(t)
    out = np.empty(xs.size // e * b, dtype=np.uint8)
    rc = lib().eff_quantize(t, xs.ctypes.data, xs.size, out.ctypes.data, out.size)
    if rc:
        raise EffError(rc, f"quantize {t}")
    return out


def repack(src, n_blocks):
    s = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(lib().eff_bytes_buffer_r(Q8_0R, n_blocks), dtype=np.uint8)
    rc = lib().eff_repack(Q8_0R, s.ctypes.data, n_blocks, out.ctypes.data, out.size)
    if rc:
        raise EffError(rc, "repack")
    return out


def unrepack(src, n_blocks):
    s = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(34 * n_blocks, dtype=np.uint8)
    rc = lib().eff_unrepack(Q8_0R, s.ctypes.data, s.size, n_blocks, out.ctypes.data)
    if rc:
        raise EffError(rc, "unrepack")
    return out


def bytes_buffer_r(n):
    return lib().eff_bytes_buffer_r(Q8_0R, n)


def bytes_reordered(n):
    return lib().eff_bytes_reordered(Q8_0R, n)


def blocks_from_buffer(nbytes):
    return lib().eff_blocks_from_buffer(Q8_0R, nbytes)


# ---- device ------------------------------------------------------------------

class Buffer:
    def __init__(self, ctx, handle, size):
        self.ctx, self.handle, self.size = ctx, handle, size

    @property
    def ptr(self):
        return lib().eff_buf_device_ptr(self.handle)

    def write(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        self.ctx._check(lib().eff_buf_write(self.ctx.h, self.handle, offset, a.ctypes.data, a.nbytes))

    def read(self, dtype=np.uint8, count=None, offset=0):
        dt = np.dtype(dtype)
        n = (self.size - offset) // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        self.ctx._check(lib().eff_buf_read(self.ctx.h, self.handle, offset, out.ctypes.data, out.nbytes))
        return out

    def mark_r(self, n_blocks):
        rc = lib().eff_buf_mark_r(self.handle, Q8_0R, n_blocks)
        if rc:
            raise EffError(rc, f"mark_r: buffer of {self.size} bytes for {n_blocks} blocks")

    def write_r(self, first_block, gguf_bytes):
        """Repack GGUF Q8_0 blocks (bytes) into this marked buffer from block first_block."""
        a = np.ascontiguousarray(gguf_bytes, dtype=np.uint8)
        if a.nbytes % 34:
            raise ValueError(f"write_r: {a.nbytes} bytes are not whole 34-byte blocks")
        self.ctx._check(lib().eff_buf_write_r(self.ctx.h, self.handle, Q8_0R, first_block, a.ctypes.data,
                                              a.nbytes // 34))

    def blocks_r(self):
        n = ctypes.c_uint32()
        rc = lib().eff_buf_blocks_r(self.handle, ctypes.byref(n))
        if rc:
            raise EffError(rc, "buffer carries no repack mark")
        return n.value

    def free(self):
        if self.handle:
            self.ctx._check(lib().eff_buf_free(self.ctx.h, self.handle))
            self.handle = None

    def retire(self):
        """Give the buffer back in stream order, without waiting (eff_buf_retire)."""
        if self.handle:
            self.ctx._check(lib().eff_buf_retire(self.ctx.h, self.handle))
            self.handle = None


class Graph:
    """Launches recorded between Context.graph_begin() and graph_end()."""

    def __init__(self, ctx, handle):
        self.ctx, self.handle = ctx, handle

    @property
    def nodes(self):
        return lib().eff_graph_nodes(self.handle)

    def launch(self):
        self.ctx._check(lib().eff_graph_launch(self.ctx.h, self.handle))

    def destroy(self):
        if self.handle:
            lib().eff_graph_destroy(self.handle)
            self.handle = None


class Context:
    """One HIP device context and its stream (eff_init)."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        rc = lib().eff_init(device, ctypes.byref(h))
        if rc:
            raise EffError(rc, f"eff_init(device={device}) failed: no usable HIP device")
        self.h = h

    def close(self):
        if self.h:
            lib().eff_shutdown(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc == NOT_APPLICABLE:
            raise NotApplicable()
        if rc:
            raise EffError(rc, lib().eff_last_error(self.h).decode())
        return rc

    @property
    def stream(self):
        return lib().eff_stream(self.h)

    def set_stream(self, stream_ptr):
        self._check(lib().eff_set_stream(self.h, stream_ptr))

    def sync(self):
        self._check(lib().eff_sync(self.h))

    def graph_begin(self):
        """Record (not run) the launches enqueued from now on (eff_graph_begin)."""
        self._check(lib().eff_graph_begin(self.h))

    def graph_end(self):
        g = ctypes.c_void_p()
        self._check(lib().eff_graph_end(self.h, ctypes.byref(g)))
        return Graph(self, g)

    def set_option(self, opt, value):
        self._check(lib().eff_set_option(self.h, opt, value))

    def stats(self):
        s = Stats()
        self._check(lib().eff_get_stats(self.h, ctypes.byref(s)))
        return {f: getattr(s, f) for f, _ in Stats._fields_}

    def alloc(self, nbytes):
        h = ctypes.c_void_p()
        self._check(lib().eff_buf_alloc(self.h, nbytes, ctypes.byref(h)))
        return Buffer(self, h, nbytes)

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        b = self.alloc(max(a.nbytes, 1))
        if a.nbytes:
            b.write(a)
        return b

    def copy(self, dst, src, n, dst_offset=0, src_offset=0):
        self._check(lib().eff_buf_copy(self.h, dst.handle, dst_offset, src.handle, src_offset, n))

    def qmatmul(self, t, w, x, y, rows, k, tokens=1):
        self._check(lib().eff_qmatmul(self.h, type_code(t), w.handle, x.handle, y.handle, rows, k, tokens))

    def qgemv(self, t, w, x, y, rows, k, tokens=1):
        self._check(lib().eff_qgemv(self.h, type_code(t), w.handle, x.handle, y.handle, rows, k, tokens))

    def qgemv_multi(self, t, mode, ws, x, ys, rows, k, tokens=1):
        """Fused GEMV (mode GEMV_SECTIONS or GEMV_SWIGLU) over the buffers ws, into ys."""
        n = len(ws)
        wa = (ctypes.c_void_p * n)(*[w.handle for w in ws])
        ya = (ctypes.c_void_p * len(ys))(*[y.handle for y in ys])
        ra = (ctypes.c_uint32 * n)(*rows)
        self._check(lib().eff_qgemv_multi(self.h, type_code(t), mode, n, wa, x.handle, ya, ra, k, tokens))

    def qgemm(self, t, w, x, y, rows, k, tokens):
        self._check(lib().eff_qgemm(self.h, type_code(t), w.handle, x.handle, y.handle, rows, k, tokens))

    def qgemm_planned(self, t, w, x, y, rows, k, tokens, plan_tokens):
        """The GEMM over `tokens` rows of x with the configuration of a `plan_tokens` batch."""
        self._check(lib().eff_qgemm_planned(self.h, type_code(t), w.handle, x.handle, y.handle, rows, k, tokens,
                                            plan_tokens))

    def gemm_x_layout(self, t, rows, k, tokens, plan_tokens=None):
        """(bytes, layout id) of x prepared for the GEMM (eff_gemm_x_layout)."""
        nb, lay = ctypes.c_size_t(), ctypes.c_uint32()
        self._check(lib().eff_gemm_x_layout(self.h, type_code(t), rows, k, tokens, plan_tokens or tokens,
                                            ctypes.byref(nb), ctypes.byref(lay)))
        return nb.value, lay.value

    def gemm_prepare_x(self, t, x, xh, rows, k, tokens, plan_tokens=None):
        self._check(lib().eff_gemm_prepare_x(self.h, type_code(t), x.handle, xh.handle, rows, k, tokens,
                                             plan_tokens or tokens))

    def qgemm_prepared(self, t, w, xh, y, rows, k, tokens, plan_tokens=None):
        self._check(lib().eff_qgemm_prepared(self.h, type_code(t), w.handle, xh.handle, y.handle, rows, k, tokens,
                                             plan_tokens or tokens))

    def qmatmul_cpu_path(self, t, w, x, y, rows, k, tokens=1):
        """Y = W X with the reference CPU path's arithmetic (Q8_0; eff_qmatmul_cpu_path)."""
        self._check(lib().eff_qmatmul_cpu_path(self.h, type_code(t), w.handle, x.handle, y.handle, rows, k, tokens))

    def qmatmul_x_layout(self, t, rows, k, tokens):
        """(bytes, layout id) of the x the router's path for this call reads
        prepared (eff_qmatmul_x_layout); NotApplicable where it reads x itself."""
        nb, lay = ctypes.c_size_t(), ctypes.c_uint32()
        self._check(lib().eff_qmatmul_x_layout(self.h, type_code(t), rows, k, tokens, ctypes.byref(nb),
                                               ctypes.byref(lay)))
        return nb.value, lay.value

    def qmatmul_prepare_x(self, t, x, xp, rows, k, tokens):
        self._check(lib().eff_qmatmul_prepare_x(self.h, type_code(t), x.handle, xp.handle, rows, k, tokens))

    def qmatmul_prepared(self, t, w, xp, y, rows, k, tokens):
        self._check(lib().eff_qmatmul_prepared(self.h, type_code(t), w.handle, xp.handle, y.handle, rows, k, tokens))

    def read_async(self, buf, dtype=np.uint8, count=None, offset=0):
        """Enqueue a readback now; returns a callable that waits and gives the array."""
        dt = np.dtype(dtype)
        n = (buf.size - offset) // dt.itemsize if count is None else count
        r = ctypes.c_void_p()
        self._check(lib().eff_read_begin(self.h, buf.handle, offset, n * dt.itemsize, ctypes.byref(r)))

        def finish():
            out = np.empty(n, dtype=dt)
            try:
                rc = lib().eff_read_end(r, out.ctypes.data)
                if rc:
                    raise EffError(rc, lib().eff_read_error(r).decode())
            finally:
                lib().eff_read_release(r)
            return out
        return finish

    def dequant(self, t, w, out, n_blocks):
        self._check(lib().eff_dequant(self.h, type_code(t), w.handle, out.handle, n_blocks))

    def gather(self, t, w, ids, out, dim, tokens):
        self._check(lib().eff_gather(self.h, type_code(t), w.handle, ids.handle, out.handle, dim, tokens))

    def gather_norm(self, t, w, ids, wn, eps, x, nrm, dim, tokens):
        self._check(lib().eff_gather_norm(self.h, type_code(t), w.handle, ids.handle, wn.handle, eps, x.handle,
                                          nrm.handle, dim, tokens))

    def topk(self, logits, base, vocab, m, penal_ids=(), serial=1, out=None):
        ids = np.ascontiguousarray(np.asarray(penal_ids, dtype=np.uint32))
        if out is None:
            out = self.alloc(lib().eff_topk_out_bytes())
        self._check(lib().eff_topk(self.h, logits.handle, base, vocab, m,
                                   ids.ctypes.data if ids.size else None, ids.size, serial, out.handle))
        return out


    def qgemv_topk(self, t, w, x, y, rows, k, m, penal_ids=(), serial=1, out=None):
        """eff_qgemv_topk: y = W x (one token), then the top-m record of y into `out`."""
        ids = np.ascontiguousarray(np.asarray(penal_ids, dtype=np.uint32))
        if out is None:
            out = self.alloc(lib().eff_topk_out_bytes())
        self._check(lib().eff_qgemv_topk(self.h, type_code(t), w.handle, x.handle, y.handle, rows, k, m,
                                         ids.ctypes.data if ids.size else None, ids.size, serial, out.handle))
        return out

    def topk_noalloc(self, logits, base, vocab, m, penal_ids=(), serial=1, out=None):
        """eff_topk_noalloc: the top-k with the library's fixed scratch (no allocation)."""
        ids = np.ascontiguousarray(np.asarray(penal_ids, dtype=np.uint32))
        if out is None:
            out = self.alloc(lib().eff_topk_out_bytes())
        self._check(lib().eff_topk_noalloc(self.h, logits.handle, base, vocab, m,
                                           ids.ctypes.data if ids.size else None, ids.size, serial, out.handle))
        return out

    def read_floor(self, src, nbytes, workgroups, unroll, sink):
        """eff_read_floor: a streaming read of nbytes of src (measurement only)."""
        self._check(lib().eff_read_floor(self.h, src.handle, nbytes, workgroups, unroll, sink.handle))


def parse_topk(u):
    """Split the top-k output record (kernels.topk.wgsl.js:50-59 layout)."""
    u = np.asarray(u, dtype=np.uint32)
    n = int(u[0])
    pairs = u[TOPK_HEADER + TOPK_P_MAX:].reshape(-1, 2)
    return {"n": n, "flags": int(u[1]), "n_penal": int(u[2]), "chunks": int(u[3]), "serial": int(u[4]),
            "penal_bits": u[TOPK_HEADER:TOPK_HEADER + int(u[2])].copy(),
            "ids": pairs[:n, 0].copy(), "bits": pairs[:n, 1].copy()}
