"""ctypes wrapper of liboracle.so, the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product never imports it.
Each function names the reference code it restates in oracle.c.
"""
import ctypes
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
# The IQ2_XXS grid as the reference holds it (quant-tables.js:40-105), read
# from the committed fixture that tests/golden/gen_iq2xxs_grid.py extracts from
# the reference's text; independent of the product's own table.
GRID_FIXTURE = os.path.join(os.path.dirname(HERE), "tests", "golden", "iq2xxs_grid.json")

Q8_0, Q2_K, Q4_K, Q6_K, IQ2_XXS, Q8_0R = 8, 10, 12, 14, 16, 264
GEOMETRY = {Q8_0: (32, 34), Q8_0R: (32, 34), Q2_K: (256, 84), Q4_K: (256, 144),
            Q6_K: (256, 210), IQ2_XXS: (256, 66)}
NAMES = {"Q8_0": Q8_0, "Q8_0R": Q8_0R, "Q2_K": Q2_K, "Q4_K": Q4_K, "Q6_K": Q6_K, "IQ2_XXS": IQ2_XXS}

_lib = None


def grid_words():
    """The IQ2_XXS grid as 512 u32 words (word 2e = bytes 0..3 of entry e)."""
    with open(GRID_FIXTURE) as f:
        words = json.load(f)["words"]
    assert len(words) == 512, len(words)
    return np.asarray(words, dtype=np.uint32)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle/liboracle.so is not built (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        p = ctypes.c_void_p
        u32, u64, i32, dbl = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_double
        L.or_def16.argtypes = [u32]; L.or_def16.restype = dbl
        L.or_af16.argtypes = [dbl]; L.or_af16.restype = u32
        L.or_set_grid.argtypes = [p]; L.or_set_grid.restype = None
        L.or_dequant.argtypes = [i32, p, u64, u32, p]; L.or_dequant.restype = i32
        L.or_dequant_cpujs.argtypes = [i32, p, u64, p]; L.or_dequant_cpujs.restype = i32
        L.or_gemv_f64.argtypes = [i32, p, u32, u32, u32, p, u32, p]; L.or_gemv_f64.restype = i32
        L.or_gemm_f16.argtypes = [i32, p, u32, u32, u32, p, u32, p]; L.or_gemm_f16.restype = i32
        L.or_topk_key.argtypes = [u32]; L.or_topk_key.restype = u32
        L.or_topk.argtypes = [p, u32, u32, p, p, ctypes.POINTER(i32)]; L.or_topk.restype = i32
        L.or_quantize_q8_0.argtypes = [p, u64, p]; L.or_quantize_q8_0.restype = i32
        L.or_bytes_reordered.argtypes = [u32]; L.or_bytes_reordered.restype = u64
        L.or_bytes_buffer_r.argtypes = [u32]; L.or_bytes_buffer_r.restype = u64
        L.or_blocks_from_buffer.argtypes = [u64]; L.or_blocks_from_buffer.restype = u32
        L.or_repack.argtypes = [p, u32, p, u64]; L.or_repack.restype = i32
        L.or_unrepack.argtypes = [p, u32, p]; L.or_unrepack.restype = i32
        L.or_cpu_matmul.argtypes = [i32, p, u32, u32, p, u32, i32, p]; L.or_cpu_matmul.restype = i32
        L.or_cpu_quantize_acts.argtypes = [p, u32, u32, p]; L.or_cpu_quantize_acts.restype = i32
        g = grid_words()
        L.or_set_grid(g.ctypes.data)
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data


def dequant(type_, blocks, n_blocks, n_tensor=0):
    """f32 weights of n_blocks blocks (bit-exact reference decoders)."""
    e, _ = GEOMETRY[type_]
    src = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * e, dtype=np.float32)
    rc = lib().or_dequant(type_, _ptr(src), n_blocks, n_tensor, _ptr(out))
    assert rc == 0, rc
    return out


def dequant_cpujs(type_, blocks, n_blocks):
    """cpu.js filaAF32 statement of the Q8_0 / Q6_K decoders."""
    e, _ = GEOMETRY[type_]
    src = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * e, dtype=np.float32)
    rc = lib().or_dequant_cpujs(type_, _ptr(src), n_blocks, _ptr(out))
    assert rc == 0, rc
    return out


def gemv_f64(type_, w, rows, k, x, tokens, n_tensor=0):
    src = np.ascontiguousarray(w, dtype=np.uint8)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(tokens * rows, dtype=np.float64)
    rc = lib().or_gemv_f64(type_, _ptr(src), n_tensor, rows, k, _ptr(xs), tokens, _ptr(y))
    assert rc == 0, rc
    return y.reshape(tokens, rows)


def gemm_f16(type_, w, rows, k, x, tokens, n_tensor=0):
    src = np.ascontiguousarray(w, dtype=np.uint8)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(tokens * rows, dtype=np.float64)
    rc = lib().or_gemm_f16(type_, _ptr(src), n_tensor, rows, k, _ptr(xs), tokens, _ptr(y))
    assert rc == 0, rc
    return y.reshape(tokens, rows)


def topk(logits_bits, m):
    """(ids, bits, nan_flag): the first m by (value desc, index asc)."""
    b = np.ascontiguousarray(logits_bits, dtype=np.uint32)
    ids = np.zeros(max(m, 1), dtype=np.uint32)
    bits = np.zeros(max(m, 1), dtype=np.uint32)
    nan = ctypes.c_int(0)
    n = lib().or_topk(_ptr(b), b.size, m, _ptr(ids), _ptr(bits), ctypes.byref(nan))
    assert n >= 0, n
    return ids[:n], bits[:n], bool(nan.value)


def topk_key(bits):
    return lib().or_topk_key(int(bits))


def quantize_q8_0(x):
    xs = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(xs.size // 32 * 34, dtype=np.uint8)
    rc = lib().or_quantize_q8_0(_ptr(xs), xs.size, _ptr(out))
    assert rc == 0, rc
    return out


def af16(v):
    return lib().or_af16(float(v))


def def16(bits):
    return lib().or_def16(int(bits))


def bytes_reordered(n):
    return lib().or_bytes_reordered(n)


def bytes_buffer_r(n):
    return lib().or_bytes_buffer_r(n)


def blocks_from_buffer(nbytes):
    return lib().or_blocks_from_buffer(nbytes)


def repack(src, n, dst_bytes=None):
    s = np.ascontiguousarray(src, dtype=np.uint8)
    size = bytes_buffer_r(n) if dst_bytes is None else dst_bytes
    out = np.full(size, 0xAA, dtype=np.uint8)
    rc = lib().or_repack(_ptr(s), n, _ptr(out), size)
    assert rc == 0, rc
    return out


def unrepack(src, n):
    s = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.zeros(34 * n, dtype=np.uint8)
    lib().or_unrepack(_ptr(s), n, _ptr(out))
    return out


# One 40-byte activation block of the CPU path as the restatement models it
# (cpu.js:25 BACT = 40): f32 d, f32 sum, 32 int8.
ACT_BLOCK = np.dtype([("d", "<f4"), ("s", "<f4"), ("q", "i1", (32,))])


def cpu_quantize_acts(x, k, tokens):
    """The CPU path's activation blocks (or_cpu_quantize_acts): per 32 values
    d = amax / 127, q = round(v / d) with ties away from zero, s = d * sum(q)."""
    xs = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(tokens * (k // 32), dtype=ACT_BLOCK)
    rc = lib().or_cpu_quantize_acts(_ptr(xs), k, tokens, _ptr(out))
    assert rc == 0, rc
    return out


def cpu_matmul(type_, w, rows, k, x, tokens, threads):
    """The CPU-path restatement: Q8_0 through quantized activations and an
    integer dot (parity unpinned), other types through f32 dequantize-and-dot."""
    src = np.ascontiguousarray(w, dtype=np.uint8)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(tokens * rows, dtype=np.float32)
    rc = lib().or_cpu_matmul(type_, _ptr(src), rows, k, _ptr(xs), tokens, threads, _ptr(y))
    assert rc == 0, rc
    return y.reshape(tokens, rows)
