"""CPU tests of the product library: the C ABI loads and exports what the
header declares, and its host-side functions (quantizers, repack, buffer
arithmetic, input generator) agree with the oracle. No device calls."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "elffuss_amd.h")
RNG = np.random.default_rng(77)


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eff_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(eff):
    lib = ctypes.CDLL(eff.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(eff.EXPORTED) == syms


def test_type_table(eff):
    for name, code in eff.TYPES.items():
        assert eff.lib().eff_type_from_name(name.encode()) == code
        assert eff.lib().eff_type_name(code).decode() == name
    assert eff.lib().eff_type_from_name(b"Q4_0") == eff.E_TYPE
    assert eff.geometry("Q4_K") == (256, 144) and eff.geometry("IQ2_XXS") == (256, 66)
    assert eff.geometry("Q8_0R") == (32, 34)


def test_fill_normal_deterministic(eff):
    a = eff.fill_normal(5, 0.02, 100001)
    b = eff.fill_normal(5, 0.02, 100001)
    assert np.array_equal(a, b)
    assert np.array_equal(eff.fill_normal(5, 0.02, 1000), a[:1000])   # element i depends on (seed, i)
    assert abs(a.mean()) < 1e-3 and abs(a.std() - 0.02) < 5e-4


def test_q8_0_quantizer_is_the_reference_one(eff, orc):
    x = RNG.normal(0, 0.02, 32 * 4096).astype(np.float32)
    x[:32] = np.linspace(-3, 3, 32)
    x[32:64] = 0
    assert np.array_equal(eff.quantize("Q8_0", x), orc.quantize_q8_0(x))


@pytest.mark.parametrize("tname,tol", [("Q4_K", 0.12), ("Q6_K", 0.03), ("Q2_K", 0.45), ("IQ2_XXS", 0.6)])
def test_own_quantizers_produce_valid_blocks(eff, orc, tname, tol):
    """The reference has no quantizer for these types; blocks must decode (with
    the reference decoders) close to the source, with relative RMS error within
    what the bit width allows."""
    t = eff.TYPES[tname]
    x = RNG.normal(0, 0.02, 256 * 512).astype(np.float32)
    q = eff.quantize(t, x)
    _, bb = eff.geometry(t)
    assert q.size == 512 * bb
    w = orc.dequant(t, q, 512)
    assert np.all(np.isfinite(w))
    rel = np.linalg.norm(w - x) / np.linalg.norm(x)
    assert rel < tol, rel
    # zeros quantize to zeros
    assert np.all(orc.dequant(t, eff.quantize(t, np.zeros(256, np.float32)), 1) == 0)


@pytest.mark.parametrize("n", [1, 3, 64, 999])
def test_repack_matches_oracle(eff, orc, n):
    src = RNG.integers(0, 256, 34 * n, dtype=np.uint8)
    out = eff.repack(src, n)
    assert np.array_equal(out, orc.repack(src, n))
    assert np.array_equal(eff.unrepack(out, n), src)
    assert eff.bytes_buffer_r(n) == orc.bytes_buffer_r(n)
    assert eff.bytes_reordered(n) == orc.bytes_reordered(n)
    for extra in (0, 4, 12, 28):
        assert eff.blocks_from_buffer(orc.bytes_reordered(n) + extra) == n


def test_repack_rejects_short_destination(eff):
    lib = eff.lib()
    src = np.zeros(34 * 4, np.uint8)
    dst = np.zeros(100, np.uint8)
    assert lib.eff_repack(eff.Q8_0R, src.ctypes.data, 4, dst.ctypes.data, dst.size) == eff.E_BOUNDS
    assert lib.eff_repack(eff.Q8_0, src.ctypes.data, 4, dst.ctypes.data, dst.size) == eff.E_TYPE


def test_quantize_rejects_bad_shapes(eff):
    lib = eff.lib()
    x = np.zeros(300, np.float32)
    out = np.zeros(1000, np.uint8)
    assert lib.eff_quantize(eff.Q4_K, x.ctypes.data, 300, out.ctypes.data, out.size) == eff.E_SHAPE
    assert lib.eff_quantize(eff.Q8_0R, x.ctypes.data, 256, out.ctypes.data, out.size) == eff.E_TYPE
