"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

The reference ships no tests or golden vectors (README.md:150-156). Each
oracle function is pinned here by something independent of its own formula:
  * numpy library routines (float16 conversions, matmul, lexsort);
  * blocks built from field values by encoders written from the encode side of
    the GGUF layouts, compared with the field-level value of each weight;
  * closed-form special blocks (unit scales, zero mins) with known answers;
  * the reference's second statement of the Q8_0/Q6_K decoders (cpu.js:45-80);
  * known answers stated in the reference's comments (repack.js:225-229,
    kernels.bloques.wgsl.js:128-135, kernels.wgsl.js:381-384);
  * the IQ2_XXS grid fixture extracted from the reference's text
    (tests/golden/iq2xxs_grid.json, quant-tables.js:40-105), which the oracle
    loads and the product's own table is compared with.
"""
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

RNG = np.random.default_rng(1234)


def f16bits(v):
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


# ---- conversions -----------------------------------------------------------

def test_def16_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float64)
    got = np.array([orc.def16(int(b)) for b in bits])
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])


def test_af16_matches_numpy_rne(orc):
    # random normals, the subnormal range, exact ties between f16 neighbours, overflow
    h = np.arange(0, 0x7C00, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2
    vals = np.concatenate([RNG.normal(0, 1, 3000), RNG.normal(0, 1e-5, 2000), mids, -mids,
                           [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, np.inf, -np.inf, 2.0 ** -25,
                            3 * 2.0 ** -26, 2.0 ** -24, 1e-8]])
    for v in vals:
        want = int(np.array([np.float32(v)], dtype=np.float32).astype(np.float16).view(np.uint16)[0])
        assert orc.af16(v) == want, (v, hex(orc.af16(v)), hex(want))
    assert orc.af16(float("nan")) & 0x7C00 == 0x7C00


# ---- the IQ2_XXS grid ---------------------------------------------------------

def test_grid_invariants(orc):
    g = orc.grid_words()
    entries = [int(g[2 * e]) | (int(g[2 * e + 1]) << 32) for e in range(256)]
    assert len(set(entries)) == 256
    counts = {}
    for v in entries:
        for j in range(8):
            b = (v >> (8 * j)) & 0xFF
            counts[b] = counts.get(b, 0) + 1
    assert counts == {8: 1127, 25: 556, 43: 365}
    # first entries of ggml's iq2xxs_grid
    assert entries[0] == 0x0808080808080808 and entries[1] == 0x080808080808082B


def test_product_grid_equals_the_reference_fixture(orc):
    """The product's table (csrc/iq2xxs_grid.inc, 256 u64) holds exactly the
    words of the reference's IQ2XXS_GRID (the fixture extracted from
    quant-tables.js:40-105), entry by entry and in order."""
    import re
    inc = os.path.join(ROOT, "elffuss-engine_amd", "csrc", "iq2xxs_grid.inc")
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]{16})ull", open(inc).read())]
    g = orc.grid_words()
    assert len(vals) == 256
    assert vals == [int(g[2 * e]) | (int(g[2 * e + 1]) << 32) for e in range(256)]


# ---- block encoders (encode side of the GGUF layouts) ------------------------

def enc_q8_0(d, q):
    out = np.zeros(34, np.uint8)
    out[0:2] = np.array([f16bits(d)], np.uint16).view(np.uint8)
    out[2:] = np.asarray(q, np.int8).view(np.uint8)
    return out


def val_q8_0(d, q):
    return np.float32(np.float16(d)) * np.asarray(q, np.float32)


def enc_q4_k(d, dmin, sc, m, q):
    out = np.zeros(144, np.uint8)
    out[0:2] = np.array([f16bits(d)], np.uint16).view(np.uint8)
    out[2:4] = np.array([f16bits(dmin)], np.uint16).view(np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j]
            s[j + 4] |= m[j]
        else:
            s[j + 4] |= (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    out[4:16] = s.astype(np.uint8)
    for j in range(4):
        for l in range(32):
            out[16 + 32 * j + l] = q[64 * j + l] | (q[64 * j + 32 + l] << 4)
    return out


def val_q4_k(d, dmin, sc, m, q):
    d, dmin = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    out = np.zeros(256, np.float32)
    for i in range(256):
        sb = i // 32
        d1 = np.float32(d * np.float32(sc[sb]))
        m1 = np.float32(dmin * np.float32(m[sb]))
        out[i] = np.float32(np.float32(d1 * np.float32(q[i])) - m1)
    return out


def enc_q6_k(d, sc, q):
    out = np.zeros(210, np.uint8)
    for n in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * n + 32 * g + l] for g in range(4))
            out[64 * n + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            out[64 * n + 32 + l] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            out[128 + 32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    out[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    out[208:210] = np.array([f16bits(d)], np.uint16).view(np.uint8)
    return out


def val_q6_k(d, sc, q):
    d = np.float32(np.float16(d))
    out = np.zeros(256, np.float32)
    for i in range(256):
        d1 = np.float32(d * np.float32(sc[i // 16]))
        out[i] = np.float32(d1 * np.float32(int(q[i]) - 32))
    return out


def enc_q2_k(d, dmin, sc, m, q):
    out = np.zeros(84, np.uint8)
    for j in range(16):
        out[j] = sc[j] | (m[j] << 4)
    for n in range(2):
        for j in range(4):
            for l in range(32):
                out[16 + 32 * n + l] |= q[128 * n + 32 * j + l] << (2 * j)
    out[80:82] = np.array([f16bits(d)], np.uint16).view(np.uint8)
    out[82:84] = np.array([f16bits(dmin)], np.uint16).view(np.uint8)
    return out


def val_q2_k(d, dmin, sc, m, q):
    d, dmin = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    out = np.zeros(256, np.float32)
    for i in range(256):
        sb = i // 16
        dl = np.float32(d * np.float32(sc[sb]))
        ml = np.float32(dmin * np.float32(m[sb]))
        out[i] = np.float32(np.float32(dl * np.float32(q[i])) - ml)
    return out


def enc_iq2_xxs(d, ls, gidx, signs7):
    out = np.zeros(66, np.uint8)
    out[0:2] = np.array([f16bits(d)], np.uint16).view(np.uint8)
    for ib in range(8):
        a0 = sum(int(gidx[ib][l]) << (8 * l) for l in range(4))
        a1 = sum(int(signs7[ib][l]) << (7 * l) for l in range(4)) | (int(ls[ib]) << 28)
        out[2 + 8 * ib: 6 + 8 * ib] = np.array([a0], np.uint32).view(np.uint8)
        out[6 + 8 * ib: 10 + 8 * ib] = np.array([a1], np.uint32).view(np.uint8)
    return out


def val_iq2_xxs(grid, d, ls, gidx, signs7):
    d = np.float32(np.float16(d))
    out = np.zeros(256, np.float32)
    for ib in range(8):
        db = np.float32(np.float32(d * np.float32(0.5 + ls[ib])) * np.float32(0.25))
        for l in range(4):
            e = int(grid[2 * gidx[ib][l]]) | (int(grid[2 * gidx[ib][l] + 1]) << 32)
            s7 = int(signs7[ib][l])
            s8 = s7 | ((bin(s7).count("1") & 1) << 7)   # kernels.wgsl.js:381-384
            for j in range(8):
                g = np.float32((e >> (8 * j)) & 0xFF)
                sg = np.float32(-1.0 if (s8 >> j) & 1 else 1.0)
                out[32 * ib + 8 * l + j] = np.float32(np.float32(db * g) * sg)
    return out


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("trial", range(4))
def test_dequant_field_encoded_blocks(orc, trial):
    r = np.random.default_rng(100 + trial)
    # Q8_0
    d = float(r.uniform(1e-4, 1e-2)); q = r.integers(-128, 128, 32)
    assert _same(orc.dequant(orc.Q8_0, enc_q8_0(d, q), 1), val_q8_0(d, q))
    # Q4_K
    d, dmin = float(r.uniform(1e-4, 1e-2)), float(r.uniform(1e-4, 1e-2))
    sc, m, q = r.integers(0, 64, 8), r.integers(0, 64, 8), r.integers(0, 16, 256)
    assert _same(orc.dequant(orc.Q4_K, enc_q4_k(d, dmin, sc, m, q), 1), val_q4_k(d, dmin, sc, m, q))
    # Q6_K
    d = float(r.uniform(1e-5, 1e-3)); sc = r.integers(-128, 128, 16); q = r.integers(0, 64, 256)
    assert _same(orc.dequant(orc.Q6_K, enc_q6_k(d, sc, q), 1), val_q6_k(d, sc, q))
    # Q2_K
    d, dmin = float(r.uniform(1e-4, 1e-2)), float(r.uniform(1e-4, 1e-2))
    sc, m, q = r.integers(0, 16, 16), r.integers(0, 16, 16), r.integers(0, 4, 256)
    assert _same(orc.dequant(orc.Q2_K, enc_q2_k(d, dmin, sc, m, q), 1), val_q2_k(d, dmin, sc, m, q))
    # IQ2_XXS
    d = float(r.uniform(1e-4, 1e-2)); ls = r.integers(0, 16, 8)
    gidx = r.integers(0, 256, (8, 4)); s7 = r.integers(0, 128, (8, 4))
    assert _same(orc.dequant(orc.IQ2_XXS, enc_iq2_xxs(d, ls, gidx, s7), 1),
                 val_iq2_xxs(orc.grid_words(), d, ls, gidx, s7))


def test_dequant_closed_forms(orc):
    # Q4_K with d = 1, dmin = 0 and unit scales: weights are the nibbles themselves
    q = np.arange(256) % 16
    blk = enc_q4_k(1.0, 0.0, [1] * 8, [0] * 8, q)
    assert np.array_equal(orc.dequant(orc.Q4_K, blk, 1), q.astype(np.float32))
    # Q4_K with d = 0, dmin = 1 and min m = 5 everywhere: every weight is -5
    blk = enc_q4_k(0.0, 1.0, [0] * 8, [5] * 8, np.zeros(256, int))
    assert np.all(orc.dequant(orc.Q4_K, blk, 1) == -5.0)
    # Q4_K sub-block 6 alone carries scale 37 (split 6-bit encoding of j >= 4)
    sc = [0] * 8; sc[6] = 37
    blk = enc_q4_k(1.0, 0.0, sc, [0] * 8, np.ones(256, int))
    want = np.zeros(256, np.float32); want[192:224] = 37.0
    assert np.array_equal(orc.dequant(orc.Q4_K, blk, 1), want)
    # Q2_K, d = 1, unit scales: weight i = q_i; q_i = (i // 32) % 4 checks the shift order
    q = (np.arange(256) // 32) % 4
    blk = enc_q2_k(1.0, 0.0, [1] * 16, [0] * 16, q)
    assert np.array_equal(orc.dequant(orc.Q2_K, blk, 1), q.astype(np.float32))
    # Q6_K, d = 1, scale 1: weight i = q_i - 32
    q = np.arange(256) % 64
    blk = enc_q6_k(1.0, [1] * 16, q)
    assert np.array_equal(orc.dequant(orc.Q6_K, blk, 1), (q - 32).astype(np.float32))
    # IQ2_XXS: d = 1, ls = 15 -> db = 3.875; entry 0 is all 8s -> 31.0; sign bit pattern 1
    # (odd) sets the parity bit, so weights 0 and 7 are negative
    blk = enc_iq2_xxs(1.0, [15] * 8, np.zeros((8, 4), int), np.ones((8, 4), int))
    w = orc.dequant(orc.IQ2_XXS, blk, 1).reshape(32, 8)
    assert np.all(w[:, 0] == -31.0) and np.all(w[:, 7] == -31.0) and np.all(w[:, 1:7] == 31.0)


def test_dequant_q6k_q80_two_reference_statements(orc):
    """kernels.wgsl.js DECODERS and cpu.js filaAF32 state Q6_K and Q8_0 twice."""
    for t, nb in ((orc.Q6_K, 64), (orc.Q8_0, 256)):
        _, bb = orc.GEOMETRY[t]
        raw = RNG.integers(0, 256, nb * bb, dtype=np.uint8)
        # keep scales finite: f16 exponents well inside range
        if t == orc.Q6_K:
            for b in range(nb):
                raw[b * 210 + 208: b * 210 + 210] = np.array([f16bits(RNG.uniform(1e-4, 1e-2))], np.uint16).view(np.uint8)
        else:
            for b in range(nb):
                raw[b * 34: b * 34 + 2] = np.array([f16bits(RNG.uniform(1e-4, 1e-2))], np.uint16).view(np.uint8)
        assert _same(orc.dequant(t, raw, nb), orc.dequant_cpujs(t, raw, nb))


# ---- Q8_0 quantizer (cpu.js:273-287) -------------------------------------------

def test_q8_0_quantizer_known_answers(orc):
    # amax 127 -> d = 1 exactly, q = Math.round(x): ties toward +infinity
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.49999, -1.5, -127.0]
    out = orc.quantize_q8_0(x)
    assert out[0:2].view(np.uint16)[0] == 0x3C00
    assert list(out[2:10].view(np.int8)) == [127, 3, -2, 1, 0, 1, -1, -127]
    # all zero block: d = 0, q = 0
    assert not np.any(orc.quantize_q8_0(np.zeros(32, np.float32)))
    # d is amax/127 rounded f64 -> f32 -> f16 (aF16)
    x = RNG.normal(0, 0.02, 32 * 64).astype(np.float32)
    out = orc.quantize_q8_0(x).reshape(64, 34)
    amax = np.abs(x.reshape(64, 32)).max(axis=1).astype(np.float64)
    want_d = np.float32(amax / 127.0).astype(np.float16).view(np.uint16)
    assert np.array_equal(out[:, 0:2].copy().view(np.uint16).ravel(), want_d)
    # the round trip error is at most half a step of the unrounded d
    deq = orc.dequant(orc.Q8_0, out.ravel(), 64).reshape(64, 32)
    step = (amax / 127.0)[:, None]
    assert np.all(np.abs(deq - x.reshape(64, 32)) <= 0.5 * step + np.abs(deq) * 2e-3 + 1e-12)


# ---- repack (repack.js, kernels.bloques.wgsl.js) --------------------------------

def test_repack_known_answers(orc):
    assert orc.bytes_reordered(64) == 2176                 # repack.js:225-226
    assert orc.blocks_from_buffer(2304) == 67              # the 256-B pool reads 67 blocks
    assert orc.bytes_buffer_r(64) == 2176
    for n in range(1, 400):                                # N = floor(2L/17) is exact for <= 7 words of slack
        base = orc.bytes_reordered(n)
        for slack_words in range(0, 8):
            assert orc.blocks_from_buffer(base + 4 * slack_words) == n


@pytest.mark.parametrize("n", [1, 2, 3, 17, 64, 1001])
def test_repack_permutation_and_round_trip(orc, n):
    src = RNG.integers(0, 256, 34 * n, dtype=np.uint8)
    out = orc.repack(src, n)
    blocks = src.reshape(n, 34)
    assert np.array_equal(out[:32 * n], blocks[:, 2:].ravel())
    assert np.array_equal(out[32 * n: 34 * n], blocks[:, :2].ravel())
    assert not np.any(out[34 * n:])
    assert len(out) == orc.bytes_buffer_r(n) and len(out) % 16 == 0
    assert np.array_equal(orc.unrepack(out, n), src)
    # Q8_0R decodes to the same f32 bits as Q8_0 (kernels.wgsl.js:831-839)
    for b in range(n):
        blocks[b, 0:2] = np.array([f16bits(RNG.uniform(1e-4, 1e-1))], np.uint16).view(np.uint8)
    out = orc.repack(blocks.ravel(), n)
    assert _same(orc.dequant(orc.Q8_0R, out, n, n_tensor=n), orc.dequant(orc.Q8_0, blocks.ravel(), n))


# ---- matmul oracles ---------------------------------------------------------------

@pytest.mark.parametrize("tname", ["Q8_0", "Q4_K", "Q6_K", "Q2_K", "IQ2_XXS"])
def test_gemv_and_gemm_oracles_match_numpy(orc, eff, tname):
    t = orc.NAMES[tname]
    rows, k, tokens = 24, 512, 3
    w = eff.quantize(t, RNG.normal(0, 0.02, rows * k).astype(np.float32))
    x = RNG.normal(0, 1, tokens * k).astype(np.float32)
    e, _ = orc.GEOMETRY[t]
    W = orc.dequant(t, w, rows * k // e).reshape(rows, k).astype(np.float64)
    X = x.reshape(tokens, k).astype(np.float64)
    np.testing.assert_allclose(orc.gemv_f64(t, w, rows, k, x, tokens), X @ W.T, rtol=1e-12, atol=1e-12)
    W16 = W.astype(np.float32).astype(np.float16).astype(np.float64)
    X16 = x.reshape(tokens, k).astype(np.float16).astype(np.float64)
    np.testing.assert_allclose(orc.gemm_f16(t, w, rows, k, x, tokens), X16 @ W16.T, rtol=1e-12, atol=1e-12)


def test_gemv_oracle_linearity_and_unit_vectors(orc, eff):
    rows, k = 16, 256
    w = eff.quantize(orc.Q4_K, RNG.normal(0, 0.02, rows * k).astype(np.float32))
    W = orc.dequant(orc.Q4_K, w, rows).reshape(rows, k)
    for i in (0, 31, 32, 255):
        e = np.zeros(k, np.float32); e[i] = 1.0
        assert np.array_equal(orc.gemv_f64(orc.Q4_K, w, rows, k, e, 1)[0], W[:, i].astype(np.float64))


# ---- top-k ------------------------------------------------------------------------

def _numpy_topk(vals, m):
    v = vals.astype(np.float64)
    order = np.lexsort((np.arange(v.size), -v))
    return order[:m]


@pytest.mark.parametrize("vocab,m", [(1, 1), (50, 40), (4096, 40), (65536, 40), (70000, 192), (10, 40)])
def test_topk_matches_lexsort(orc, vocab, m):
    vals = RNG.normal(0, 3, vocab).astype(np.float32)
    vals[RNG.integers(0, vocab, max(1, vocab // 10))] = 1.25       # many ties
    ids, bits, nan = orc.topk(vals.view(np.uint32), m)
    assert not nan
    assert np.array_equal(ids, _numpy_topk(vals, m))
    assert np.array_equal(bits, vals.view(np.uint32)[ids])


def test_topk_signed_zero_and_nan(orc):
    vals = np.array([-0.0, 0.0, -1.0, -0.0, 2.0], np.float32)
    ids, _, nan = orc.topk(vals.view(np.uint32), 5)
    assert list(ids) == [4, 0, 1, 3, 2] and not nan                 # -0 == +0, ties by index
    vals[2] = np.nan
    _, _, nan = orc.topk(vals.view(np.uint32), 2)
    assert nan
    assert orc.topk_key(0x80000000) == orc.topk_key(0)


# ---- CPU path: the restatement pinned to its stated model ---------------------------
# The reference's CPU kernels ship only as compiled WebAssembly (not decoded, not runnable
# here). The restatement models them from the JS-visible contract: 40-byte activation blocks
# (cpu.js:25) as f32 d = amax/127, f32 s = d * sum(q), 32 int8 q = round(v/d) (C roundf, ties
# away from zero, as ggml's Q8_1 quantizer), an int32 dot per block and an f32 combine
# (cpu.js:350-381), over row chunks claimed by a pool (cpu.js:140-206, cpu-trabajo.js:27-72).
# What pins each part of that model is below; the literal WASM stays unpinned.

def _gamma(n):
    u = 2.0 ** -24
    return n * u / (1 - n * u)


def test_cpu_acts_fields(orc):
    """Every block: |q| <= 127, a +-127 in every nonzero block, x within half a
    step of q*d, the sum field equal to d times the integer sum, and a zero
    block all zero."""
    k, tokens = 2048, 3
    x = RNG.normal(0, 1, tokens * k).astype(np.float32)
    x[64:96] = 0.0                                   # one zero block
    x[300] = 1e30                                     # a block with one outlier
    a = orc.cpu_quantize_acts(x, k, tokens)
    q = a["q"].astype(np.int64)
    d = a["d"].astype(np.float64)
    xb = x.reshape(-1, 32).astype(np.float64)
    assert np.all(np.abs(q) <= 127)
    nz = np.any(xb != 0, axis=1)
    assert np.all(np.max(np.abs(q[nz]), axis=1) == 127)
    assert np.all(np.abs(xb - q * d[:, None]) <= d[:, None] * (0.5 + 2.0 ** -20))
    amax = np.max(np.abs(xb), axis=1)
    assert np.all(np.abs(d - amax / 127) <= amax / 127 * 2.0 ** -23)   # d = amax / 127 in f32
    assert np.array_equal(a["s"], (a["d"] * q.sum(axis=1).astype(np.float32)).astype(np.float32))
    z = 2                                             # x[64:96] is block 2
    assert a["d"][z] == 0 and a["s"][z] == 0 and not np.any(a["q"][z])


def test_cpu_acts_half_steps_round_away_from_zero(orc):
    """With amax = 127 the step d is 1 and q = round(v) exactly: ties go away
    from zero (C roundf, the modelled choice; JS Math.round would send -2.5 to
    -2 and -0.5 to -0)."""
    v = np.zeros(32, np.float32)
    v[:9] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -3.4999998]
    a = orc.cpu_quantize_acts(v, 32, 1)
    assert a["d"][0] == 1.0
    assert a["q"][0][:9].tolist() == [127, 3, -3, 1, -1, 2, -2, 127, -3]


@pytest.mark.parametrize("e", [-10, 0, 7])
def test_cpu_path_lossless_blocks_match_f64(orc, eff, e):
    """x of integers in [-127, 127] times 2^e with a +-127 in every block: the
    quantization is lossless (d = 2^e) and the integer dots exact, so the
    output differs from the f64 product only by the f32 combine, within
    gamma_(nb+1) * sum of |block terms| (recursive summation)."""
    rows, k, tokens = 96, 2048, 3
    xi = RNG.integers(-127, 128, tokens * k).astype(np.float64)
    xi[::32] = np.where(RNG.random(tokens * k // 32) < 0.5, -127.0, 127.0)
    x = (xi * 2.0 ** e).astype(np.float32)
    a = orc.cpu_quantize_acts(x, k, tokens)
    assert np.all(a["d"] == np.float32(2.0 ** e))
    w = eff.quantize(orc.Q8_0, RNG.normal(0, 0.02, rows * k).astype(np.float32))
    got = orc.cpu_matmul(orc.Q8_0, w, rows, k, x, tokens, 3).astype(np.float64)
    ref = orc.gemv_f64(orc.Q8_0, w, rows, k, x, tokens)
    wd = orc.dequant(orc.Q8_0, w, rows * k // 32).astype(np.float64).reshape(rows, k // 32, 32)
    terms = np.abs(np.einsum("rbi,tbi->trb", wd, x.astype(np.float64).reshape(tokens, k // 32, 32))).sum(axis=2)
    bound = _gamma(k // 32 + 1) * terms * 1.0001
    assert np.all(np.abs(got - ref) <= bound + 1e-300)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-6


def test_cpu_path_zero_block_and_one_element(orc, eff):
    """A zero x block contributes nothing (the output keeps its bits whatever
    the weights of that block); a block holding one nonzero value v gives
    w * v within the rounding of d and of the combine."""
    rows, k = 64, 1024
    w = eff.quantize(orc.Q8_0, RNG.normal(0, 0.02, rows * k).astype(np.float32))
    x = RNG.normal(0, 1, k).astype(np.float32)
    x[256:288] = 0.0                                  # block 8
    y1 = orc.cpu_matmul(orc.Q8_0, w, rows, k, x, 1, 1)
    w2 = w.copy().reshape(rows, k // 32, 34)
    w2[:, 8, 2:] = RNG.integers(0, 256, (rows, 32), dtype=np.uint8)
    y2 = orc.cpu_matmul(orc.Q8_0, w2.reshape(-1), rows, k, x, 1, 1)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    x1 = np.zeros(k, np.float32)
    x1[300] = np.float32(-0.7318)
    y = orc.cpu_matmul(orc.Q8_0, w, rows, k, x1, 1, 2)[0].astype(np.float64)
    wd = orc.dequant(orc.Q8_0, w, rows * k // 32).astype(np.float64).reshape(rows, k)
    want = wd[:, 300] * np.float64(x1[300])
    assert np.all(np.abs(y - want) <= np.abs(want) * 4 * 2.0 ** -24)


def test_cpu_path_same_bits_for_any_threads_and_chunks(orc, eff):
    """The rows a thread takes are summed alone, so the output has the same
    bits for 1 to 16 threads and for row counts that are no multiple of the
    chunk (cpu.js:140,173: chunks of max(4, ceil(rows / 4n / 4) * 4) rows)."""
    k = 512
    for rows in (1, 5, 67, 1000, 4097):
        w = eff.quantize(orc.Q8_0, RNG.normal(0, 0.02, rows * k).astype(np.float32))
        x = RNG.normal(0, 1, 2 * k).astype(np.float32)
        base = orc.cpu_matmul(orc.Q8_0, w, rows, k, x, 2, 1).view(np.uint32)
        for threads in (2, 3, 4, 7, 8, 16):
            got = orc.cpu_matmul(orc.Q8_0, w, rows, k, x, 2, threads).view(np.uint32)
            assert np.array_equal(got, base), (rows, threads)


def test_cpu_path_close_to_f64(orc, eff):
    rows, k = 64, 2048
    x = RNG.normal(0, 1, k).astype(np.float32)
    for t in (orc.Q8_0, orc.Q4_K):
        w = eff.quantize(t, RNG.normal(0, 0.02, rows * k).astype(np.float32))
        ref = orc.gemv_f64(t, w, rows, k, x, 1)[0]
        for threads in (1, 3):
            got = orc.cpu_matmul(t, w, rows, k, x, 1, threads)[0]
            rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
            assert rel < (2e-2 if t == orc.Q8_0 else 1e-6), (t, threads, rel)
