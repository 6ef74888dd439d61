"""The BASELINE.json configurations at their full sizes, through the C ABI,
against the oracle (whole outputs everywhere; the large products also against
the oracle's own routines on row slices) and, for C4, the top-40 of the GPU's
own logits bit-exact."""
import numpy as np
import pytest

from test_gpu_parity import check_close, make_weights, oracle_type, upload_w

pytestmark = pytest.mark.gpu


def run(ctx, eff, tname, rows, k, tokens, seed, force=None):
    t, data, gguf, n = make_weights(eff, tname, rows, k, seed)
    x = eff.fill_normal(seed + 1, 1.0, tokens * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    if force == "gemm":
        ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
    else:
        ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    y = yb.read(np.float32).reshape(tokens, rows)
    for b in (wb, xb, yb):
        b.free()
    return gguf, x, y


def row_slice(eff, tname, gguf, k, r0, r1):
    base = "Q8_0" if tname == "Q8_0R" else tname
    e, bb = eff.geometry(base)
    rb = k // e * bb
    return gguf[r0 * rb: r1 * rb]


@pytest.mark.parametrize("tname", ["Q8_0", "Q8_0R"])
def test_c1_q8_0_gemv_8192x2048(ctx, eff, orc, tname):
    gguf, x, y = run(ctx, eff, tname, 8192, 2048, 1, 101)
    check_close(y, orc.gemv_f64(orc.Q8_0, gguf, 8192, 2048, x, 1), f"C1 {tname}")


@pytest.mark.parametrize("tokens", [1, 512])
def test_c1_c3_cpu_path_product_bit_exact(ctx, eff, orc, tokens):
    """C1 (one token) and C3 M = 512 through the CPU path's arithmetic
    (eff_qmatmul_cpu_path): every output bit-equal to the oracle's restatement
    of cpu-kernels.js (or_cpu_matmul), the path north_star names."""
    rows, k = 8192, 2048
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 105 + tokens)
    x = eff.fill_normal(106 + tokens, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qmatmul_cpu_path(t, wb, xb, yb, rows, k, tokens)
    got = yb.read(np.uint32, tokens * rows)
    for b in (wb, xb, yb):
        b.free()
    ref = orc.cpu_matmul(orc.Q8_0, gguf, rows, k, x, tokens, 8)
    assert np.array_equal(got, ref.view(np.uint32).reshape(-1)), \
        f"{int(np.sum(got != ref.view(np.uint32).reshape(-1)))} of {got.size} outputs differ"


def test_c2_q4_k_gemv_2048x8192(ctx, eff, orc):
    gguf, x, y = run(ctx, eff, "Q4_K", 2048, 8192, 1, 202)
    check_close(y, orc.gemv_f64(orc.Q4_K, gguf, 2048, 8192, x, 1), "C2 Q4_K")


def full_f16_ref(orc, ot, gguf, rows, k, x, tokens):
    """The fp16-rounded oracle over every row: the exact f32 dequantization
    rounded to fp16 (fp16(d q), the reference's f16 weight tile) times x
    rounded to fp16, accumulated in f64 (equal to orc.gemm_f16, which
    tests/test_oracle.py checks)."""
    w16 = orc.dequant(ot, gguf, rows * k // orc.GEOMETRY[ot][0]).astype(np.float16).astype(np.float64)
    x16 = np.asarray(x, np.float32).astype(np.float16).astype(np.float64)
    return x16.reshape(tokens, k) @ w16.reshape(rows, k).T


def full_f64_ref(orc, ot, gguf, rows, k, x, tokens):
    """The f64 oracle over every row: the exact dequantization times f32 x."""
    w = orc.dequant(ot, gguf, rows * k // orc.GEOMETRY[ot][0]).astype(np.float64)
    return np.asarray(x, np.float64).reshape(tokens, k) @ w.reshape(rows, k).T


@pytest.mark.parametrize("tokens", [512, 2048])
def test_c3_q8_0_gemm(ctx, eff, orc, tokens):
    """The whole output (all 8192 rows), against the fp16-rounded oracle; the
    oracle's own gemm_f16 on two row slices as a cross-check."""
    rows, k = 8192, 2048
    gguf, x, y = run(ctx, eff, "Q8_0", rows, k, tokens, 303)
    check_close(y, full_f16_ref(orc, orc.Q8_0, gguf, rows, k, x, tokens), f"C3 M={tokens} all rows")
    for r0, r1 in ((0, 96), (rows - 160, rows)):
        ref = orc.gemm_f16(orc.Q8_0, row_slice(eff, "Q8_0", gguf, k, r0, r1), r1 - r0, k, x, tokens)
        check_close(y[:, r0:r1], ref, f"C3 M={tokens} rows {r0}:{r1}")


def test_c4_q6_k_head_and_top40(ctx, eff, orc):
    rows, k = 65536, 2048
    t, data, gguf, n = make_weights(eff, "Q6_K", rows, k, 404)
    x = eff.fill_normal(405, 1.0, k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(rows * 4)
    ctx.qmatmul(t, wb, xb, yb, rows, k, 1)
    out = ctx.topk(yb, 0, rows, 40, penal_ids=[3, 77], serial=9)
    y = yb.read(np.float32)
    r = eff.parse_topk(out.read(np.uint32))
    check_close(y[None, :], orc.gemv_f64(orc.Q6_K, gguf, rows, k, x, 1), "C4 Q6_K logits")
    ids, bits, nan = orc.topk(y.view(np.uint32), 40)
    assert not nan and r["flags"] == 0 and r["n"] == 40 and r["serial"] == 9
    assert np.array_equal(r["ids"], ids) and np.array_equal(r["bits"], bits)
    assert np.array_equal(r["penal_bits"], y.view(np.uint32)[[3, 77]])


@pytest.mark.parametrize("tname", ["Q2_K", "IQ2_XXS"])
@pytest.mark.parametrize("tokens", [1, 8, 32, 128])
def test_c5_low_bit_sweep(ctx, eff, orc, tname, tokens):
    rows, k = 8192, 2048
    gguf, x, y = run(ctx, eff, tname, rows, k, tokens, 505 + tokens)
    # f32 accuracy at every M (the split-x product from 4 tokens, the GEMV below)
    ot = oracle_type(orc, tname)
    if tokens < 64:
        check_close(y, orc.gemv_f64(ot, gguf, rows, k, x, tokens), f"C5 {tname} M={tokens}")
    else:
        check_close(y, full_f64_ref(orc, ot, gguf, rows, k, x, tokens), f"C5 {tname} M={tokens} all rows")
        for r0, r1 in ((0, 512), (rows - 512, rows)):
            ref = orc.gemv_f64(ot, row_slice(eff, tname, gguf, k, r0, r1), r1 - r0, k, x, tokens)
            check_close(y[:, r0:r1], ref, f"C5 {tname} M={tokens} rows {r0}:{r1}")
