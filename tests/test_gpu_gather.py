"""Embedding gather (quant.gather) and the gather fused with the first layer's
RMS norm (fusion.gatherNorma) on the GPU, against the oracle: the rows
bit-exact with the oracle's dequantization, the norm against f64."""
import numpy as np
import pytest

from test_gpu_parity import TYPES, make_weights, oracle_type, upload_w

pytestmark = pytest.mark.gpu


def oracle_rows(eff, orc, tname, gguf, n, dim, ids):
    base = "Q8_0" if tname == "Q8_0R" else tname
    e, _ = eff.geometry(base)
    table = orc.dequant(oracle_type(orc, tname), gguf, n).reshape(-1, dim)
    return table[ids]


@pytest.mark.parametrize("tname", TYPES)
@pytest.mark.parametrize("dim", [256, 2048])
def test_gather_bit_exact(ctx, eff, orc, tname, dim):
    rows, tokens = 300, 37
    t, data, gguf, n = make_weights(eff, tname, rows, dim, 500 + dim)
    ids = np.random.default_rng(dim).integers(0, rows, tokens).astype(np.uint32)
    ids[:3] = [0, rows - 1, 0]                    # first, last and a repeated row
    wb, ib, out = upload_w(ctx, eff, tname, data, n), ctx.upload(ids), ctx.alloc(tokens * dim * 4)
    before = ctx.stats()["gather"]
    ctx.gather(t, wb, ib, out, dim, tokens)
    assert ctx.stats()["gather"] == before + 1
    want = oracle_rows(eff, orc, tname, gguf, n, dim, ids)
    assert np.array_equal(out.read(np.uint32).reshape(tokens, dim), want.view(np.uint32))
    for b in (wb, ib, out):
        b.free()


@pytest.mark.parametrize("tname", ["Q8_0", "Q8_0R", "Q4_K", "Q6_K", "Q2_K"])
@pytest.mark.parametrize("dim", [256, 2048, 8192])
def test_gather_norm(ctx, eff, orc, tname, dim):
    rows, tokens, eps = 200, 9, 1e-6
    t, data, gguf, n = make_weights(eff, tname, rows, dim, 600 + dim)
    ids = np.random.default_rng(dim + 1).integers(0, rows, tokens).astype(np.uint32)
    wn = eff.fill_normal(601, 1.0, dim)
    wb, ib, wnb = upload_w(ctx, eff, tname, data, n), ctx.upload(ids), ctx.upload(wn)
    x, nrm = ctx.alloc(tokens * dim * 4), ctx.alloc(tokens * dim * 4)
    ctx.gather_norm(t, wb, ib, wnb, eps, x, nrm, dim, tokens)
    rows_f = oracle_rows(eff, orc, tname, gguf, n, dim, ids)
    assert np.array_equal(x.read(np.uint32).reshape(tokens, dim), rows_f.view(np.uint32))
    r64 = rows_f.astype(np.float64)
    scale = 1.0 / np.sqrt((r64 * r64).sum(axis=1, keepdims=True) / dim + eps)
    want = r64 * scale * wn.astype(np.float64)[None, :]
    got = nrm.read(np.float32).reshape(tokens, dim).astype(np.float64)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 2e-6


def test_gather_errors(ctx, eff):
    rows, dim = 8, 256
    t, data, gguf, n = make_weights(eff, "Q4_K", rows, dim, 1)
    wb, ib, out = ctx.upload(data), ctx.upload(np.zeros(4, np.uint32)), ctx.alloc(4 * dim * 4)
    with pytest.raises(eff.EffError) as e:
        ctx.gather(t, wb, ib, out, 300, 1)
    assert e.value.code == eff.E_SHAPE
    with pytest.raises(eff.EffError) as e:
        ctx.gather(t, wb, ib, out, dim, 5)                 # 5 ids, the buffer holds 4
    assert e.value.code == eff.E_BOUNDS
    ctx.gather(t, wb, ib, out, dim, 0)                     # nothing to do
    ti, di, _, ni = make_weights(eff, "IQ2_XXS", rows, dim, 2)
    wi, wn = ctx.upload(di), ctx.upload(np.ones(dim, np.float32))
    with pytest.raises(eff.EffError) as e:
        ctx.gather_norm(ti, wi, ib, wn, 1e-6, out, out, dim, 1)
    assert e.value.code == eff.E_TYPE
    _, dr, _, nr = make_weights(eff, "Q8_0R", rows, dim, 3)
    rb = ctx.upload(dr)
    with pytest.raises(eff.EffError) as e:
        ctx.gather(eff.Q8_0R, rb, ib, out, dim, 1)          # unmarked repacked buffer
    assert e.value.code == eff.E_MARK
