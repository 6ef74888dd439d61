"""eff_topk_noalloc through the C ABI against eff_topk: the same record on two
calls in a row, the second over a smaller vocabulary (the fixed scratch still
holds the first call's candidates when it starts), with ties, a penalty list
and a base offset; and the vocabulary limit of the fixed scratch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_topk_noalloc_matches_topk_on_two_calls(ctx, eff):
    rng = np.random.default_rng(5)
    cases = [(200000, 40, [3, 150000], 0), (4097, 100, [7], 33)]
    bufs, want = [], []
    for vocab, m, pen, base in cases:
        vals = np.zeros(base + vocab, np.float32)
        vals[base:] = rng.normal(0, 3, vocab).astype(np.float32)
        vals[base + 10:base + 50] = vals[base:].max()     # exact ties at the top
        lb = ctx.upload(vals)
        bufs.append(lb)
        want.append(ctx.topk(lb, base, vocab, m, pen, serial=11).read(np.uint32))
    outs = [ctx.alloc(eff.lib().eff_topk_out_bytes()) for _ in cases]
    for (vocab, m, pen, base), lb, out in zip(cases, bufs, outs):
        ctx.topk_noalloc(lb, base, vocab, m, pen, serial=11, out=out)
    for (vocab, m, pen, base), out, w in zip(cases, outs, want):
        got = out.read(np.uint32)
        assert np.array_equal(got, w), (vocab, m)
        r = eff.parse_topk(got)
        assert r["n"] == m and r["serial"] == 11 and r["flags"] == 0
    for b in bufs + outs:
        b.free()


def test_topk_noalloc_limit_and_not_applicable(ctx, eff):
    big = ctx.alloc(4 * (eff.TOPK_NOALLOC_MAX_VOCAB + 1))
    with pytest.raises(eff.EffError) as e:
        ctx.topk_noalloc(big, 0, eff.TOPK_NOALLOC_MAX_VOCAB + 1, 40)
    assert e.value.code == eff.E_BOUNDS and "262144" in str(e.value)
    with pytest.raises(eff.NotApplicable):
        ctx.topk_noalloc(big, 0, 1000, eff.TOPK_M_MAX + 1)
    out = ctx.topk_noalloc(big, 0, eff.TOPK_NOALLOC_MAX_VOCAB, 5)    # exactly at the limit
    assert eff.parse_topk(out.read(np.uint32))["n"] == 5
    big.free()
    out.free()
