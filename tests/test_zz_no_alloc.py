"""eff_topk_noalloc through the C ABI against eff_topk: the same record on two
calls in a row, the second over a smaller vocabulary (the fixed scratch still
holds the first call's candidates when it starts), with ties, a penalty list
and a base offset; a large vocabulary; and the calls it does not apply to."""
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


def test_topk_noalloc_large_vocab_and_not_applicable(ctx, eff):
    """The fixed scratch holds the records of every vocabulary the top-k
    accepts (below 2^24): 2^20 logits give eff_topk's record; past the
    limits it answers NOT_APPLICABLE as eff_topk does."""
    vocab = 1 << 20
    vals = np.random.default_rng(9).normal(0, 2, vocab).astype(np.float32)
    lb = ctx.upload(vals)
    want = ctx.topk(lb, 0, vocab, 100, [1, 2], serial=3).read(np.uint32)
    got = ctx.topk_noalloc(lb, 0, vocab, 100, [1, 2], serial=3).read(np.uint32)
    assert np.array_equal(got, want)
    with pytest.raises(eff.NotApplicable):
        ctx.topk_noalloc(lb, 0, 1000, eff.TOPK_M_MAX + 1)
    with pytest.raises(eff.NotApplicable):
        ctx.topk_noalloc(lb, 0, 1000, 40, penal_ids=list(range(eff.TOPK_P_MAX + 1)))
    lb.free()
