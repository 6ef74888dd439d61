"""Two host threads, each with its own context (its own stream and scratch
buffers), running products and top-ks at the same time: every output has the
bits of the same call made alone. The calls go through ctypes, which releases
the interpreter lock, so the library's shared state (the per-device kernel
attributes) is reached from both threads at once, and each context's own
scratch (the split-x x parts, the GEMM's fp16 x, the top-k records, and the
head's records written by the row GEMV) is used concurrently with the other
context's. The no-alloc top-k is left out: its fixed scratch is shared by every
context of a GPU, and calls that overlap race by design."""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (type, rows, k, tokens): the int8 matrix-core GEMV, the token-group GEMV (k
# not a multiple of 256), the split-x product, the Q8_0 GEMM and the Q6_K row GEMV
CASES = [("Q4_K", 300, 2048, 1), ("Q8_0", 520, 544, 20), ("Q2_K", 256, 1024, 16),
         ("Q8_0", 600, 544, 300), ("Q6_K", 32800, 512, 1)]


def run_cases(eff, ctx, inputs, rounds):
    outs = []
    bufs = []
    for (tname, rows, k, tokens), (w, x) in zip(CASES, inputs):
        wb, xb, yb = ctx.upload(w), ctx.upload(x), ctx.alloc(tokens * rows * 4)
        bufs.append((wb, xb, yb))
    for _ in range(rounds):
        for (tname, rows, k, tokens), (wb, xb, yb) in zip(CASES, bufs):
            ctx.qmatmul(eff.TYPES[tname], wb, xb, yb, rows, k, tokens)
        outs.append([yb.read(np.uint32) for _, _, yb in bufs])
        lb = bufs[-1][2]
        outs[-1].append(ctx.topk(lb, 0, CASES[-1][1], 40, [5], serial=3).read(np.uint32))
        # the decode head: the row GEMV writing its records into this context's scratch, then the selection
        wb, xb, _ = bufs[-1]
        yh = ctx.alloc(CASES[-1][1] * 4)
        rec = ctx.qgemv_topk(eff.TYPES["Q6_K"], wb, xb, yh, CASES[-1][1], CASES[-1][2], 40, [5], serial=3)
        outs[-1].append(rec.read(np.uint32))
        outs[-1].append(yh.read(np.uint32))
        rec.free()
        yh.free()
    for b in bufs:
        for x in b:
            x.free()
    return outs


def test_two_threads_two_contexts_same_bits(eff):
    inputs = []
    for i, (tname, rows, k, tokens) in enumerate(CASES):
        w = eff.quantize(tname, eff.fill_normal(900 + i, 0.02, rows * k))
        inputs.append((w, eff.fill_normal(950 + i, 1.0, tokens * k)))
    with eff.Context(0) as c:
        want = run_cases(eff, c, inputs, 1)[0]
    results, errors = [None, None], []

    def worker(slot):
        try:
            with eff.Context(0) as c:
                results[slot] = run_cases(eff, c, inputs, 6)
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for slot in range(2):
        for rnd, outs in enumerate(results[slot]):
            for case, (got, exp) in enumerate(zip(outs, want)):
                assert np.array_equal(got, exp), f"thread {slot} round {rnd} case {case}"
