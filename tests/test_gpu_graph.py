"""Recorded launches (eff_graph_*), the calls refused while recording, buffers
given back in stream order (eff_buf_retire) and read tickets that outlive
their context."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_graph_replays_give_the_eager_bits(ctx, eff):
    """A chain of products and a top-k recorded once replays with the bits of
    the same calls made eagerly, for each new x written between replays."""
    rows, k = 2048, 2048
    w4 = ctx.upload(eff.quantize("Q4_K", eff.fill_normal(31, 0.02, rows * k)))
    w6 = ctx.upload(eff.quantize("Q6_K", eff.fill_normal(32, 0.02, 40000 * k)))
    xin, y1, y2 = ctx.alloc(k * 4), ctx.alloc(rows * 4), ctx.alloc(rows * 4)
    logits, out = ctx.alloc(40000 * 4), ctx.alloc(eff.lib().eff_topk_out_bytes())
    xs = [eff.fill_normal(40 + i, 1.0, k) for i in range(3)]

    def chain():
        ctx.qmatmul(eff.Q4_K, w4, xin, y1, rows, k, 1)
        ctx.qmatmul(eff.Q4_K, w4, y1, y2, rows, k, 1)
        ctx.qgemv_topk(eff.Q6_K, w6, y2, logits, 40000, k, 40, [7], serial=9, out=out)

    eager = []
    for x in xs:
        xin.write(x)
        chain()
        eager.append((y2.read(np.uint32), logits.read(np.uint32), out.read(np.uint32)))
    ctx.graph_begin()
    chain()
    g = ctx.graph_end()
    assert g.nodes >= 4
    for rnd in range(2):
        for x, want in zip(xs, eager):
            xin.write(np.zeros(k, np.float32))
            xin.write(x)
            g.launch()
            got = (y2.read(np.uint32), logits.read(np.uint32), out.read(np.uint32))
            for a, b in zip(got, want):
                assert np.array_equal(a, b), rnd
    g.destroy()
    for b in (w4, w6, xin, y1, y2, logits, out):
        b.free()


def test_calls_refused_while_recording(eff):
    """Waits, allocations, host copies and scratch growth are refused while
    recording (EFF_E_INVALID) and leave the recording usable. A context of
    its own, so that its split-x scratch holds exactly 16 tokens."""
    with eff.Context(0) as ctx:
        _refused_while_recording(ctx, eff)


def _refused_while_recording(ctx, eff):
    rows, k = 256, 1024
    w = ctx.upload(eff.quantize("Q2_K", eff.fill_normal(51, 0.02, rows * k)))
    x = ctx.upload(eff.fill_normal(52, 1.0, 64 * k))
    y, y_ref = ctx.alloc(64 * rows * 4), ctx.alloc(64 * rows * 4)
    ctx.qmatmul(eff.Q2_K, w, x, y_ref, rows, k, 16)    # grows the split-x scratch for 16 tokens
    ctx.graph_begin()
    calls = {"alloc": lambda: ctx.alloc(64), "write": lambda: y.write(np.zeros(4, np.float32)),
             "read": lambda: y.read(np.uint32, 4), "sync": lambda: ctx.sync(),
             "readback": lambda: ctx.read_async(y, np.uint32, 4), "retire": lambda: w.retire(),
             "free": lambda: y_ref.free(),
             "grow": lambda: ctx.qmatmul(eff.Q2_K, w, x, y, rows, k, 64)}   # 64 tokens: the scratch would grow
    for name, call in calls.items():
        with pytest.raises(eff.EffError) as e:
            call()
        assert e.value.code == eff.E_INVALID, name
    ctx.qmatmul(eff.Q2_K, w, x, y, rows, k, 16)
    g = ctx.graph_end()
    g.launch()
    assert np.array_equal(y.read(np.uint32, 16 * rows), y_ref.read(np.uint32, 16 * rows))
    g.destroy()
    with pytest.raises(eff.EffError):
        ctx.graph_end()                                   # no recording open
    for b in (w, x, y, y_ref):
        b.free()


def test_retire_is_stream_ordered(ctx, eff):
    """A weight buffer given back right after a product is enqueued, and a new
    buffer of the same size filled with other weights at once: the product
    still reads the first weights."""
    rows, k = 8192, 2048
    wa = eff.quantize("Q8_0", eff.fill_normal(61, 0.02, rows * k))
    wb_ = eff.quantize("Q8_0", eff.fill_normal(62, 0.02, rows * k))
    x = ctx.upload(eff.fill_normal(63, 1.0, 512 * k))
    y, y2 = ctx.alloc(512 * rows * 4), ctx.alloc(512 * rows * 4)
    w = ctx.upload(wa)
    ctx.qmatmul(eff.Q8_0, w, x, y2, rows, k, 512)
    want = y2.read(np.uint32)
    ctx.sync()
    for _ in range(4):
        ctx.qmatmul(eff.Q8_0, w, x, y, rows, k, 512)
    w.retire()
    w2 = ctx.alloc(wa.nbytes)
    w2.write(wb_[:1 << 20])                                # staged, not waited for
    assert np.array_equal(y.read(np.uint32), want)
    for b in (x, y, y2, w2):
        b.free()


def test_read_ticket_outlives_its_context(eff):
    """A readback begun before eff_shutdown can be ended and released after it."""
    c = eff.Context(0)
    data = np.arange(1 << 16, dtype=np.uint32)
    b = c.upload(data)
    finish = c.read_async(b, np.uint32)
    finish2 = c.read_async(b, np.uint32, 16, offset=64)
    b.free()
    c.close()
    assert np.array_equal(finish(), data)
    assert np.array_equal(finish2(), data[16:32])


def test_read_poll_then_end(ctx, eff):
    """eff_read_poll answers without waiting (0 while the copy is in flight,
    1 once it has completed) and eff_read_end then gives the bytes."""
    import ctypes
    data = np.arange(1 << 20, dtype=np.uint32)
    b = ctx.upload(data)
    r = ctypes.c_void_p()
    ctx._check(eff.lib().eff_read_begin(ctx.h, b.handle, 0, data.nbytes, ctypes.byref(r)))
    seen = set()
    while True:
        rc = eff.lib().eff_read_poll(r)
        assert rc in (0, 1), rc
        seen.add(rc)
        if rc == 1:
            break
    assert 1 in seen
    out = np.empty_like(data)
    assert eff.lib().eff_read_end(r, out.ctypes.data) == 0
    assert eff.lib().eff_read_release(r) == 0
    assert np.array_equal(out, data)
    b.free()
