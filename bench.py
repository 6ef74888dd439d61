"""Benchmark of the quantized matrix-product path on one MI355X.

Headline (`value`): BASELINE.json configs[3], the largest single-GPU
configuration: the Q6_K output-projection GEMV N=65536 x K=2048 (M=1) followed
by the exact top-40 over its logits, as algorithmic HBM GB/s = (weight block
bytes + x bytes + logits bytes) / time per step. A step is one head GEMV plus
one top-k over one batch. Inputs are resident in HBM before the timed region.

Weight rotation: every configuration keeps C distinct copies of W totalling
>= 1 GiB (four times the 256 MB MALL), step i reads copy i % C, and every
timed replay of the K captured steps is preceded by an untimed replay of the
steps that complete the cycle, so every copy is read again only after all C
copies (>= 1 GiB) have been streamed: no step is served by the MALL, whatever
K is. The timed steps are replayed from a HIP graph (torch.cuda.CUDAGraph over
the library's launches on torch's stream) and bracketed with HIP events on
that stream.

Also reported: the roofline fraction of the dominant kernel (the GEMV, timed
alone the same way), the reference CPU path timed on this host
(cpu_baseline: the oracle's restatement of cpu-kernels.js's Q8_0 integer path,
which runs the Q6_K head requantized to Q8_0), and a sweep of every
BASELINE.json configuration.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__ as ge  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP16_PEAK_TFLOPS = 2516.6      # MI355X dense fp16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
ROTATE_BYTES = 1 << 30         # distinct weight bytes cycled through per config
MALL_BYTES = 256 << 20         # MI355X Infinity Cache
METRIC = "Q-GEMV HBM GB/s and Q-GEMM TFLOPS, % of MI355X roofline, per quant type"


def alg_bytes(eff, tname, rows, k, tokens):
    base = "Q8_0" if tname == "Q8_0R" else tname
    e, b = eff.geometry(base)
    grid = 2048 if tname == "IQ2_XXS" else 0
    return rows * (k // e) * b + 4 * tokens * k + 4 * tokens * rows + grid


class Config:
    def __init__(self, eff, ctx, tname, rows, k, tokens, seed, topk=0, fused_head=True, cpu_path=False):
        self.tname, self.rows, self.k, self.tokens, self.topk = tname, rows, k, tokens, topk
        self.cpu_path = cpu_path
        self.fused_head = fused_head and tokens == 1
        base = "Q8_0" if tname == "Q8_0R" else tname
        self.t = eff.TYPES[tname]
        w = eff.quantize(base, eff.fill_normal(seed, 0.02, rows * k))
        e, _ = eff.geometry(base)
        n = rows * k // e
        data = eff.repack(w, n) if tname == "Q8_0R" else w
        self.w_bytes = data.nbytes
        self.copies = max(2, min(256, ROTATE_BYTES // data.nbytes + 1))
        self.w = []
        first = ctx.upload(data)
        if tname == "Q8_0R":
            first.mark_r(n)
        self.w.append(first)
        for _ in range(self.copies - 1):
            b = ctx.alloc(data.nbytes)
            ctx.copy(b, first, data.nbytes)
            if tname == "Q8_0R":
                b.mark_r(n)
            self.w.append(b)
        self.x = ctx.upload(eff.fill_normal(seed + 1, 1.0, tokens * k))
        self.y = ctx.alloc(tokens * rows * 4)
        self.out = ctx.alloc(eff.lib().eff_topk_out_bytes()) if topk else None
        ctx.sync()
        self.bytes = alg_bytes(eff, tname, rows, k, tokens)
        self.flops = 2.0 * rows * k * tokens
        self.gemm = tokens >= 64

    def step(self, ctx, i):
        w = self.w[i % self.copies]
        if self.topk and self.fused_head:
            # the decode head: the GEMV and the top-k of its logits as one call
            ctx.qgemv_topk(self.t, w, self.x, self.y, self.rows, self.k, self.topk, (), i + 1, self.out)
            return
        if self.cpu_path:
            ctx.qmatmul_cpu_path(self.t, w, self.x, self.y, self.rows, self.k, self.tokens)
            return
        ctx.qmatmul(self.t, w, self.x, self.y, self.rows, self.k, self.tokens)
        if self.topk:
            ctx.topk(self.y, 0, self.rows, self.topk, (), i + 1, self.out)

    def free(self):
        for b in self.w + [self.x, self.y] + ([self.out] if self.out else []):
            b.free()


class FusedConfig:
    """Several matrices of one type sharing x, 1 token: the fused GEMV
    (gemv.gateUp / gemv.secciones) as one step, or the one-matrix GEMVs."""

    def __init__(self, eff, ctx, tname, rows_list, k, mode, seed, fused=True):
        self.eff, self.tname, self.rows, self.k, self.mode, self.fused = eff, tname, rows_list, k, mode, fused
        self.t = eff.TYPES[tname]
        self.sets = []
        data = [eff.quantize(tname, eff.fill_normal(seed + i, 0.02, r * k)) for i, r in enumerate(rows_list)]
        per = sum(d.nbytes for d in data)
        self.w_bytes = per
        self.copies = max(2, min(256, ROTATE_BYTES // per + 1))
        for _ in range(self.copies):
            self.sets.append([ctx.upload(d) for d in data])
        self.x = ctx.upload(eff.fill_normal(seed + 9, 1.0, k))
        nout = 1 if mode == eff.GEMV_SWIGLU else len(rows_list)
        self.ys = [ctx.alloc(rows_list[i] * 4) for i in range(nout)]
        self.yt = [ctx.alloc(r * 4) for r in rows_list]   # outputs of the one-matrix GEMVs
        ctx.sync()
        self.bytes = per + 4 * k + 4 * sum(rows_list[:nout])
        self.flops = 2.0 * k * sum(rows_list)
        self.gemm = False

    def step(self, ctx, i):
        ws = self.sets[i % self.copies]
        if self.fused:
            ctx.qgemv_multi(self.t, self.mode, ws, self.x, self.ys, self.rows, self.k, 1)
        else:
            for w, y, r in zip(ws, self.yt, self.rows):
                ctx.qgemv(self.t, w, self.x, y, r, self.k, 1)

    def free(self):
        for b in [b for st in self.sets for b in st] + [self.x] + self.ys + self.yt:
            b.free()


class SharedXConfig:
    """n products of one x (a layer's q, k and v): eff_qmatmul per product,
    each preparing x for the split-x product, or x prepared once
    (eff_qmatmul_prepare_x) and eff_qmatmul_prepared per product. The weight
    copies rotate over the products."""

    def __init__(self, eff, ctx, tname, rows, k, tokens, n, seed, shared):
        self.inner = Config(eff, ctx, tname, rows, k, tokens, seed)
        self.copies, self.w_bytes = self.inner.copies, self.inner.w_bytes
        self.n, self.shared, self.t = n, shared, self.inner.t
        self.rows, self.k, self.tokens = rows, k, tokens
        self.xp = ctx.alloc(ctx.qmatmul_x_layout(self.t, rows, k, tokens)[0])
        self.bytes = n * self.inner.bytes
        self.flops = n * self.inner.flops
        self.gemm = self.inner.gemm

    def step(self, ctx, i):
        c = self.inner
        if self.shared:
            ctx.qmatmul_prepare_x(self.t, c.x, self.xp, self.rows, self.k, self.tokens)
        for j in range(self.n):
            w = c.w[(i * self.n + j) % c.copies]
            if self.shared:
                ctx.qmatmul_prepared(self.t, w, self.xp, c.y, self.rows, self.k, self.tokens)
            else:
                ctx.qmatmul(self.t, w, c.x, c.y, self.rows, self.k, self.tokens)

    def free(self):
        self.inner.free()
        self.xp.free()


class ReadConfig:
    """A plain streaming read of a configuration's weight copies
    (eff_read_floor), rotated like its steps: the floor a GEMV's time is
    compared with, beside the HBM roofline."""

    def __init__(self, cfg, workgroups, unroll, sink):
        self.w, self.copies, self.w_bytes = cfg.w, cfg.copies, cfg.w_bytes
        self.workgroups, self.unroll, self.sink = workgroups, unroll, sink

    def step(self, ctx, i):
        ctx.read_floor(self.w[i % self.copies], self.w_bytes, self.workgroups, self.unroll, self.sink)


# grid shapes of the read (workgroups of 256 threads, 16-byte loads in flight per lane): the fastest of them per
# size in a sweep of 256-2048 workgroups x 1, 2, 4 loads
READ_SHAPES = ((2048, 1), (1024, 2), (1024, 4))


def read_floor_ms(torch, ctx, cfg, sink, steps):
    """The fastest read of cfg's weight bytes over READ_SHAPES, ms per step."""
    return min(time_steps(torch, ctx, ReadConfig(cfg, wg, un, sink), steps, 5, warm_replays=3, timed=3)
               for wg, un in READ_SHAPES)


def vendor_gemm_ms(torch, m, k, n, reps=50):
    """ms of torch.matmul on fp16 operands [m, k] x [k, n] (hipBLASLt on ROCm), replayed `reps` times in a
    graph, median of 5: the library's own speed on this box for a shape the quantized GEMM runs, measured
    only as a calibration (nothing of the quantized path uses it)."""
    a = torch.randn(m, k, device="cuda", dtype=torch.float16)
    b = torch.randn(k, n, device="cuda", dtype=torch.float16)
    for _ in range(5):
        c = a @ b
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            c = a @ b
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(5):
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        g.replay()
        s1.record()
        torch.cuda.synchronize()
        ts.append(s0.elapsed_time(s1) / reps)
    del g, a, b, c
    return sorted(ts)[2]


def rotation(cfg, steps):
    """What the timed steps of `cfg` read: copies, bytes, reuse distance."""
    per = cfg.w_bytes
    return {"copies": cfg.copies, "bytes_per_copy": per, "reuse_distance_bytes": cfg.copies * per,
            "distinct_bytes_in_timed_steps": min(steps, cfg.copies) * per}


def time_steps(torch, ctx, cfg, steps, warmup, warm_replays=1, timed=1, lead_ms=2.0):
    """Average ms per step over `steps` graph-replayed steps (after `warmup`
    eager steps and `warm_replays` untimed replays); with `timed` > 1 the
    median of that many timed replays.

    Every replay of the timed graph is preceded, without a wait, by an untimed
    lead-in graph of L steps: L = -steps (mod copies), so that every weight
    copy is reused only after all of them, and large enough that the lead-in
    keeps the GPU busy for at least `lead_ms` (L from the time per step of a
    warm replay). The host submits the lead-in, the start event, the timed
    graph and the end event while the GPU is still running the lead-in, so the
    timed region holds the K steps back to back and none of the host's
    submission (a fixed cost per graph launch, tens of microseconds), whatever
    K is."""
    rot = rotation(cfg, steps)
    assert rot["reuse_distance_bytes"] >= 2 * MALL_BYTES, rot
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    for i in range(warmup):
        cfg.step(ctx, i)
    torch.cuda.synchronize()

    def capture(first, n):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            for i in range(first, first + n):
                cfg.step(ctx, i)
        ctx.set_stream(stream.cuda_stream)
        return gr

    def events():
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    g = capture(0, steps)
    # one replay to size the lead-in (the first replay of a graph is not timed)
    g.replay()
    a, b = events()
    a.record(stream)
    g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    est = max(a.elapsed_time(b) / steps, 1e-4)
    lead = (-steps) % cfg.copies
    while lead == 0 or lead * est < lead_ms:
        lead += cfg.copies
    glead = capture(steps, lead)
    for _ in range(warm_replays):    # untimed replays: first touch of the lead-in graph, and warm-up
        glead.replay()
        g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(timed):
        glead.replay()
        start, end = events()
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    ms = sorted(times)[len(times) // 2]
    del g, glead
    ctx.set_stream(None)
    return ms


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def time_cpu(fn, seconds):
    """(runs, seconds) of fn() repeated for about `seconds` after one warm-up."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            return n, dt


def cpu_baseline(eff, orc, seconds, ctx=None):
    """The reference CPU path (cpu-kernels.js driven by cpu-trabajo.js) as the
    oracle restates it: x quantized to 8-bit blocks, integer dots against Q8_0
    blocks, a pool of threads claiming row chunks (cpu.js:140-216, 350-381).
    Threads: the reference policy min(8, cores/2) (cpu.js:107-113), and all
    cores of this process (at most 16, the box's share of one GPU).

    Headline leg (C4): the reference's CPU path has no Q6_K kernel and runs a
    tied Q6_K head requantized to Q8_0 at load (cpu.js:268-287), so one step is
    the 65536 x 2048 Q8_0 matvec over the requantized head plus the exact
    top-40 of its logits; `value` is the headline's algorithmic bytes per
    second of that step, so that it reads beside the GPU's `value`.
    Sweep legs: C1 (Q8_0 GEMV 8192 x 2048) and C3 M=512 (Q8_0 8192 x 2048 x 512)."""
    cores = host_cores()
    pol = max(1, min(8, cores // 2))
    allc = max(1, min(16, cores))
    rows, k = 65536, 2048
    q6 = eff.quantize("Q6_K", eff.fill_normal(404, 0.02, rows * k))
    head = orc.quantize_q8_0(orc.dequant(orc.Q6_K, q6, rows * k // 256))   # load-time requantization
    x = eff.fill_normal(405, 1.0, k)

    def head_step(threads):
        def f():
            y = orc.cpu_matmul(orc.Q8_0, head, rows, k, x, 1, threads)
            orc.topk(y.view(np.uint32).ravel(), 40)
        return f

    head_bytes = alg_bytes(eff, "Q6_K", rows, k, 1)
    n, dt = time_cpu(head_step(pol), seconds * 0.4)
    n2, dt2 = time_cpu(head_step(allc), seconds * 0.15)
    out = {"value": round(head_bytes * n / dt / 1e9, 3), "unit": "GB/s", "cores": pol, "kind": "port",
           "sample": (f"{n} steps of the C4 head on the reference CPU path in {dt:.1f} s with {pol} threads: "
                      f"65536x2048 Q8_0 matvec over the head requantized from Q6_K (cpu.js:268-287) with "
                      f"8-bit x blocks and integer dots (cpu.js:350-381), plus the exact top-40; value = the "
                      f"headline's {head_bytes} algorithmic bytes per step / step time; "
                      f"{1e3 * dt / n:.2f} ms per step"),
           "ms_per_step": round(1e3 * dt / n, 3),
           "all_cores": {"value": round(head_bytes * n2 / dt2 / 1e9, 3), "cores": allc,
                         "ms_per_step": round(1e3 * dt2 / n2, 3)},
           "cpu_model": cpu_model(), "host_cores": cores}
    sweep = {}
    for tag, r, kk, m, sec in (("C1 Q8_0 N=8192 K=2048 M=1", 8192, 2048, 1, seconds * 0.15),
                               ("C3 Q8_0 N=8192 K=2048 M=512", 8192, 2048, 512, seconds * 0.3)):
        w = eff.quantize("Q8_0", eff.fill_normal(7, 0.02, r * kk))
        xs = eff.fill_normal(8, 1.0, m * kk)
        n, dt = time_cpu(lambda: orc.cpu_matmul(orc.Q8_0, w, r, kk, xs, m, pol), sec)
        ms = 1e3 * dt / n
        e = {"ms": round(ms, 3), "threads": pol}
        if m == 1:
            e["GB/s"] = round(alg_bytes(eff, "Q8_0", r, kk, 1) / (ms * 1e-3) / 1e9, 3)
        else:
            e["TFLOP/s"] = round(2.0 * r * kk * m / (ms * 1e-3) / 1e12, 4)
        sweep[tag] = e
    out["sweep"] = sweep
    # the CPU path's arithmetic against the f64 product of the same bytes (C1): its 8-bit x blocks make this
    # gap by design (the GPU GEMVs keep 22 bits of each x group and sit near 1e-6)
    r, kk = 8192, 2048
    w = eff.quantize("Q8_0", eff.fill_normal(7, 0.02, r * kk))
    xs = eff.fill_normal(8, 1.0, kk)
    y = orc.cpu_matmul(orc.Q8_0, w, r, kk, xs, 1, pol)[0].astype(np.float64)
    ref = orc.gemv_f64(orc.Q8_0, w, r, kk, xs, 1)[0]
    nrm = float(np.linalg.norm(ref))
    out["gap_vs_f64"] = {"config": "C1 Q8_0 N=8192 K=2048 M=1", "rel_l2": float(np.linalg.norm(y - ref)) / nrm,
                         "max_abs_over_norm": float(np.max(np.abs(y - ref))) / nrm}
    if ctx is not None:
        # the GPU's product with the CPU path's arithmetic (eff_qmatmul_cpu_path) on the same bytes
        wb, xb, yb = ctx.upload(w), ctx.upload(xs), ctx.alloc(r * 4)
        ctx.qmatmul_cpu_path(eff.Q8_0, wb, xb, yb, r, kk, 1)
        g = yb.read(np.uint32, r)
        for b in (wb, xb, yb):
            b.free()
        yc = y.astype(np.float32).view(np.uint32)
        out["gpu_cpu_path"] = {"config": "C1 Q8_0 N=8192 K=2048 M=1", "outputs": int(r),
                               "bits_equal": bool(np.array_equal(g, yc)),
                               "what": "eff_qmatmul_cpu_path on the GPU against this restatement of the CPU path"}
    return out


def chain_kernel_us(torch, eff, ctx, ops=30, replays=50):
    """Time per operation of the js_chain's token (`ops` Q4_K 2048 x 2048
    GEMVs, each one's output the next one's input, one weight buffer) replayed
    from a HIP graph: the device time the chain's host cost is compared with."""
    rows = k = 2048
    w = ctx.upload(eff.quantize("Q4_K", eff.fill_normal(1, 0.02, rows * k)))
    xs = [ctx.upload(eff.fill_normal(2, 1.0, k))] + [ctx.alloc(rows * 4) for _ in range(ops)]
    ctx.sync()
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    for i in range(ops):
        ctx.qmatmul(eff.Q4_K, w, xs[i], xs[i + 1], rows, k, 1)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        for i in range(ops):
            ctx.qmatmul(eff.Q4_K, w, xs[i], xs[i + 1], rows, k, 1)
    ctx.set_stream(stream.cuda_stream)
    for _ in range(3):
        g.replay()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(replays):
        g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / (replays * ops)
    del g
    ctx.set_stream(None)
    for bf in [w] + xs:
        bf.free()
    return us


def js_chain():
    """Wall time per operation of a Node-driven decode chain through the N-API
    addon (elffuss-engine_amd/js/bench_cadena.js), or None without node."""
    import shutil
    import subprocess
    node = shutil.which("node")
    if not node:
        return None
    r = subprocess.run([node, os.path.join(ROOT, "elffuss-engine_amd", "js", "bench_cadena.js"), "200", "30"],
                       capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": (r.stderr or r.stdout)[-300:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-js", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--only", default="", help="run only sweep entries whose name contains this text")
    ap.add_argument("--no-head", action="store_true", help="skip the headline measurement")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run 5 device-to-device copies of MIB MiB (calibration of the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path is single-GPU by design (got --gpus {args.gpus}); "
              "how it would shard over several GPUs is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch

    eff = ge.package()
    ctx = eff.Context(0)
    torch.cuda.init()

    # Headline: configs[3], the Q6_K head GEMV + top-40 (the largest single-GPU configuration)
    rows, k = 65536, 2048
    ms = ms_gemv = gbs = gemv_gbs = float("nan")
    rot = floor = None
    sink = ctx.alloc(4 * 65536)
    if not args.no_head:
        head = Config(eff, ctx, "Q6_K", rows, k, 1, 404, topk=40)
        # W eager warm-up steps, three untimed replays of the K captured steps, then the median of five
        # timed replays, each behind >= 2 ms of queued lead-in steps
        ms = time_steps(torch, ctx, head, args.steps, args.warmup, warm_replays=3, timed=5)
        rot = rotation(head, args.steps)
        gbs = head.bytes / (ms * 1e-3) / 1e9
        # the dominant kernel alone (same weights and rotation): the GEMV's time per launch
        head.topk = 0
        ms_gemv = time_steps(torch, ctx, head, args.steps, args.warmup, warm_replays=3, timed=5)
        gemv_gbs = head.bytes / (ms_gemv * 1e-3) / 1e9
        # the same weight bytes read plainly, rotated the same way
        f_ms = read_floor_ms(torch, ctx, head, sink, args.steps)
        floor = {"us": round(f_ms * 1e3, 2), "GB/s": round(head.w_bytes / (f_ms * 1e-3) / 1e9, 1),
                 "gemv_frac_of_read": round(f_ms / ms_gemv, 4),
                 "what": "eff_read_floor: the weight bytes read with 16-byte loads, no compute, the fastest of "
                         + ", ".join(f"{w} x {u}" for w, u in READ_SHAPES) + " (workgroups x loads in flight)"}
        head.free()
        print(f"# headline: {ms * 1e3:.2f} us per step ({gbs:.1f} GB/s), GEMV alone {ms_gemv * 1e3:.2f} us",
              file=sys.stderr, flush=True)

    if args.copy_probe:
        nbytes = args.copy_probe << 20
        src, dst = ctx.alloc(nbytes), ctx.alloc(nbytes)
        for _ in range(5):
            ctx.copy(dst, src, nbytes)
        ctx.sync()
        src.free()
        dst.free()

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("q6_k_gemv_65536x2048", {}).get("hbm_bytes_per_dispatch")

    sweep = {}
    if not args.no_sweep:
        plan = [("C1", "Q8_0", 8192, 2048, 1, 0), ("C1", "Q8_0R", 8192, 2048, 1, 0),
                ("C2", "Q4_K", 2048, 8192, 1, 0),
                ("C3", "Q8_0", 8192, 2048, 512, 0), ("C3", "Q8_0", 8192, 2048, 2048, 0),
                ("C3", "Q8_0R", 8192, 2048, 512, 0),
                ("C4", "Q6_K", 65536, 2048, 1, 0), ("C4+top40", "Q6_K", 65536, 2048, 1, 40),
                ("C4+top40 separate", "Q6_K", 65536, 2048, 1, -40)]
        for tn in ("Q2_K", "IQ2_XXS"):
            for m in (1, 8, 32, 128):
                plan.append(("C5", tn, 8192, 2048, m, 0))
        # the FFN down projection (C2's 2048 x 8192) beyond one token: few rows, so the split-x product and
        # the GEMM cut k into slices over workgroups
        plan += [("C2-shape", "Q8_0", 2048, 8192, 8, 0), ("C2-shape", "Q4_K", 2048, 8192, 64, 0),
                 ("C2-shape", "Q8_0", 2048, 8192, 512, 0)]
        for tag, tn, r, kk, m, tk in plan:
            key = f"{tag} {tn} N={r} K={kk} M={m}" + (" +top40" if tk else "")
            if args.only and args.only not in key:
                continue
            # tk < 0: the GEMV and the top-k as two calls (eff_qmatmul, eff_topk)
            cfg = Config(eff, ctx, tn, r, kk, m, 300 + r + m, topk=abs(tk), fused_head=tk > 0)
            # the router's choice for this shape, from its launch counters
            before = ctx.stats()
            cfg.step(ctx, 0)
            after = ctx.stats()
            groups = after["skinny"] - before["skinny"]
            path = "gemm" if after["gemm"] > before["gemm"] else (
                "split-x" if after["split"] > before["split"] else (
                    f"gemv x {groups} token groups" if groups else "gemv"))
            steps = 40 if cfg.gemm else 100
            # steady state: the median of three timed replays after three untimed ones
            t_ms = time_steps(torch, ctx, cfg, steps, 5, warm_replays=3, timed=3)
            gb = cfg.bytes / (t_ms * 1e-3) / 1e9
            tf = cfg.flops / (t_ms * 1e-3) / 1e12
            hbm_t = cfg.bytes / (HBM_PEAK_GBS * 1e9)
            mfma_t = cfg.flops / (FP16_PEAK_TFLOPS * 1e12)
            bound = "mfma" if mfma_t > hbm_t else "hbm"
            sweep[key] = {"us": round(t_ms * 1e3, 2), "GB/s": round(gb, 1), "TFLOP/s": round(tf, 2),
                          "bound": bound,
                          "roofline_frac": round((mfma_t if bound == "mfma" else hbm_t) / (t_ms * 1e-3), 4),
                          "path": path + (" + top-k" if tk < 0 else " + fused top-k records" if tk else ""),
                          "reuse_distance_MB": round(rotation(cfg, steps)["reuse_distance_bytes"] / 1e6)}
            if bound == "hbm" and not tk:
                # a plain read of the same weight bytes (x and y not included), as a floor beside the roofline
                f_ms = read_floor_ms(torch, ctx, cfg, sink, steps)
                sweep[key]["read_floor_us"] = round(f_ms * 1e3, 2)
                sweep[key]["frac_of_read_floor"] = round(f_ms / t_ms, 4)
            if bound == "mfma":
                # the vendor's fp16 GEMM of the same shape (no dequantization, no x conversion), as a
                # calibration beside the roofline
                v_ms = vendor_gemm_ms(torch, m, kk, r)
                sweep[key]["vendor_fp16_gemm_us"] = round(v_ms * 1e3, 2)
                sweep[key]["frac_of_vendor"] = round(v_ms / t_ms, 4)
            cfg.free()
            print(f"# {key}: {sweep[key]}", file=sys.stderr, flush=True)

    # F1: the fused decode GEMV against the one-matrix GEMVs it replaces
    if not args.no_sweep:
        fplan = [("F1 gate+up", "Q4_K", [8192, 8192], 2048, eff.GEMV_SWIGLU),
                 ("F1 sections q+k+v", "Q4_K", [2048, 512, 512], 2048, eff.GEMV_SECTIONS)]
        for tag, tn, rl, kk, mode in fplan:
            key = f"{tag} {tn} rows={'+'.join(map(str, rl))} K={kk} M=1"
            if args.only and args.only not in key:
                continue
            res = {}
            for fused in (True, False):
                cfg = FusedConfig(eff, ctx, tn, rl, kk, mode, 900 + len(rl), fused)
                t_ms = time_steps(torch, ctx, cfg, 100, 5, warm_replays=3, timed=3)
                res["fused" if fused else "separate"] = t_ms
                nbytes = cfg.bytes
                cfg.free()
            sweep[key] = {"us": round(res["fused"] * 1e3, 2), "separate_us": round(res["separate"] * 1e3, 2),
                          "GB/s": round(nbytes / (res["fused"] * 1e-3) / 1e9, 1), "bound": "hbm",
                          "roofline_frac": round(nbytes / (HBM_PEAK_GBS * 1e9) / (res["fused"] * 1e-3), 4),
                          "path": "fused gemv"}
            print(f"# {key}: {sweep[key]}", file=sys.stderr, flush=True)

    # the CPU path's arithmetic on the GPU (eff_qmatmul_cpu_path): C1 and C3 M=512
    if not args.no_sweep:
        for m in (1, 512):
            key = f"CPU-path arithmetic Q8_0 N=8192 K=2048 M={m}"
            if args.only and args.only not in key:
                continue
            cfg = Config(eff, ctx, "Q8_0", 8192, 2048, m, 300 + 8192 + m, cpu_path=True)
            t_ms = time_steps(torch, ctx, cfg, 40 if m > 1 else 100, 5, warm_replays=3, timed=3)
            sweep[key] = {"us": round(t_ms * 1e3, 2), "GB/s": round(cfg.bytes / (t_ms * 1e-3) / 1e9, 1),
                          "TFLOP/s": round(cfg.flops / (t_ms * 1e-3) / 1e12, 2),
                          "path": "eff_qmatmul_cpu_path: 8-bit x blocks, int32 block dots, f32 terms in block order "
                                  "(the bits of the CPU path's restatement)"}
            cfg.free()
            print(f"# {key}: {sweep[key]}", file=sys.stderr, flush=True)

    # P1: the router's x prepared once for three products of one activation
    if not args.no_sweep:
        for tn, m in (("Q4_K", 32), ("Q2_K", 128)):
            key = f"P1 q+k+v shared x 3 x {tn} N=8192 K=2048 M={m}"
            if args.only and args.only not in key:
                continue
            res = {}
            for shared in (True, False):
                cfg = SharedXConfig(eff, ctx, tn, 8192, 2048, m, 3, 950 + m, shared)
                res[shared] = time_steps(torch, ctx, cfg, 40, 5, warm_replays=3, timed=3)
                nbytes, flops = cfg.bytes, cfg.flops
                cfg.free()
            sweep[key] = {"us": round(res[True] * 1e3, 2), "separate_us": round(res[False] * 1e3, 2),
                          "TFLOP/s": round(flops / (res[True] * 1e-3) / 1e12, 2),
                          "GB/s": round(nbytes / (res[True] * 1e-3) / 1e9, 1),
                          "path": "split-x, x prepared once (eff_qmatmul_prepare_x + 3 x eff_qmatmul_prepared)"}
            print(f"# {key}: {sweep[key]}", file=sys.stderr, flush=True)

    chain = None
    if not args.no_js and not args.only:
        chain = js_chain()
        if chain is not None and "error" not in chain:
            chain["kernel_us_per_op"] = round(chain_kernel_us(torch, eff, ctx), 3)
        print(f"# js chain: {chain}", file=sys.stderr, flush=True)

    base = None
    if not args.no_cpu:
        base = cpu_baseline(eff, ge.oracle(), args.cpu_seconds, ctx)

    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 dot products (v_dot4_i32_i8: Q6_K weights as int8, x as 3 int8 digit planes = 22 bits per "
                 "32-value group, exact int32 sums; f32 scales); top-k on u32 keys",
        "data": "synthetic (weights N(0,0.02) quantized to Q6_K, x N(0,1), fixed seeds)",
        "config": {"workload": "configs[3]: Q6_K output-projection GEMV N=65536 x K=2048, M=1, + exact top-40 "
                               "of the logits (decode head)",
                   "rows": rows, "k": k, "tokens": 1, "top_k": 40, "weight_rotation": rot,
                   "gemv_alone_ms_per_step": round(ms_gemv, 5)},
        "roofline": {"bound": "hbm", "kernel": "k_gemv_rows_q6k (Q6_K, 1 token)", "achieved": round(gemv_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "read_floor": floor,
        "cpu_baseline": base,
        "js_chain": chain,
        "sweep": sweep,
    }
    sink.free()
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
