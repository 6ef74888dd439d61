"""Benchmark of the quantized matrix-product path on one MI355X.

Headline (`value`): BASELINE.json configs[1], Q4_K GEMV N=2048 x K=8192, M=1,
as algorithmic HBM GB/s = (weight block bytes + x bytes + y bytes) / time per
step. A step is one GEMV over one batch. Inputs are resident in HBM before the
timed region; each step reads a different copy of W (copies rotate over more
than 1 GiB, four times the 256 MB MALL), so no step is served by cache. The
timed steps are replayed from a HIP graph (torch.cuda.CUDAGraph over the
library's launches on torch's stream) and bracketed with HIP events on that
stream.

Also reported: the roofline fraction of the GEMV kernel, the reference CPU
path timed on this host (oracle restatement, cpu_baseline), and a sweep of
every BASELINE.json configuration (GB/s or TFLOP/s and roofline fraction).
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
METRIC = "Q-GEMV HBM GB/s and Q-GEMM TFLOPS, % of MI355X roofline, per quant type"


def alg_bytes(eff, tname, rows, k, tokens):
    base = "Q8_0" if tname == "Q8_0R" else tname
    e, b = eff.geometry(base)
    grid = 2048 if tname == "IQ2_XXS" else 0
    return rows * (k // e) * b + 4 * tokens * k + 4 * tokens * rows + grid


class Config:
    def __init__(self, eff, ctx, tname, rows, k, tokens, seed, topk=0):
        self.tname, self.rows, self.k, self.tokens, self.topk = tname, rows, k, tokens, topk
        base = "Q8_0" if tname == "Q8_0R" else tname
        self.t = eff.TYPES[tname]
        w = eff.quantize(base, eff.fill_normal(seed, 0.02, rows * k))
        e, _ = eff.geometry(base)
        n = rows * k // e
        data = eff.repack(w, n) if tname == "Q8_0R" else w
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
        ctx.qmatmul(self.t, self.w[i % self.copies], self.x, self.y, self.rows, self.k, self.tokens)
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


def time_steps(torch, ctx, cfg, steps, warmup, warm_replays=1, timed=1):
    """Average ms per step over `steps` graph-replayed steps (after `warmup`
    eager steps and `warm_replays` untimed replays); with `timed` > 1 the
    median of that many timed replays."""
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    for i in range(warmup):
        cfg.step(ctx, i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        for i in range(steps):
            cfg.step(ctx, i)
    ctx.set_stream(stream.cuda_stream)
    for _ in range(warm_replays):    # untimed replays: first touch of the graph, and warm-up
        g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(timed):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    ms = sorted(times)[len(times) // 2]
    del g
    ctx.set_stream(None)
    return ms


def cpu_baseline(eff, orc, tname, rows, k, seconds):
    """The reference CPU path restated (oracle): Q8_0 via quantized activations
    and integer dots, other types via f32 dequantize-and-dot, pool of threads
    claiming row chunks. Threads: the reference policy min(8, cores/2)
    (cpu.js:107-113) and all cores."""
    base = "Q8_0" if tname == "Q8_0R" else tname
    w = eff.quantize(base, eff.fill_normal(7, 0.02, rows * k))
    x = eff.fill_normal(8, 1.0, k)
    cores = os.cpu_count() or 1
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    res = {}
    for label, threads in (("reference_policy", max(1, min(8, cores // 2))), ("all_cores", cores)):
        orc.cpu_matmul(orc.NAMES[base], w, rows, k, x, 1, threads)   # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            orc.cpu_matmul(orc.NAMES[base], w, rows, k, x, 1, threads)
            n += 1
            dt = time.perf_counter() - t0
            if dt >= seconds / 2:
                break
        res[label] = (threads, n, dt)
    bytes_ = alg_bytes(eff, tname, rows, k, 1)
    th, n, dt = res["reference_policy"]
    th2, n2, dt2 = res["all_cores"]
    kind_note = ("integer-dot path of cpu-kernels.js (Q8 activations), restated"
                 if base == "Q8_0" else
                 "f32 dequantize-and-dot restatement (the reference CPU path has no kernel for this type)")
    return {"value": round(bytes_ * n / dt / 1e9, 3), "unit": "GB/s", "cores": th, "kind": "port",
            "sample": f"{n} full {tname} GEMVs N={rows} K={k} M=1 in {dt:.1f} s with {th} threads; {kind_note}",
            "all_cores": {"value": round(bytes_ * n2 / dt2 / 1e9, 3), "cores": th2}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--only", default="", help="run only sweep entries whose name contains this text")
    ap.add_argument("--no-head", action="store_true", help="skip the headline measurement")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run 5 device-to-device copies of MIB MiB (calibration of the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path is single-GPU by design (got --gpus {args.gpus}); "
              "the sharding design is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch

    eff = ge.package()
    ctx = eff.Context(0)
    torch.cuda.init()

    # Headline: configs[1]
    ms, gbs = float("nan"), float("nan")
    if not args.no_head:
        head = Config(eff, ctx, "Q4_K", 2048, 8192, 1, 202)
        # W eager warm-up steps and three untimed replays of the K captured steps, then one timed replay
        ms = time_steps(torch, ctx, head, args.steps, args.warmup, warm_replays=3)
        gbs = head.bytes / (ms * 1e-3) / 1e9
        head.free()

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
            traffic = json.load(f).get("q4_k_gemv_2048x8192", {}).get("hbm_bytes_per_dispatch")

    sweep = {}
    if not args.no_sweep:
        plan = [("C1", "Q8_0", 8192, 2048, 1, 0), ("C1", "Q8_0R", 8192, 2048, 1, 0),
                ("C2", "Q4_K", 2048, 8192, 1, 0),
                ("C3", "Q8_0", 8192, 2048, 512, 0), ("C3", "Q8_0", 8192, 2048, 2048, 0),
                ("C4", "Q6_K", 65536, 2048, 1, 0), ("C4+top40", "Q6_K", 65536, 2048, 1, 40)]
        for tn in ("Q2_K", "IQ2_XXS"):
            for m in (1, 8, 32, 128):
                plan.append(("C5", tn, 8192, 2048, m, 0))
        for tag, tn, rows, k, m, tk in plan:
            key = f"{tag} {tn} N={rows} K={k} M={m}" + (" +top40" if tk else "")
            if args.only and args.only not in key:
                continue
            cfg = Config(eff, ctx, tn, rows, k, m, 300 + rows + m, topk=tk)
            # the router's choice for this shape, from its launch counters
            before = ctx.stats()
            cfg.step(ctx, 0)
            after = ctx.stats()
            groups = after["skinny"] - before["skinny"]
            path = "gemm" if after["gemm"] > before["gemm"] else (
                "split-x" if after["split"] > before["split"] else (
                    f"gemv x {groups} token groups" if groups else "gemv"))
            steps = 40 if cfg.gemm else 100
            # steady state: the first replays over the >= 1 GiB weight rotation run slower
            t_ms = time_steps(torch, ctx, cfg, steps, 5, warm_replays=3, timed=3)
            gb = cfg.bytes / (t_ms * 1e-3) / 1e9
            tf = cfg.flops / (t_ms * 1e-3) / 1e12
            hbm_t = cfg.bytes / (HBM_PEAK_GBS * 1e9)
            mfma_t = cfg.flops / (FP16_PEAK_TFLOPS * 1e12)
            bound = "mfma" if mfma_t > hbm_t else "hbm"
            sweep[key] = {"us": round(t_ms * 1e3, 2), "GB/s": round(gb, 1), "TFLOP/s": round(tf, 2),
                          "bound": bound,
                          "roofline_frac": round((mfma_t if bound == "mfma" else hbm_t) / (t_ms * 1e-3), 4),
                          "path": path}
            cfg.free()
            print(f"# {key}: {sweep[key]}", file=sys.stderr, flush=True)

    # F1: the fused decode GEMV against the one-matrix GEMVs it replaces
    if not args.no_sweep:
        fplan = [("F1 gate+up", "Q4_K", [8192, 8192], 2048, eff.GEMV_SWIGLU),
                 ("F1 sections q+k+v", "Q4_K", [2048, 512, 512], 2048, eff.GEMV_SECTIONS)]
        for tag, tn, rl, k, mode in fplan:
            key = f"{tag} {tn} rows={'+'.join(map(str, rl))} K={k} M=1"
            if args.only and args.only not in key:
                continue
            res = {}
            for fused in (True, False):
                cfg = FusedConfig(eff, ctx, tn, rl, k, mode, 900 + len(rl), fused)
                t_ms = time_steps(torch, ctx, cfg, 100, 5, warm_replays=3, timed=3)
                res["fused" if fused else "separate"] = t_ms
                nbytes = cfg.bytes
                cfg.free()
            sweep[key] = {"us": round(res["fused"] * 1e3, 2), "separate_us": round(res["separate"] * 1e3, 2),
                          "GB/s": round(nbytes / (res["fused"] * 1e-3) / 1e9, 1), "bound": "hbm",
                          "roofline_frac": round(nbytes / (HBM_PEAK_GBS * 1e9) / (res["fused"] * 1e-3), 4),
                          "path": "fused gemv"}
            print(f"# {key}: {sweep[key]}", file=sys.stderr, flush=True)

    base = None
    if not args.no_cpu:
        orc = ge.oracle()
        base = cpu_baseline(eff, orc, "Q4_K", 2048, 8192, args.cpu_seconds)

    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (weights N(0,0.02) quantized to Q4_K, x N(0,1), fixed seeds)",
        "config": {"workload": "configs[1]: Q4_K GEMV N=2048 x K=8192, M=1 (decode)", "rows": 2048, "k": 8192,
                   "tokens": 1, "weight_copies_rotated": ">= 1 GiB"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "cpu_baseline": base,
        "sweep": sweep,
    }
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
