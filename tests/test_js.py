"""The JavaScript host (elffuss-engine_amd/js) on the CPU: runs tests/js/shim_cpu.js
under node (no device calls)."""
import json
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_shim_cpu(eff):
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_cpu.js")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "shim_cpu ok" in r.stdout


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_sampler_cpu(eff):
    """sample() against closed forms and its distributions; the candidate step
    against sample() over the whole vector (tests/js/shim_muestreo.js)."""
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_muestreo.js")], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "shim_muestreo ok" in r.stdout


def mulberry32(seed):
    """One step of Tommy Ettinger's published mulberry32 from state `seed`,
    as a double in [0, 1): z = seed + 0x6D2B79F5; z = (z ^ z >> 15) * (z | 1);
    z ^= z + (z ^ z >> 7) * (z | 61); (z ^ z >> 14) / 2^32, all mod 2^32."""
    m = 0xFFFFFFFF
    z = (seed + 0x6D2B79F5) & m
    z = ((z ^ (z >> 15)) * (z | 1)) & m
    z ^= (z + (((z ^ (z >> 7)) * (z | 61)) & m)) & m
    return ((z ^ (z >> 14)) & m) / 4294967296.0


def expected_token(logits, temperature, top_k, top_p, min_p, seed):
    """sample() without penalties (sample.js:78-153), stated independently:
    the top_k ids by (logit desc, id asc); top-p keeps the shortest prefix
    whose untempered probability reaches top_p; min-p keeps the prefix with
    weight >= min_p times the first; the draw u * S lands in the first
    cumulative tempered weight >= it."""
    l = np.asarray(logits, np.float32).astype(np.float64)
    order = sorted(range(l.size), key=lambda i: (-l[i], i))[:top_k]
    mx = l[order[0]]
    base = [math.exp(l[i] - mx) for i in order]
    total = math.fsum(base)
    cut = len(order)
    if top_p < 1:
        cum = np.cumsum(np.array(base) / total)
        cut = int(np.argmax(cum >= top_p)) + 1 if np.any(cum >= top_p) else len(order)
    if min_p > 0:
        j = 1
        while j < cut and base[j] >= min_p * base[0]:
            j += 1
        cut = j
    p = [math.exp((l[i] - mx) / temperature) for i in order[:cut]]
    target = mulberry32(seed) * math.fsum(p)
    cum = np.cumsum(p)
    hit = np.nonzero(cum >= target)[0]
    return order[int(hit[0]) if hit.size else cut - 1], target, cum


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_draws_pinned_by_mulberry32_and_softmax_cdf(eff, tmp_path):
    """uniforme() equals mulberry32 exactly, and sample()'s token equals the
    draw over the softmax CDF, on 400 random settings (cases whose draw lands
    within 1e-9 of a CDF step are skipped: the order of the f64 sums decides
    those)."""
    rng = np.random.default_rng(2024)
    seeds = [0, 1, 2, 3, 7, 42, 12345, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF] + \
        [int(v) for v in rng.integers(0, 2**32, 200)]
    cases, want = [], []
    for i in range(400):
        n = int(rng.integers(2, 300))
        logits = (rng.normal(0, rng.choice([0.5, 2.0, 6.0]), n)).astype(np.float32)
        if i % 5 == 0:
            logits[rng.integers(0, n, n // 3)] = logits[0]   # exact ties
        top_k = int(rng.integers(1, min(n, 60) + 1))
        opts = {"temperature": float(rng.choice([0.3, 0.8, 1.0, 1.7])), "topK": top_k,
                "topP": float(rng.choice([1.0, 0.9, 0.5])), "minP": float(rng.choice([0.0, 0.05, 0.2])),
                "seed": int(rng.integers(0, 2**31)), "repeatPenalty": 1}
        tok, target, cum = expected_token(logits, opts["temperature"], top_k, opts["topP"], opts["minP"], opts["seed"])
        if np.min(np.abs(cum - target)) < 1e-9 * max(cum[-1], 1e-300):
            continue
        cases.append({"logits": logits.tolist(), "opts": opts})
        want.append(tok)
    assert len(cases) > 380
    (tmp_path / "sorteo.json").write_text(json.dumps({"seeds": seeds, "cases": cases}))
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_sorteo.js"), str(tmp_path)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = json.loads((tmp_path / "sorteo_out.json").read_text())
    assert out["uniforme"] == [mulberry32(s) for s in seeds]
    assert out["tokens"] == want
