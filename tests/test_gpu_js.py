"""The JavaScript host on the GPU: tests/js/shim_gpu.js drives createQuantOps,
gemv, gemm2, dequant, the Q8_0R marks and createTopKGPU through the N-API
addon; its outputs are checked here against the oracle."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_shim_gpu(eff, orc, tmp_path):
    cases = []
    spec = [("q4k_t1", "Q4_K", 96, 2048, 1), ("q8r_t3", "Q8_0R", 64, 1024, 3), ("q6k_t2", "Q6_K", 40, 512, 2),
            ("iq2_t9", "IQ2_XXS", 48, 512, 9), ("q2k_t64", "Q2_K", 64, 512, 64), ("q6k_t64", "Q6_K", 48, 512, 64),
            ("q8_t100", "Q8_0", 64, 512, 100), ("q8_t300", "Q8_0", 80, 512, 300), ("q8r_t70", "Q8_0R", 32, 256, 70)]
    data = {}
    for i, (name, t, rows, k, tokens) in enumerate(spec):
        base = "Q8_0" if t == "Q8_0R" else t
        w = eff.quantize(base, eff.fill_normal(70 + i, 0.02, rows * k))
        x = eff.fill_normal(80 + i, 1.0, tokens * k)
        w.tofile(tmp_path / f"{name}.w")
        x.tofile(tmp_path / f"{name}.x")
        data[name] = (base, w, x, rows, k, tokens)
        cases.append({"name": name, "type": t, "rows": rows, "k": k, "tokens": tokens,
                      "w": f"{name}.w", "x": f"{name}.x"})
    logits = eff.fill_normal(99, 3.0, 70000)
    logits[100:140] = 2.5
    logits.tofile(tmp_path / "logits.bin")
    meta = {"cases": cases, "topk": {"logits": "logits.bin", "m": 40, "S": [5, 69999]}}
    (tmp_path / "meta.json").write_text(json.dumps(meta))
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_gpu.js"), str(tmp_path)], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    out = json.loads((tmp_path / "out.json").read_text())
    for name, (base, w, x, rows, k, tokens) in data.items():
        ot = orc.NAMES[base]
        # matmul: f32-accurate below 64 tokens and for every type but Q8_0 at any M; the fp16 GEMM
        # (the reference's DRIFT/GEMM2 rounding) for Q8_0 and Q8_0R from 64 tokens
        f32 = tokens < 64 or base != "Q8_0"
        ref = (orc.gemv_f64 if f32 else orc.gemm_f16)(ot, w, rows, k, x, tokens)
        check_close(np.array(out[name], np.float32), ref, f"js matmul {name}")
        if tokens <= 8:
            check_close(np.array(out[name + ":gemv"], np.float32), ref, f"js gemv {name}")
        if tokens <= 3:
            yg = np.array(out[name + ":gemv"], np.float32)
            assert np.array_equal(np.array(out[name + ":sec0"], np.float32).view(np.uint32), yg.view(np.uint32))
            assert np.array_equal(np.array(out[name + ":sec1"], np.float32).view(np.uint32), yg.view(np.uint32))
            want = (yg / (np.float32(1) + np.exp(-yg))) * yg
            assert np.allclose(np.array(out[name + ":gateup"], np.float32), want, rtol=4e-6, atol=0)
        if tokens >= 64 and base == "Q8_0":
            check_close(np.array(out[name + ":gemm2"], np.float32), orc.gemm_f16(ot, w, rows, k, x, tokens),
                        f"js gemm2 {name}")
            assert out[name + ":cola"] is True
        e, _ = eff.geometry(base)
        table = orc.dequant(ot, w, rows * k // e)
        assert np.array_equal(np.array(out[name + ":dequant"], np.uint32), table.view(np.uint32))
        sel = table.reshape(rows, k)[[0, rows - 1, 1]]
        assert np.array_equal(np.array(out[name + ":gather"], np.uint32).reshape(3, k), sel.view(np.uint32))
        if name + ":gnx" in out:
            assert np.array_equal(np.array(out[name + ":gnx"], np.uint32).reshape(3, k), sel.view(np.uint32))
            s64 = sel.astype(np.float64)
            want = s64 / np.sqrt((s64 * s64).sum(axis=1, keepdims=True) / k + 1e-6) * 1.5
            got = np.array(out[name + ":gnn"], np.float64).reshape(3, k)
            assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 2e-6
    ids, bits, _ = orc.topk(logits.view(np.uint32), 40)
    assert out["topk"]["ids"] == ids.tolist() and out["topk"]["bits"] == bits.tolist()
    assert out["topk"]["bitsS"] == logits.view(np.uint32)[[5, 69999]].tolist()
    # sample() over the device candidates gives the token of sample() over the whole vector
    assert len(out["muestrea"]) == 20
    for i, m in enumerate(out["muestrea"]):
        assert m["got"] is not None and m["got"] == m["want"], (i, m)
    assert out["topkStats"]["gpu"] == 20 and out["topkStats"]["respaldo"] == 1
    assert out["topkStats"]["motivos"] == {"muestreo sin tope": 1}
    assert out["stats"]["topk"] == 21 and out["stats"]["gemm"] >= 1 and out["stats"]["split"] >= 2
    assert out["cabeza"] is True   # the head GEMV + top-k in one call, checked inside the shim


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_graph_pool_and_gemv2_applicability(eff, orc):
    """tests/js/shim_grafo.js: gemv ops are null where GEMV2 is (and lend
    nothing), gemm2 converts x once per allocation mark (olvida() clears
    it), quant.matmul prepares the split-x product's x once per layout for the
    products of one x, quant.matmulCPU gives the CPU path's bits, recycle() destroys an expired size class without waiting for the
    device, and a recorded chain of 30 quant.matmul calls replays bit-equal to
    the eager chain for each new x (the checks of bits are inside the shim)."""
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_grafo.js")], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["gemv2"] is True
    # gemm2's aF16 memo: q and k of one x share one conversion; olvida(), a new mark, no mark: one each
    assert out["memo"] == {"q_k_shared": 1, "after_olvida": 1, "new_mark": 1, "no_mark": 2}, out["memo"]
    # quant.matmul at 33 tokens: Q4_K (twice), Q6_K and IQ2_XXS of one x prepare it twice (two layouts)
    assert out["memoSplit"] == {"shared": 2, "after_olvida": 1, "no_mark": 4}, out["memoSplit"]
    # quant.matmulCPU: the CPU path's bits (Q8_0, 96 x 512, 3 tokens), null for Q4_K
    mc = out["matmulCPU"]
    assert mc["q4k_null"] is True
    w = eff.quantize("Q8_0", eff.fill_normal(41, 0.02, 96 * 512))
    ref = orc.cpu_matmul(orc.Q8_0, w, 96, 512, eff.fill_normal(43, 1.0, 3 * 512), 3, 2)
    assert mc["y"] == ref.view(np.uint32).reshape(-1).tolist()
    rc = out["recycle"]
    # 60 GEMMs of 2048 x 8192 x 2048 were still running when recycle() returned
    assert rc["drain_us"] > 2000, rc
    assert rc["recycle_us"] < 0.1 * rc["drain_us"], rc
    g = out["grafo"]
    assert g["us_per_op_graph"] < g["us_per_op_eager"], g
