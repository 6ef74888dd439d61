"""The load path on the GPU: the chunked Q8_0R upload (eff_buf_write_r, one
chunk of subeReordenadoPorTrozos, repack.js:318-345) against the whole-tensor
repack, and the JavaScript loader (cargaTensores over a tensor table, the
upload of model.js:141-330) checked byte for byte against the file it read."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_write_r_chunks_match_whole_repack(eff, orc, ctx):
    rows, k = 13, 2464
    n = rows * k // 32                                   # 1001 blocks, odd
    w = eff.quantize("Q8_0", eff.fill_normal(7, 0.02, rows * k))
    whole = eff.repack(w, n)
    buf = ctx.alloc(eff.bytes_buffer_r(n))
    buf.mark_r(n)
    # odd and even chunk sizes, written out of order
    cuts, b0, sizes = [], 0, [1, 2, 7, 64, 3, 300, 5]
    while b0 < n:
        nb = min(sizes[len(cuts) % len(sizes)], n - b0)
        cuts.append((b0, nb))
        b0 += nb
    for b0, nb in cuts[1::2] + cuts[0::2]:
        buf.write_r(b0, w[34 * b0:34 * (b0 + nb)])
    got = buf.read()
    assert np.array_equal(got[:34 * n], whole[:34 * n])
    assert not got[34 * n:].any()
    assert buf.blocks_r() == n
    x = eff.fill_normal(8, 1.0, k)
    xb, yb = ctx.upload(x), ctx.alloc(rows * 4)
    ctx.qmatmul("Q8_0R", buf, xb, yb, rows, k, 1)
    check_close(yb.read(np.float32), orc.gemv_f64(orc.NAMES["Q8_0"], w, rows, k, x, 1), "Q8_0R after chunked upload")
    # an empty chunk is a no-op; a chunk past the tensor, a buffer without the
    # mark and a type that is not repacked are errors
    buf.write_r(n, w[:0])
    with pytest.raises(eff.EffError) as e:
        buf.write_r(n - 1, w[:68])
    assert e.value.code == eff.E_BOUNDS
    plain = ctx.alloc(eff.bytes_buffer_r(n))
    with pytest.raises(eff.EffError) as e:
        plain.write_r(0, w[:34])
    assert e.value.code == eff.E_MARK
    rc = eff.lib().eff_buf_write_r(ctx.h, buf.handle, eff.Q8_0, 0, w.ctypes.data, 1)
    assert rc == eff.E_TYPE
    for b in (buf, plain, xb, yb):
        b.free()


def _table(eff):
    """A tensor table over a synthetic file: spans broken by padding, tensors
    larger than a span (one of them an odd number of Q8_0 blocks), tiny float
    tensors whose size is not a multiple of 4."""
    spec = [("blk.0.attn_q.weight", "Q8_0", [256, 8]), ("blk.0.attn_norm.weight", "F32", [256]), None,
            ("blk.0.ffn_up.weight", "Q4_K", [512, 4]), ("blk.0.ffn_down.weight", "Q8_0", [352, 33]),
            ("output.weight", "Q6_K", [256, 40]), ("rope_freqs", "F16", [6]),
            ("token_embd.weight", "Q8_0", [64, 2])]
    pos, parts, table = 64, [np.full(64, 0x5A, np.uint8)], []
    for i, s in enumerate(spec):
        if s is None:                                    # 32 bytes of padding between two tensors
            parts.append(np.full(32, 0xAB, np.uint8))
            pos += 32
            continue
        name, t, dims = s
        ne = int(np.prod(dims))
        if t == "F32":
            raw = eff.fill_normal(40 + i, 1.0, ne).view(np.uint8)
        elif t == "F16":
            raw = eff.fill_normal(40 + i, 1.0, ne).astype(np.float16).view(np.uint8)
        else:
            raw = eff.quantize(t, eff.fill_normal(40 + i, 0.02, ne))
        table.append({"name": name, "typeName": t, "dims": dims, "nElements": ne, "nBytes": int(raw.size),
                      "start": pos})
        parts.append(raw)
        pos += raw.size
    return table, np.concatenate(parts)


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_loader_gpu(eff, orc, tmp_path):
    table, data = _table(eff)
    data.tofile(tmp_path / "model.bin")
    big = next(t for t in table if t["name"] == "blk.0.ffn_down.weight")
    rows, k = big["dims"][1], big["dims"][0]
    x = eff.fill_normal(3, 1.0, k)
    x.tofile(tmp_path / "x.bin")
    meta = {"file": "model.bin", "tensores": table, "tramo": 8192, "trozo": 1000,
            "gemv": {"name": big["name"], "rows": rows, "k": k, "x": "x.bin"}}
    (tmp_path / "meta.json").write_text(json.dumps(meta))
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_carga.js"), str(tmp_path)], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    out = json.loads((tmp_path / "out.json").read_text())
    total = sum(t["nBytes"] for t in table)
    want_y = orc.gemv_f64(orc.NAMES["Q8_0"], data[big["start"]:big["start"] + big["nBytes"]], rows, k, x, 1)
    for modo, reorden in (("plano", False), ("r", True)):
        o = out[modo]
        # spans: [attn_q, attn_norm], [ffn_up] (after padding), ffn_down and
        # output alone (larger than a span, read in chunks), [rope_freqs, token_embd]
        assert o["stats"]["tramos"] == 5
        assert o["stats"]["trozos"] == 3 + 13 + 9
        assert o["stats"]["reordenados"] == (3 if reorden else 0)
        assert o["stats"]["bytes"] == total
        us = [p[0] for p in o["prog"]]
        assert us == sorted(us) and o["prog"][-1] == [total, total, "token_embd.weight"]
        for t in table:
            raw = data[t["start"]:t["start"] + t["nBytes"]]
            got = np.fromfile(tmp_path / f"{modo}.{t['name']}.bin", np.uint8)
            d = o["tensores"][t["name"]]
            assert d["size"] == got.size
            if reorden and t["typeName"] == "Q8_0":
                n = t["nElements"] // 32
                assert d["typeName"] == "Q8_0R" and d["typeNameGGUF"] == "Q8_0" and d["bloquesR"] == n
                assert got.size == eff.bytes_buffer_r(n)
                assert np.array_equal(got[:34 * n], eff.repack(raw, n)[:34 * n]), t["name"]
                assert not got[34 * n:].any()
            else:
                assert d["typeName"] == t["typeName"] and d["typeNameGGUF"] is None and d["bloquesR"] is None
                assert got.size == (t["nBytes"] + 4 + 3) // 4 * 4     # 4 bytes of slack, zero
                assert np.array_equal(got[:t["nBytes"]], raw), t["name"]
                assert not got[t["nBytes"]:].any()
        check_close(np.array(o["gemv"], np.float32), want_y, f"loaded {big['name']} ({modo})")
