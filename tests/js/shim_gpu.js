'use strict';
// GPU run of the JavaScript host: reads a case written by tests/test_gpu_js.py,
// runs the operators through the addon exactly as the engine would call them,
// and writes the results back for the Python side to check against the oracle.
const assert = require('assert');
const fs = require('fs');
const path = require('path');
const eff = require(path.join(__dirname, '..', '..', 'elffuss-engine_amd', 'js', 'index.js'));

// A file of float32 values. readFileSync may return a view into a shared
// pool for small files, so the copy starts at the view's own offset.
function leeF32(file) {
  const b = fs.readFileSync(file);
  return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.length));
}

async function main() {
  const dir = process.argv[2];
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  const device = await eff.requestDevice();
  const ops = eff.createQuantOps(device);
  // the same context with quant.gemv widened to every type (and matmul to 8 tokens)
  const amp = eff.createQuantOps(device, { ctx: ops.ctx, gemvAmpliado: true });
  const out = {};
  const rd = async (buf, n) => new Float32Array(await eff.readback(device, buf, 0, n * 4));
  for (const c of meta.cases) {
    const w = fs.readFileSync(path.join(dir, c.w));
    const x = leeF32(path.join(dir, c.x));
    let wBuf;
    if (c.type === 'Q8_0R') {
      const n = c.rows * c.k / 32;
      wBuf = device.createBuffer({ size: eff.bytesBufferR('Q8_0R', n), label: 'w' });
      device.queue.writeBuffer(wBuf, 0, eff.reordena('Q8_0', w, n));
      assert.throws(() => eff.compruebaBufferR('Q8_0R', wBuf, {}, 'matmul'), /marca/);
      eff.marcaBufferR(wBuf, 'Q8_0R', n);
      assert.strictEqual(eff.bloquesR(wBuf), n);
    } else {
      wBuf = ops.upload(w, 'w');
    }
    const xBuf = ops.upload(x, 'x');
    const y = await ops.matmul(c.type, wBuf, xBuf, c.rows, c.k, c.tokens);
    out[c.name] = Array.from(await rd(y, c.rows * c.tokens));
    // quant.gemv applies where the reference's GEMV2 does (Q8_0, Q8_0R, Q6_K; 1-3 tokens)
    const gemv2 = eff.GEMV2_TIPOS.has(c.type) && c.tokens <= eff.GEMV2_MAX_TOKENS;
    if (c.tokens <= 3) {
      // the fused forms over the same matrix twice: silu(y) * y, and [y, y]
      const g = gemv2 ? ops.gemv : amp.gemv;
      const ysw = await g.gateUp(c.type, wBuf, wBuf, xBuf, c.rows, c.k, c.tokens);
      out[c.name + ':gateup'] = Array.from(await rd(ysw, c.rows * c.tokens));
      const ys = await g.secciones(c.type, [wBuf, wBuf], xBuf, [c.rows, c.rows], c.k, c.tokens);
      out[c.name + ':sec0'] = Array.from(await rd(ys[0], c.rows * c.tokens));
      out[c.name + ':sec1'] = Array.from(await rd(ys[1], c.rows * c.tokens));
      assert.strictEqual(await g.secciones(c.type, [wBuf], xBuf, [c.rows], c.k, c.tokens), null);
    }
    if (!gemv2) {
      assert.strictEqual(await ops.gemv.matmul(c.type, wBuf, xBuf, c.rows, c.k, c.tokens), null);
      assert.strictEqual(await ops.gemv.gateUp(c.type, wBuf, wBuf, xBuf, c.rows, c.k, c.tokens), null);
    }
    if (c.tokens <= 8) {
      const yg = await (gemv2 ? ops.gemv : amp.gemv).matmul(c.type, wBuf, xBuf, c.rows, c.k, c.tokens);
      out[c.name + ':gemv'] = Array.from(await rd(yg, c.rows * c.tokens));
    } else {
      assert.strictEqual(await amp.gemv.matmul(c.type, wBuf, xBuf, c.rows, c.k, c.tokens), null);
    }
    if (c.tokens >= 64) {
      const ym = await ops.gemm2.matmul(c.type, wBuf, xBuf, c.rows, c.k, c.tokens);
      if (eff.GEMM2_TIPOS.has(c.type)) {
        out[c.name + ':gemm2'] = Array.from(await rd(ym, c.rows * c.tokens));
        // the tail: the last token alone with the batch's plan gives its row's bits
        assert.ok(ops.gemm2.reproducible(c.type, c.rows, c.k, c.tokens));
        const x1 = ops.upload(x.subarray((c.tokens - 1) * c.k), 'x1');
        const yc = await ops.gemm2.cola(c.type, wBuf, x1, c.rows, c.k, c.tokens);
        const cola = new Uint32Array(await eff.readback(device, yc, 0, c.rows * 4));
        const ult = new Uint32Array(await eff.readback(device, ym, (c.tokens - 1) * c.rows * 4, c.rows * 4));
        assert.deepStrictEqual(Array.from(cola), Array.from(ult));
        out[c.name + ':cola'] = true;
      } else {
        assert.strictEqual(ym, null);
        assert.strictEqual(ops.gemm2.plan(c.type, c.rows, c.k, c.tokens), null);
        assert.strictEqual(ops.gemm2.reproducible(c.type, c.rows, c.k, c.tokens), false);
        assert.strictEqual(await ops.gemm2.cola(c.type, wBuf, xBuf, c.rows, c.k, c.tokens), null);
      }
    } else {
      assert.strictEqual(await ops.gemm2.matmul(c.type, wBuf, xBuf, c.rows, c.k, c.tokens), null);
    }
    // embedding rows 0, rows-1 and 1 of the same table, and the fused norm
    const ids = ops.upload(Uint32Array.from([0, c.rows - 1, 1]), 'ids');
    const ge = await ops.gather(c.type, wBuf, ids, c.k, 3);
    out[c.name + ':gather'] = Array.from(new Uint32Array(await eff.readback(device, ge, 0, 3 * c.k * 4)));
    if (eff.TIPOS_GATHER_NORMA.has(c.type)) {
      const wn = ops.upload(new Float32Array(c.k).fill(1.5), 'wn');
      const fus = eff.createFusionOps(device, { ctx: ops.ctx });
      const r = await fus.gatherNorma(c.type, wBuf, ids, wn, c.k, 3, 1e-6);
      out[c.name + ':gnx'] = Array.from(new Uint32Array(await eff.readback(device, r.x, 0, 3 * c.k * 4)));
      out[c.name + ':gnn'] = Array.from(await rd(r.nrm, 3 * c.k));
    } else {
      const fus = eff.createFusionOps(device, { ctx: ops.ctx });
      assert.throws(() => fus.gatherNorma(c.type, wBuf, ids, ids, c.k, 3, 1e-6), /lector/);
    }
    const nb = c.rows * c.k / eff.QUANT_TYPES[c.type].blockElems;
    const dq = await ops.dequant(c.type, wBuf, nb);
    out[c.name + ':dequant'] = Array.from(new Uint32Array(await eff.readback(device, dq, 0, nb * eff.QUANT_TYPES[c.type].blockElems * 4)));
    assert.throws(() => ops.matmul(c.type, wBuf, xBuf, c.rows, c.k + 1, 1), /múltiplo/);
    // the pool lends the same buffers again after the token, without new allocations
    const clases = ops.ctx.scratch.map((e) => e.size);
    const antes = new Set(ops.ctx.scratch.map((e) => e.buf));
    ops.ctx.recycle();
    for (const sz of clases) assert.ok(antes.has(ops.ctx.alloc(sz)));
    ops.ctx.recycle();
  }
  // top-k over a logits vector, candidates through createTopKGPU
  const logits = leeF32(path.join(dir, meta.topk.logits));
  const lb = ops.upload(logits, 'logits');
  const tk = eff.createTopKGPU(device, ops.ctx);
  const c = await tk.candidatos(lb, 0, logits.length, { M: meta.topk.m, S: Uint32Array.from(meta.topk.S) });
  out.topk = { ids: Array.from(c.ids), bits: Array.from(c.bits), bitsS: Array.from(c.bitsS) };
  // the whole step: plan, device candidates, sample() on the handful, against
  // sample() over the vector read back
  const todo = new Float32Array(await eff.readback(device, lb, 0, logits.length * 4));
  const ajustes = [
    [{}, [5, 69999, 120], [101, 101]],
    [{ repeatPenalty: 1 }, [], []],
    [{ temperature: 0.8, topK: 40, topP: 0.9, minP: 0.05, seed: 7 }, [100, 101, 102], [139]],
    [{ temperature: 1.3, topK: 150, seed: 12345, presence: 1.5, repeatLastN: 32 }, Array.from({ length: 40 }, (_, i) => 100 + i), [3]],
    [{ temperature: 0.5, topK: 1, seed: 3, repeatPenalty: 0.7 }, [100, -1, 70000], []],
  ];
  out.muestrea = [];
  for (const [opts, A, B] of ajustes) {
    for (let paso = 0; paso < 4; paso++) {
      const o = Object.assign({}, opts, { seed: (opts.seed || 1) + paso });
      const r = await tk.muestrea(lb, 0, logits.length, o, A, B);
      const want = eff.sample(Float32Array.from(todo), Object.assign({}, o, { previos: A.concat(B) }));
      out.muestrea.push({ got: r === null ? null : r.id, want });
    }
  }
  // a temperature without top-k cannot use the handful
  assert.strictEqual(await tk.muestrea(lb, 0, logits.length, { temperature: 1 }, [], []), null);
  out.topkStats = JSON.parse(JSON.stringify(tk.stats));
  out.stats = device.stats();
  // the head in one call (cabeza): the logits of quant.matmul and the
  // candidates candidatos() finds in them, bit for bit; muestreaCabeza picks
  // the token muestrea picks from those logits (a second top-k object, so the
  // counts above stay the first one's)
  {
    const tk2 = eff.createTopKGPU(device, ops.ctx);
    const rows = 40000, k = 512;
    const wB = ops.upload(eff.quantize('Q6_K', eff.fillNormal(77, 0.02, rows * k)), 'head');
    const xh = ops.upload(eff.fillNormal(78, 1.0, k), 'xh');
    const plan = { M: 40, S: Uint32Array.from([3, rows - 1]) };
    const r = await tk2.cabeza('Q6_K', wB, xh, rows, k, plan);
    const y = await ops.matmul('Q6_K', wB, xh, rows, k, 1);
    const a = new Uint32Array(await eff.readback(device, r.logits, 0, rows * 4));
    const b = new Uint32Array(await eff.readback(device, y, 0, rows * 4));
    assert.deepStrictEqual(Array.from(a), Array.from(b));
    const c2 = await tk2.candidatos(y, 0, rows, plan);
    assert.ok(r.candidatos !== null && c2 !== null);
    assert.deepStrictEqual(Array.from(r.candidatos.ids), Array.from(c2.ids));
    assert.deepStrictEqual(Array.from(r.candidatos.bits), Array.from(c2.bits));
    assert.deepStrictEqual(Array.from(r.candidatos.bitsS), Array.from(c2.bitsS));
    const o = { temperature: 0.8, topK: 40, topP: 0.9, seed: 5 };
    const m1 = await tk2.muestreaCabeza('Q6_K', wB, xh, rows, k, o, [3], [rows - 1]);
    const m2 = await tk2.muestrea(y, 0, rows, o, [3], [rows - 1]);
    assert.ok(m1.id !== null && m1.id === m2.id);
    // no top-k in the settings: no plan, the logits alone
    const m3 = await tk2.muestreaCabeza('Q6_K', wB, xh, rows, k, { temperature: 1 }, [], []);
    assert.strictEqual(m3.id, null);
    const c3 = new Uint32Array(await eff.readback(device, m3.logits, 0, rows * 4));
    assert.deepStrictEqual(Array.from(c3), Array.from(b));
    await assert.rejects(tk2.cabeza('Q6_K', wB, xh, rows, k + 1, plan), /múltiplo/);
    out.cabeza = true;
    tk2.destroy();
  }
  fs.writeFileSync(path.join(dir, 'out.json'), JSON.stringify(out));
  device.destroy();
  console.log('shim_gpu ok');
}
main().catch((e) => { console.error(e); process.exit(1); });
