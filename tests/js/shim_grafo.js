'use strict';
// GPU run of the JavaScript host's recorded launches and pool behaviour:
//   * gemv ops answer null where the reference's GEMV2 does (types outside
//     GEMV2_TIPOS, more than 3 tokens, an unmarked Q8_0R buffer), lending
//     nothing from the pool; `gemvAmpliado` widens them;
//   * ctx.recycle() destroys an expired size class without waiting for the
//     device (the work enqueued before it still runs, and gives its result);
//   * quant.matmul prepares the split-x product's x once for the products of
//     one activation (one preparation per layout), with the bits of a
//     preparation per call;
//   * ctx.grabaGrafo records a chain of quant.matmul calls, and each replay,
//     after new x is written, gives the bits of the same chain run eagerly.
// Prints one JSON line with the figures the Python side checks.
const assert = require('assert');
const path = require('path');
const eff = require(path.join(__dirname, '..', '..', 'elffuss-engine_amd', 'js', 'index.js'));

const ahora = () => Number(process.hrtime.bigint()) / 1e3;   // microseconds

async function main() {
  const device = await eff.requestDevice();
  const ops = eff.createQuantOps(device);
  const ctx = ops.ctx;
  const out = {};
  const rd = async (buf, n) => new Uint32Array(await eff.readback(device, buf, 0, n * 4));

  // ---- GEMV2 applicability ---------------------------------------------------
  {
    const rows = 64, k = 512;
    const x = ops.upload(eff.fillNormal(5, 1.0, 4 * k), 'x');
    const w4 = ops.upload(eff.quantize('Q4_K', eff.fillNormal(6, 0.02, rows * k)), 'w4');
    const w8 = ops.upload(eff.quantize('Q8_0', eff.fillNormal(7, 0.02, rows * k)), 'w8');
    const n = rows * k / 32;
    const wr = device.createBuffer({ size: eff.bytesBufferR('Q8_0R', n), label: 'wr' });
    device.queue.writeBuffer(wr, 0, eff.reordena('Q8_0', eff.quantize('Q8_0', eff.fillNormal(7, 0.02, rows * k)), n));
    const prestados = ctx.scratch.length;
    const nulos = [
      await ops.gemv.matmul('Q4_K', w4, x, rows, k, 1),
      await ops.gemv.matmul('Q8_0', w8, x, rows, k, 4),
      await ops.gemv.matmul('Q8_0R', wr, x, rows, k, 1),          // unmarked
      await ops.gemv.gateUp('Q4_K', w4, w4, x, rows, k, 1),
      await ops.gemv.secciones('Q2_K', [w4, w4], x, [rows, rows], k, 1),
      await ops.gemv.gateUp('Q8_0', w8, w8, x, rows, k, 4),
    ];
    assert.ok(nulos.every((v) => v === null));
    assert.strictEqual(ctx.scratch.length, prestados);   // nothing was lent
    assert.throws(() => ops.matmul('Q8_0R', wr, x, rows, k, 1), /marca/);
    eff.marcaBufferR(wr, 'Q8_0R', n);
    const a = await ops.gemv.matmul('Q8_0R', wr, x, rows, k, 3);
    const b = await ops.gemv.matmul('Q8_0', w8, x, rows, k, 3);
    assert.deepStrictEqual(Array.from(await rd(a, 3 * rows)), Array.from(await rd(b, 3 * rows)));
    const amp = eff.createQuantOps(device, { ctx, gemvAmpliado: true });
    const c = await amp.gemv.matmul('Q4_K', w4, x, rows, k, 4);
    const d = await ops.matmul('Q4_K', w4, x, rows, k, 4);
    assert.deepStrictEqual(Array.from(await rd(c, 4 * rows)), Array.from(await rd(d, 4 * rows)));
    assert.strictEqual(await amp.gemv.matmul('Q4_K', w4, x, rows, k, 9), null);
    out.gemv2 = true;
    ctx.recycle();
  }

  // ---- gemm2's x -> fp16 memo (aF16, keyed on the allocation mark) ------------
  {
    const k = 1024, m = 300;
    const wq = device.createBuffer({ size: 272 * k / 32 * 34 + 4, label: 'wq' });
    const wk = device.createBuffer({ size: 160 * k / 32 * 34 + 4, label: 'wk' });
    device.queue.writeBuffer(wq, 0, eff.quantize('Q8_0', eff.fillNormal(21, 0.02, 272 * k)));
    device.queue.writeBuffer(wk, 0, eff.quantize('Q8_0', eff.fillNormal(22, 0.02, 160 * k)));
    const xv = eff.fillNormal(23, 1.0, m * k);
    const x = ops.upload(xv, 'x');                       // a pool buffer: it has a mark
    const conv = () => device.stats().gemmX;
    const c0 = conv();
    const yq = await ops.gemm2.matmul('Q8_0', wq, x, 272, k, m);
    const yk = await ops.gemm2.matmul('Q8_0', wk, x, 160, k, m);
    const c1 = conv();
    // the same products without the memo: after olvida() the conversion is paid again
    ops.gemm2.olvida();
    const yk2 = await ops.gemm2.matmul('Q8_0', wk, x, 160, k, m);
    const c2 = conv();
    // x lent again (a new mark) is converted again
    ctx.recycle();
    const x2 = ops.upload(xv, 'x');
    const yq2 = await ops.gemm2.matmul('Q8_0', wq, x2, 272, k, m);
    const c3 = conv();
    // a buffer from outside the pool has no mark: converted on every call
    const xo = device.createBuffer({ size: m * k * 4, label: 'xo' });
    device.queue.writeBuffer(xo, 0, xv);
    const yq3 = await ops.gemm2.matmul('Q8_0', wq, xo, 272, k, m);
    await ops.gemm2.matmul('Q8_0', wq, xo, 272, k, m);
    const c4 = conv();
    const ref = new Uint32Array(await eff.readback(device, yq, 0, 272 * m * 4));
    assert.deepStrictEqual(Array.from(await rd(yq2, 272 * m)), Array.from(ref));
    assert.deepStrictEqual(Array.from(await rd(yq3, 272 * m)), Array.from(ref));
    assert.deepStrictEqual(Array.from(await rd(yk, 160 * m)), Array.from(await rd(yk2, 160 * m)));
    out.memo = { q_k_shared: c1 - c0, after_olvida: c2 - c1, new_mark: c3 - c2, no_mark: c4 - c3 };
    ctx.recycle();
    xo.destroy(); wq.destroy(); wk.destroy();
  }

  // ---- quant.matmul's prepared x (split-x), shared by the products of one x -----
  {
    const k = 2048, m = 33;
    const bytes = { Q4_K: 144, Q6_K: 210, IQ2_XXS: 66 };
    const mats = [['Q4_K', 256, 31], ['Q6_K', 128, 32], ['IQ2_XXS', 192, 33], ['Q4_K', 96, 34]];
    const ws = mats.map(([tipo, rows, seed]) => {
      const b = device.createBuffer({ size: Math.ceil((rows * k / 256 * bytes[tipo] + 4) / 4) * 4, label: tipo });
      device.queue.writeBuffer(b, 0, eff.quantize(tipo, eff.fillNormal(seed, 0.02, rows * k)));
      return b;
    });
    const xv = eff.fillNormal(35, 1.0, m * k);
    const x = ops.upload(xv, 'x');                       // a pool buffer: it has a mark
    const prep = () => device.stats().splitX;
    const p0 = prep();
    const ys = [];
    for (let i = 0; i < mats.length; i++) ys.push(await ops.matmul(mats[i][0], ws[i], x, mats[i][1], k, m));
    const p1 = prep();
    ops.olvida();
    await ops.matmul('Q4_K', ws[0], x, 256, k, m);
    const p2 = prep();
    // an x from outside the pool has no mark: prepared per call, the same bits
    const xo = device.createBuffer({ size: m * k * 4, label: 'xo' });
    device.queue.writeBuffer(xo, 0, xv);
    for (let i = 0; i < mats.length; i++) {
      const y = await ops.matmul(mats[i][0], ws[i], xo, mats[i][1], k, m);
      assert.deepStrictEqual(Array.from(await rd(y, mats[i][1] * m)), Array.from(await rd(ys[i], mats[i][1] * m)));
    }
    const p3 = prep();
    out.memoSplit = { shared: p1 - p0, after_olvida: p2 - p1, no_mark: p3 - p2 };
    ctx.recycle();
    xo.destroy();
    for (const b of ws) b.destroy();
  }

  // ---- quant.matmulCPU: the CPU path's arithmetic (Q8_0), null for other types -----
  {
    const rows = 96, k = 512, m = 3;
    const wq = ops.upload(eff.quantize('Q8_0', eff.fillNormal(41, 0.02, rows * k)), 'w');
    const w4 = ops.upload(eff.quantize('Q4_K', eff.fillNormal(42, 0.02, rows * k)), 'w4');
    const x = ops.upload(eff.fillNormal(43, 1.0, m * k), 'x');
    const y = await ops.matmulCPU('Q8_0', wq, x, rows, k, m);
    out.matmulCPU = { q4k_null: (await ops.matmulCPU('Q4_K', w4, x, rows, k, m)) === null,
      y: Array.from(await rd(y, rows * m)) };
    ctx.recycle();
  }

  // ---- recycle() without a device wait ----------------------------------------
  {
    const rows = 8192, k = 2048, m = 2048, reps = 60;
    const w = device.createBuffer({ size: rows * k / 32 * 34 + 4, label: 'w' });
    device.queue.writeBuffer(w, 0, eff.quantize('Q8_0', eff.fillNormal(8, 0.02, rows * k)));
    const x = ctx.alloc(m * k * 4, 'x');
    for (let i = 0; i < m; i += 64) device.queue.writeBuffer(x, i * k * 4, eff.fillNormal(9 + i, 1.0, 64 * k));
    const y0 = await ops.matmul('Q8_0', w, x, rows, k, m);
    const ref = await rd(y0, 4096);
    ctx.alloc(12345, 'caduca');                       // a size class lent once
    ctx.recycle(); ctx.recycle();
    const talla = Math.ceil(12345 / 256) * 256;
    assert.ok(ctx.scratchFree.has(talla));
    const ys = ctx.alloc(m * rows * 4, 'y');            // the next token's output
    await eff.readback(device, ys, 0, 4);              // the device is idle here
    const t0 = ahora();
    for (let i = 0; i < reps; i++) native(ops, w, x, ys, rows, k, m);
    const t1 = ahora();
    ctx.recycle();                                     // destroys the expired class
    const t2 = ahora();
    assert.ok(!ctx.scratchFree.has(talla));
    const last = await rd(ys, 4096);
    const t3 = ahora();
    assert.deepStrictEqual(Array.from(last), Array.from(ref));
    out.recycle = { enqueue_us: t1 - t0, recycle_us: t2 - t1, drain_us: t3 - t2 };
  }

  // ---- recorded chain -----------------------------------------------------------
  {
    const rows = 2048, k = 2048, porToken = 30;
    const w = device.createBuffer({ size: Math.ceil((rows * k / 256 * 144 + 4) / 4) * 4, label: 'w' });
    device.queue.writeBuffer(w, 0, eff.quantize('Q4_K', eff.fillNormal(1, 0.02, rows * k)));
    const xIn = device.createBuffer({ size: k * 4, label: 'xin' });
    const cadena = async () => {
      let x = xIn;
      for (let i = 0; i < porToken; i++) x = await ops.matmul('Q4_K', w, x, rows, k, 1);
      return x;
    };
    const xs = [eff.fillNormal(2, 1.0, k), eff.fillNormal(3, 1.0, k), eff.fillNormal(4, 1.0, k)];
    const eager = [];
    for (const xv of xs) {
      device.queue.writeBuffer(xIn, 0, xv);
      eager.push(Array.from(await rd(await cadena(), 64)));
      ctx.recycle();
    }
    // while recording, a readback or an upload is refused and the recording is dropped
    await assert.rejects(ctx.grabaGrafo(async () => {
      const y = await cadena();
      await eff.readback(device, y, 0, 16);
      return y;
    }), /graph|grafo/);
    const g = await ctx.grabaGrafo(cadena);
    assert.ok(g.nodos >= porToken, `nodos ${g.nodos}`);
    const replays = [];
    for (let r = 0; r < 2; r++) {
      for (const xv of xs) {
        device.queue.writeBuffer(xIn, 0, xv);
        g.lanza();
        replays.push(Array.from(await rd(g.salida, 64)));
        ctx.recycle();                                 // the recording keeps its buffers
      }
    }
    for (let i = 0; i < replays.length; i++) assert.deepStrictEqual(replays[i], eager[i % 3]);
    // host cost per operation: eager chain against replays
    const tokens = 200;
    let t0 = ahora();
    for (let i = 0; i < tokens; i++) { device.queue.writeBuffer(xIn, 0, xs[0]); await cadena(); ctx.recycle(); }
    await eff.readback(device, xIn, 0, 4);
    const eagerUs = (ahora() - t0) / (tokens * porToken);
    t0 = ahora();
    for (let i = 0; i < tokens; i++) { device.queue.writeBuffer(xIn, 0, xs[0]); g.lanza(); }
    await eff.readback(device, g.salida, 0, 4);
    const grafoUs = (ahora() - t0) / (tokens * porToken);
    g.destroy();
    g.destroy();
    assert.throws(() => g.lanza(), /destruy/);
    out.grafo = { nodos: g.nodos, us_per_op_eager: eagerUs, us_per_op_graph: grafoUs };
  }
  ctx.destroy();
  device.destroy();
  console.log(JSON.stringify(out));
}

// quant.matmul without the pool (the GEMM into a fixed y), for the enqueue loop
function native(ops, w, x, y, rows, k, m) {
  eff.native.qmatmul(ops.ctx.device._ctx, eff.QUANT_TYPES.Q8_0.code, w._h, x._h, y._h, rows, k, m);
}

main().catch((e) => { console.error(e); process.exit(1); });
