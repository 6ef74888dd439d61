'use strict';
// CPU-only checks of the JavaScript host (no device calls): type table,
// Q8_0R buffer arithmetic with the reference's known answers, repack round
// trip, and the error behaviour of quantInfo.
const assert = require('assert');
const path = require('path');
const eff = require(path.join(__dirname, '..', '..', 'elffuss-engine_amd', 'js', 'index.js'));

assert.strictEqual(eff.QUANT_TYPES.Q4_K.blockBytes, 144);
assert.strictEqual(eff.QUANT_TYPES.Q6_K.blockBytes, 210);
assert.strictEqual(eff.QUANT_TYPES.IQ2_XXS.table, 'IQ2XXS');
assert.throws(() => eff.quantInfo('Q4_0'), /no soportado/);

// repack.js:225-229 known answers
assert.strictEqual(eff.bytesReordenado('Q8_0R', 64), 2176);
assert.strictEqual(eff.bytesBufferR('Q8_0R', 64), 2176);
assert.strictEqual(eff.bloquesDeBuffer('Q8_0R', 2304), 67);
assert.strictEqual(eff.escalasDesde('Q8_0R', 10), 80);
for (let n = 1; n < 300; n++) {
  for (let extra = 0; extra <= 28; extra += 4) assert.strictEqual(eff.bloquesDeBuffer('Q8_0R', eff.bytesReordenado('Q8_0R', n) + extra), n);
}

// round trip, odd block counts, destination with slack zeroed
for (const n of [1, 3, 17, 256]) {
  const src = new Uint8Array(34 * n);
  for (let i = 0; i < src.length; i++) src[i] = (i * 131 + 7) & 255;
  const r = eff.reordena('Q8_0', src, n);
  assert.strictEqual(r.length, eff.bytesBufferR('Q8_0R', n));
  for (let i = 0; i < n; i++) {
    for (let j = 0; j < 32; j++) assert.strictEqual(r[32 * i + j], src[34 * i + 2 + j]);
    assert.strictEqual(r[32 * n + 2 * i], src[34 * i]);
    assert.strictEqual(r[32 * n + 2 * i + 1], src[34 * i + 1]);
  }
  for (let i = 34 * n; i < r.length; i++) assert.strictEqual(r[i], 0);
  assert.deepStrictEqual(Array.from(eff.vuelveAlGGUF('Q8_0R', r, n)), Array.from(src));
}
assert.throws(() => eff.reordena('Q8_0', new Uint8Array(68), 2, new Uint8Array(10)), /destino/);

// Q8_0 quantizer (cpu.js:273-287): amax 127 -> d = 1, Math.round ties toward +infinity
const x = new Float32Array(32);
x.set([127, 2.5, -2.5, 0.5, -0.5, -127]);
const q = eff.quantize('Q8_0', x);
assert.strictEqual(q[0] | (q[1] << 8), 0x3C00);
assert.deepStrictEqual(Array.from(new Int8Array(q.buffer, 2, 6)), [127, 3, -2, 1, 0, -127]);

// deterministic generator
const a = eff.fillNormal(5, 0.02, 1000), b = eff.fillNormal(5, 0.02, 10);
for (let i = 0; i < 10; i++) assert.strictEqual(a[i], b[i]);

// The load path over a recording device (the repacked form needs the
// library's device buffers and is checked on the GPU): spans, chunks, the
// 4 bytes of slack, progress, and the errors raised before a byte moves.
async function cargaCpu() {
  const file = new Uint8Array(1200);
  for (let i = 0; i < file.length; i++) file[i] = (i * 7 + 3) & 255;
  const lecturas = [];
  const ranged = {
    size: file.length,
    slice(off, len) { lecturas.push([off, len]); return Promise.resolve(file.slice(off, off + len).buffer); },
  };
  const dev = {
    limits: { maxStorageBufferBindingSize: 4096 },
    createBuffer(d) { return { size: d.size, label: d.label, datos: new Uint8Array(d.size) }; },
    queue: { writeBuffer(b, off, data) { b.datos.set(new Uint8Array(data), off); } },
  };
  const t = (name, typeName, dims, start) => ({ name, typeName, dims, nElements: dims.reduce((p, q) => p * q, 1),
    nBytes: eff.tensorBytes(dims, typeName), start });
  const tabla = [t('a', 'Q8_0', [64, 2], 0), t('b', 'F32', [3], 136), t('c', 'Q4_K', [256], 160),
    t('d', 'Q6_K', [256, 4], 304), t('e', 'F16', [5], 1144)];
  assert.deepStrictEqual(tabla.map((u) => u.nBytes), [136, 12, 144, 840, 10]);
  const prog = [];
  const { pesos, stats } = await eff.cargaTensores(dev, ranged, tabla,
    { tramo: 512, trozo: 300, onProgress: (u, tot, n) => prog.push([u, tot, n]) });
  // [a b] one span; c after 12 bytes of padding; d larger than a span, in
  // chunks of 300; e does not fit in d's span
  assert.deepStrictEqual(lecturas, [[0, 148], [160, 144], [304, 300], [604, 300], [904, 240], [1144, 10]]);
  assert.strictEqual(stats.tramos, 4);
  assert.strictEqual(stats.trozos, 6);
  assert.strictEqual(stats.reordenados, 0);
  assert.deepStrictEqual(prog[prog.length - 1], [1142, 1142, 'e']);
  for (const u of tabla) {
    const { buf, t: d } = pesos.get(u.name);
    assert.strictEqual(d, u);
    assert.strictEqual(buf.size, Math.ceil((u.nBytes + 4) / 4) * 4);
    assert.deepStrictEqual(Array.from(buf.datos.subarray(0, u.nBytes)), Array.from(file.subarray(u.start, u.start + u.nBytes)));
    assert.ok(buf.datos.subarray(u.nBytes).every((v) => v === 0));
  }
  await assert.rejects(eff.cargaTensores(dev, ranged, [t('x', 'Q8_0', [32, 200], 0)], {}), /límite de binding/);
  await assert.rejects(eff.cargaTensores(dev, ranged, [t('x', 'Q4_0', [32], 0), t('y', 'BF16', [2], 18)], {}),
    /sin kernel: Q4_0 \(p\.ej\. «x»\), BF16 \(p\.ej\. «y»\)/);
  assert.deepStrictEqual(eff.comoReordenado(tabla[0], 'Q8_0R'), Object.assign({}, tabla[0], { typeName: 'Q8_0R', typeNameGGUF: 'Q8_0' }));
}

// The ops-context pool (ops.js:233-307) over a recording device: size classes
// of 256 bytes, buffers lent again after recycle() without creating or
// destroying anything, a fresh handout mark each time, recycleDesde keeping
// the live buffers, and classes idle for more than two tokens destroyed.
function poolCpu() {
  const creados = [], destruidos = [];
  const dev = {
    createBuffer(d) {
      const b = { size: d.size, label: d.label, destroy() { destruidos.push(b); } };
      creados.push(b);
      return b;
    },
  };
  const ctx = eff.createContext(dev);
  const a = ctx.alloc(10, 'a'), b = ctx.alloc(256, 'b'), c = ctx.alloc(257, 'c');
  assert.deepStrictEqual([a.size, b.size, c.size], [256, 256, 512]);
  assert.notStrictEqual(a, b);
  assert.strictEqual(ctx.vivosBytes, 1024);
  const marcaA = ctx.marcaDe.get(a);
  ctx.recycle();
  assert.strictEqual(ctx.vivosBytes, 0);
  assert.strictEqual(ctx.picoBytes, 1024);
  const a2 = ctx.alloc(200), c2 = ctx.alloc(400);
  assert.ok(a2 === a || a2 === b);
  assert.strictEqual(c2, c);
  assert.notStrictEqual(ctx.marcaDe.get(a2), marcaA);
  assert.strictEqual(creados.length, 3);
  // between layers: everything after the mark goes back except the survivors
  const marca = ctx.scratch.length;
  const d = ctx.alloc(256), e = ctx.alloc(1000), f = ctx.alloc(256);
  ctx.recycleDesde(marca, e);
  assert.deepStrictEqual(ctx.scratch.map((x) => x.buf), [a2, c2, e]);
  assert.strictEqual(ctx.alloc(256), f);
  assert.strictEqual(ctx.alloc(256), d);
  assert.strictEqual(destruidos.length, 0);
  // a class nobody asks for during more than POZO_RESPIRO tokens is destroyed
  ctx.recycle();
  for (let i = 0; i < 3; i++) { ctx.alloc(256); ctx.recycle(); }
  assert.ok(destruidos.includes(c) && destruidos.includes(e));
  assert.ok(!destruidos.includes(a) && !destruidos.includes(b));
  ctx.destroy();
  assert.strictEqual(new Set(destruidos).size, creados.length);
}

// gemm2.plan / reproducible (ops.gemm2.js:82-126, 282-303): the fp16 GEMM
// only for Q8_0 and Q8_0R, k a multiple of 32, tokens from the DRIFT
// threshold and rows a multiple of 16; null otherwise.
function gemm2Cpu() {
  const device = { option: (o) => (o === eff.OPT.GEMM_MIN_TOKENS ? 64 : 8) };
  const g = eff.createGemm2Ops({ device });
  assert.ok(g.plan('Q8_0', 4096, 2048, 64));
  assert.ok(g.plan('Q8_0R', 4096, 2048, 512));
  for (const [t, rows, k, n] of [['Q8_0', 4096, 2048, 63], ['Q8_0', 4100, 2048, 512], ['Q4_K', 4096, 2048, 512],
    ['Q6_K', 4096, 2048, 512], ['Q2_K', 4096, 2048, 512], ['IQ2_XXS', 4096, 2048, 512], ['Q4_0', 4096, 2048, 512]]) {
    assert.strictEqual(g.plan(t, rows, k, n), null, `${t} ${rows} ${k} ${n}`);
    assert.strictEqual(g.reproducible(t, rows, k, n), false);
  }
  assert.strictEqual(g.reproducible('Q8_0', 4096, 2048, 300), true);
}

poolCpu();
gemm2Cpu();
cargaCpu().then(() => console.log('shim_cpu ok'), (e) => { console.error(e); process.exit(1); });
