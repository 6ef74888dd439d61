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
console.log('shim_cpu ok');
