'use strict';
// CPU checks of the host sampler and of the candidate step (no device calls):
//   * the uniform generator and sample() against closed forms and the
//     distributions they must draw from;
//   * the candidate step against sample() over the whole vector: with the
//     exact top-M and the raw logits of S computed here by brute force, the
//     token must be the same, bit for bit, over many random vectors, windows
//     and settings (the invariant the device path relies on).
const assert = require('assert');
const path = require('path');
const eff = require(path.join(__dirname, '..', '..', 'elffuss-engine_amd', 'js', 'index.js'));

// a small seeded generator for the test's own inputs (not the sampler's)
function rng(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s / 4294967296;
  };
}

// ---- the uniform draw ------------------------------------------------------
{
  const N = 200000, bins = new Array(16).fill(0);
  let sum = 0, lag = 0, prev = eff.uniforme(0);
  for (let s = 0; s < N; s++) {
    const u = eff.uniforme(s);
    assert.ok(u >= 0 && u < 1, `uniforme(${s}) = ${u}`);
    bins[Math.floor(u * 16)]++;
    sum += u;
    if (s) lag += (u - 0.5) * (prev - 0.5);
    prev = u;
  }
  for (const s of [4294967295, -1, 2 ** 31, 12345678901]) {
    const u = eff.uniforme(s);
    assert.ok(u >= 0 && u < 1);
  }
  assert.strictEqual(eff.uniforme(-1), eff.uniforme(4294967295));   // the seed is taken mod 2^32
  assert.ok(Math.abs(sum / N - 0.5) < 0.003, `mean ${sum / N}`);
  let chi = 0;
  for (const b of bins) chi += (b - N / 16) ** 2 / (N / 16);
  assert.ok(chi < 45, `chi2 ${chi}`);                                // 15 dof: p < 1e-4 beyond
  assert.ok(Math.abs(lag / N * 12) < 0.01, `consecutive seeds correlate: ${lag / N * 12}`);
}

// ---- topKIndices against a full sort ------------------------------------------
const porOrden = (l) => (a, b) => (l[a] > l[b] || (l[a] === l[b] && a < b) ? -1 : 1);
{
  const r = rng(3);
  for (let rep = 0; rep < 200; rep++) {
    const n = 1 + Math.floor(r() * 300);
    const l = new Float32Array(n);
    for (let i = 0; i < n; i++) l[i] = rep % 2 ? Math.floor(r() * 6) - 3 : r() * 10 - 5;
    if (n > 3) { l[1] = -0; l[2] = 0; }
    const all = Array.from({ length: n }, (_, i) => i).sort(porOrden(l));
    for (const k of [1, 2, 5, 40, n, n + 3]) {
      assert.deepStrictEqual(eff.topKIndices(l, k), all.slice(0, Math.min(k, n)));
    }
  }
}

// ---- sample(): closed forms --------------------------------------------------
const f32 = (a) => Float32Array.from(a);
assert.strictEqual(eff.sample(f32([1, 3, 3, 2])), 1);                                  // first of the tied maxima
assert.strictEqual(eff.sample(f32([2, 1.9]), { previos: [0] }), 1);                    // 2 / 1.1 < 1.9
assert.strictEqual(eff.sample(f32([2, 1.9]), { previos: [0], repeatPenalty: 1 }), 0);  // no penalty
assert.strictEqual(eff.sample(f32([-1, -1.05]), { previos: [0] }), 1);                 // -1 * 1.1 < -1.05
assert.strictEqual(eff.sample(f32([1, 0.5]), { previos: [0], repeatPenalty: 1, presence: 0.6 }), 1);
assert.strictEqual(eff.sample(f32([1, 0.5]), { previos: [0], repeatPenalty: 1, presence: 0.4 }), 0);
// only the last repeatLastN ids count, each once, and ids outside the vocabulary are skipped
assert.strictEqual(eff.sample(f32([2, 1.9, 0]), { previos: [0, 2, 2], repeatLastN: 2 }), 0);
assert.strictEqual(eff.sample(f32([2, 1.9, 0]), { previos: [0, 2, 2], repeatLastN: 3 }), 1);
assert.strictEqual(eff.sample(f32([2, 1.9]), { previos: [-1, 2, 7] }), 0);
{
  const l = f32([2, -3, 5]);
  eff.sample(l, { previos: [0, 1, 0, 1], repeatPenalty: 2, presence: 0.5 });
  assert.deepStrictEqual(Array.from(l), [0.5, -6.5, 5]);                              // in place, once per id
}
// top-k 1 with a temperature is the argmax; a tiny top-p keeps only the first
for (let s = 1; s < 50; s++) {
  assert.strictEqual(eff.sample(f32([0, 2, 2, 1]), { temperature: 1.3, topK: 1, seed: s }), 1);
  assert.strictEqual(eff.sample(f32([0, 2, 1.5, 1]), { temperature: 1.3, topP: 1e-9, seed: s }), 1);
}

// ---- sample(): the distributions it draws from ---------------------------------
function frecuencias(l, opts, N) {
  const f = new Array(l.length).fill(0);
  for (let s = 1; s <= N; s++) f[eff.sample(f32(l), Object.assign({}, opts, { seed: s }))]++;
  return f;
}
function chi2(f, p, N) {
  let c = 0;
  for (let i = 0; i < f.length; i++) {
    if (p[i] === 0) { assert.strictEqual(f[i], 0, `id ${i} drawn ${f[i]} times with probability 0`); continue; }
    c += (f[i] - N * p[i]) ** 2 / (N * p[i]);
  }
  return c;
}
function softmax(l, T, keep) {
  const m = Math.max(...keep.map((i) => l[i]));
  const p = new Array(l.length).fill(0);
  let z = 0;
  for (const i of keep) { p[i] = Math.exp((l[i] - m) / T); z += p[i]; }
  return p.map((v) => v / z);
}
{
  const l = [0, 1, 2, -1, 0.5], N = 40000;
  const all = [0, 1, 2, 3, 4];
  // temperature alone: softmax(l / T) over every id (all within 40 of the maximum)
  assert.ok(chi2(frecuencias(l, { temperature: 0.7 }, N), softmax(l, 0.7, all), N) < 25);
  // top-k 3: the three best only
  assert.ok(chi2(frecuencias(l, { temperature: 1.5, topK: 3 }, N), softmax(l, 1.5, [2, 1, 4]), N) < 20);
  // top-p on the untempered distribution: cumulative 0.563, 0.770, 0.896, ... -> 0.75 keeps
  // two ids, 0.8 three
  assert.ok(chi2(frecuencias(l, { temperature: 2, topP: 0.75 }, N), softmax(l, 2, [2, 1]), N) < 15);
  assert.ok(chi2(frecuencias(l, { temperature: 2, topP: 0.8 }, N), softmax(l, 2, [2, 1, 4]), N) < 20);
  // min-p: weight >= 0.3 of the best's -> e^(l-2) >= 0.3 keeps ids 2 and 1 (e^-1 = 0.37, e^-1.5 = 0.22)
  assert.ok(chi2(frecuencias(l, { temperature: 0.9, minP: 0.3 }, N), softmax(l, 0.9, [2, 1]), N) < 15);
  // the 40-nat window: ids more than 40 below the maximum are never drawn
  const far = frecuencias([0, 50, 10.5, 50, 9.5], { temperature: 50 }, 4000);
  assert.strictEqual(far[0] + far[4], 0);
  assert.ok(far[2] > 0 && far[1] > 0 && far[3] > 0);
}

// ---- planTopK ---------------------------------------------------------------------
{
  const p = eff.planTopK(1000, { temperature: 0.8, topK: 40 }, [5, 7, 5, 1200], [9, -2, 7]);
  assert.strictEqual(p.K, 40);
  assert.deepStrictEqual(Array.from(p.S), [5, 7, 9]);
  assert.deepStrictEqual(p.ventana, [5, 7, 5, 1200, 9, -2, 7]);
  assert.strictEqual(p.M, 43);
  assert.strictEqual(eff.planTopK(1000, {}, [], []).M, 1);
  assert.strictEqual(eff.planTopK(1000, { repeatPenalty: 1 }, [5], []).S.length, 0);    // no penalty, no S
  assert.deepStrictEqual(eff.planTopK(1000, {}, [1, 2, 3, 4], [5, 6], undefined).ventana, [1, 2, 3, 4, 5, 6]);
  assert.deepStrictEqual(eff.planTopK(1000, { repeatLastN: 2 }, [1, 2, 3, 4], [5]).ventana, [4, 5]);
  assert.strictEqual(eff.planTopK(1000, { temperature: 0.8 }), null);                     // no top-k: unbounded
  assert.strictEqual(eff.planTopK(1000, { temperature: 0.8, topK: 2.5 }), null);
  assert.strictEqual(eff.planTopK(1000, {}, [1.5]), null);                                // not an integer id
  assert.strictEqual(eff.planTopK(1000, { repeatPenalty: 0 }, [1]), null);
  assert.strictEqual(eff.planTopK(1000, { repeatPenalty: Infinity }, [1]), null);
  assert.strictEqual(eff.planTopK(1000, { repeatPenalty: NaN }, [1]), null);
  assert.strictEqual(eff.planTopK(1000, { repeatPenalty: 1, presence: Infinity }, [1]), null);
  assert.notStrictEqual(eff.planTopK(1000, { repeatPenalty: 0 }, [2000]), null);          // S empty: nothing to break
  const ids = Array.from({ length: 129 }, (_, i) => i);
  assert.strictEqual(eff.planTopK(1000, { repeatLastN: 200 }, ids), null);                // |S| > 128
  assert.notStrictEqual(eff.planTopK(1000, { repeatLastN: 200 }, ids.slice(0, 128)), null);
  assert.strictEqual(eff.planTopK(1000, { temperature: 1, topK: 100, repeatLastN: 200 }, ids.slice(0, 93)), null);  // M 193
  assert.strictEqual(eff.planTopK(1000, { temperature: 1, topK: 100, repeatLastN: 200 }, ids.slice(0, 92)).M, 192);
  assert.strictEqual(eff.planTopK(0, {}), null);
}

// ---- leeSalidaTopK -------------------------------------------------------------
{
  const u = new Uint32Array(8 + 128 + 512);
  const plan = { S: Uint32Array.from([3, 4]) };
  u[0] = 2; u[2] = 2; u[3] = 5; u[4] = 9; u[8] = 11; u[9] = 12;
  u[136] = 70; u[137] = 0x3f800000; u[138] = 71; u[139] = 0x3f000000;
  const r = eff.leeSalidaTopK(u, plan, 5, 9);
  assert.deepStrictEqual(Array.from(r.ids), [70, 71]);
  assert.deepStrictEqual(Array.from(r.bits), [0x3f800000, 0x3f000000]);
  assert.deepStrictEqual(Array.from(r.bitsS), [11, 12]);
  assert.strictEqual(eff.leeSalidaTopK(u, plan, 5, 8).motivo, 'serie');
  assert.strictEqual(eff.leeSalidaTopK(u, plan, 6, 9).motivo, 'cabecera');
  assert.strictEqual(eff.leeSalidaTopK(u, { S: new Uint32Array(1) }, 5, 9).motivo, 'cabecera');
  u[1] = 2; assert.strictEqual(eff.leeSalidaTopK(u, plan, 5, 9).motivo, 'NaN');
  u[1] = 1; assert.strictEqual(eff.leeSalidaTopK(u, plan, 5, 9).motivo, 'no cupo');
  u[1] = 0; u[0] = 257; assert.strictEqual(eff.leeSalidaTopK(u, plan, 5, 9).motivo, 'cabecera');
}

// ---- the candidate step gives sample()'s token --------------------------------------
function candidatosExactos(l, vocab, plan) {
  const orden = Array.from({ length: vocab }, (_, i) => i).sort(porOrden(l));
  const top = orden.slice(0, Math.min(plan.M, vocab));
  const bitsL = new Uint32Array(l.buffer, l.byteOffset, l.length);
  return {
    ids: Uint32Array.from(top),
    bits: Uint32Array.from(top.map((i) => bitsL[i])),
    bitsS: Uint32Array.from(Array.from(plan.S, (i) => bitsL[i])),
  };
}
{
  const r = rng(11);
  let casos = 0, tempCasos = 0;
  for (let rep = 0; rep < 1500; rep++) {
    const vocab = 1 + Math.floor(r() * (rep % 3 ? 600 : 40));
    const l = new Float32Array(vocab);
    const discreto = rep % 4 === 0;                       // many exact ties
    for (let i = 0; i < vocab; i++) l[i] = discreto ? Math.floor(r() * 5) - 2 : (r() * 2 - 1) * 8;
    const greedy = r() < 0.35;
    const opts = {
      temperature: greedy ? 0 : 0.2 + r() * 2,
      topK: greedy ? 0 : 1 + Math.floor(r() * 60),
      topP: r() < 0.5 ? 1 : 0.3 + r() * 0.7,
      minP: r() < 0.5 ? 0 : r() * 0.3,
      seed: Math.floor(r() * 1e6),
      repeatPenalty: [1, 1.1, 1.3, 0.8, -1.2][Math.floor(r() * 5)],
      repeatLastN: [64, 8, 3, 200][Math.floor(r() * 4)],
      presence: r() < 0.6 ? 0 : [1.5, -0.7][Math.floor(r() * 2)],
    };
    const n1 = Math.floor(r() * 30), n2 = Math.floor(r() * 30);
    const pick = () => (r() < 0.1 ? [-1, vocab, vocab + 7][Math.floor(r() * 3)] : Math.floor(r() * vocab));
    const A = Array.from({ length: n1 }, pick), B = Array.from({ length: n2 }, pick);
    const plan = eff.planTopK(vocab, opts, A, B);
    if (!plan) continue;
    const c = candidatosExactos(l, vocab, plan);
    const got = eff.muestraCandidatos(plan, c.ids, c.bits, c.bitsS, opts);
    const want = eff.sample(Float32Array.from(l), Object.assign({}, opts, { previos: A.concat(B) }));
    assert.strictEqual(got, want, `case ${rep}: ${JSON.stringify(opts)} vocab ${vocab}`);
    casos++;
    if (!greedy) tempCasos++;
  }
  assert.ok(casos > 1000 && tempCasos > 500, `${casos} cases, ${tempCasos} with a temperature`);
  // incoherent records are refused
  const l = f32([1, 5, 3, 2]);
  const plan = eff.planTopK(4, { temperature: 1, topK: 2 }, [2], []);
  const c = candidatosExactos(l, 4, plan);
  assert.strictEqual(eff.muestraCandidatos(plan, c.ids.slice(0, 2), c.bits.slice(0, 2), c.bitsS, {}), null);  // too few
  assert.strictEqual(eff.muestraCandidatos(plan, Uint32Array.from([1, 1, 2]), c.bits, c.bitsS, {}), null);   // repeated id
  assert.strictEqual(eff.muestraCandidatos(plan, Uint32Array.from([1, 9, 2]), c.bits, c.bitsS, {}), null);   // outside
  assert.strictEqual(eff.muestraCandidatos(plan, c.ids, c.bits, Uint32Array.from([7]), {}), null);           // S disagrees
}
console.log('shim_muestreo ok');
