'use strict';
// Sampling on the host over a logits vector, and over the handful of
// candidates the device top-k returns (sample.js:17-153, topk.js:62-155).
//
// The candidate step gives the token sample() would give over the whole
// vector, bit for bit, without reading the vector back:
//   * sample() applies the penalties to the ids of the recent window S (at
//     most repeatLastN distinct ids), then only looks at the K' best ids by
//     (logit desc, index asc): K' = 1 greedy, K' = topK with a temperature;
//     top-p, min-p and the temperature read only those K' values;
//   * a penalty only moves the logits of S, and outside S the order of two
//     ids does not change, so each of the K' best after the penalties is
//     either in S or among the raw top K' + |S|;
//   * the candidates are handed to sample() ordered by ascending id, so
//     "lower index first" breaks ties the same way in the handful as in the
//     vocabulary, and the f32 values are the device's raw bits.
// Cases the handful cannot reproduce return null and the caller reads the
// whole vector: a temperature without top-k (everything within 40 of the
// maximum is kept, with no bound), a window id that is not an integer, more
// candidates than the record holds, NaN logits (flagged by the device), and
// penalties that can create a NaN (factor NaN, ±inf or 0; presence ±inf).
// Node >= 12, no dependencies.

const TOPK_M_MAX = 192;   // candidates the device returns at most
const TOPK_P_MAX = 128;   // penalised ids at most
const TOPK_CAP = 256;     // (id, bits) pairs in the record
const TOPK_CABECERA = 8;  // header words of the record

// mulberry32 (Tommy Ettinger's published 32-bit generator), a single step from
// the seed: uniform in [0, 1) (sample.js:33-38). Callers pass seed + step.
function uniforme(seed) {
  let t = ((seed >>> 0) + 0x6D2B79F5) >>> 0;
  t = Math.imul(t ^ (t >>> 15), t | 1);
  t ^= t + Math.imul(t ^ (t >>> 7), t | 61);
  return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
}

// Does id a come before id b: larger logit first, lower index on equal logits
// (-0 equals +0). Not a total order when NaN is present.
function delante(l, a, b) {
  const x = l[a], y = l[b];
  return x > y || (x === y && a < b);
}

// The k best ids in order (sample.js:44-67). A sorted window of k ids: an id
// enters when it beats the last, by binary search for its place.
function topKIndices(logits, k) {
  const n = logits.length;
  const kk = Math.max(0, Math.floor(Math.min(k, n)));
  const best = [];
  for (let i = 0; i < n && kk > 0; i++) {
    if (best.length === kk && !delante(logits, i, best[kk - 1])) continue;
    let lo = 0, hi = best.length;
    while (lo < hi) {
      const mid = (lo + hi) >> 1;
      if (delante(logits, best[mid], i)) lo = mid + 1; else hi = mid;
    }
    best.splice(lo, 0, i);
    if (best.length > kk) best.pop();
  }
  return best;
}

// Without top-k: the ids within `margen` of the maximum, in order (sample.js:70-76).
function dentroDelMargen(logits, margen) {
  let max = -Infinity;
  for (let i = 0; i < logits.length; i++) if (logits[i] > max) max = logits[i];
  const out = [];
  for (let i = 0; i < logits.length; i++) if (logits[i] >= max - margen) out.push(i);
  return out.sort((a, b) => (delante(logits, a, b) ? -1 : 1));
}

// The token of one logits vector (sample.js:78-153), in llama.cpp's order:
// penalties (over the last repeatLastN ids of `previos`, applied to `logits`
// in place) -> greedy argmax when temperature <= 0 -> top-k (or the 40-nat
// window) -> top-p and min-p on the untempered distribution -> temperature
// among the survivors -> one uniform draw from `seed`.
function sample(logits, opts) {
  const o = opts || {};
  const temperature = o.temperature === undefined ? 0 : o.temperature;
  const topP = o.topP === undefined ? 1 : o.topP;
  const topK = o.topK === undefined ? 0 : o.topK;
  const minP = o.minP === undefined ? 0 : o.minP;
  const seed = o.seed === undefined ? 1 : o.seed;
  const repeatPenalty = o.repeatPenalty === undefined ? 1.1 : o.repeatPenalty;
  const repeatLastN = o.repeatLastN === undefined ? 64 : o.repeatLastN;
  const presence = o.presence === undefined ? 0 : o.presence;
  const previos = o.previos || null;
  const n = logits.length;

  if (previos && previos.length && (repeatPenalty !== 1 || presence)) {
    const ids = new Set();
    for (let i = Math.max(0, previos.length - repeatLastN); i < previos.length; i++) ids.add(previos[i]);
    for (const id of ids) {
      if (id < 0 || id >= n) continue;
      if (repeatPenalty !== 1) logits[id] = logits[id] > 0 ? logits[id] / repeatPenalty : logits[id] * repeatPenalty;
      if (presence) logits[id] -= presence;
    }
  }
  if (temperature <= 0) {
    let best = 0;
    for (let i = 1; i < n; i++) if (logits[i] > logits[best]) best = i;
    return best;
  }

  const idx = topK > 0 ? topKIndices(logits, Math.min(topK, n)) : dentroDelMargen(logits, 40);
  const keep = idx.length;
  const max = logits[idx[0]];
  const w = new Float64Array(keep);          // untempered weights, relative to the maximum
  let total = 0;
  for (let i = 0; i < keep; i++) { w[i] = Math.exp(logits[idx[i]] - max); total += w[i]; }
  let corte = keep;
  if (topP < 1) {
    let acc = 0;
    for (let i = 0; i < keep; i++) {
      acc += w[i] / total;
      if (acc >= topP) { corte = i + 1; break; }
    }
  }
  if (minP > 0) {
    const umbral = minP * w[0];
    let j = 1;
    while (j < corte && w[j] >= umbral) j++;
    corte = j;
  }
  const p = new Float64Array(corte);
  let suma = 0;
  for (let i = 0; i < corte; i++) { p[i] = Math.exp((logits[idx[i]] - max) / temperature); suma += p[i]; }
  let r = uniforme(seed) * suma;
  for (let i = 0; i < corte; i++) {
    r -= p[i];
    if (r <= 0) return idx[i];
  }
  return idx[corte - 1];
}

// Which candidates this step needs (planTopK, topk.js:62-94), or null when
// the handful cannot reproduce sample(). `previosA` and `previosB` are the two
// halves of the window (prompt and generated ids), walked as one list. The
// defaults are sample()'s.
function planTopK(vocab, opts, previosA, previosB) {
  const o = opts || {};
  const temperature = o.temperature === undefined ? 0 : o.temperature;
  const topK = o.topK === undefined ? 0 : o.topK;
  const repeatPenalty = o.repeatPenalty === undefined ? 1.1 : o.repeatPenalty;
  const repeatLastN = o.repeatLastN === undefined ? 64 : o.repeatLastN;
  const presence = o.presence === undefined ? 0 : o.presence;
  if (!(vocab >= 1)) return null;
  let K;
  if (temperature <= 0) K = 1;
  else if (topK > 0 && Number.isInteger(topK)) K = Math.min(topK, vocab);
  else return null;

  const a = previosA || [], b = previosB || [];
  const largo = a.length + b.length;
  const penaliza = !!(largo && (repeatPenalty !== 1 || presence));
  const ventana = [];
  const S = [];
  if (penaliza) {
    // the same start (possibly fractional) and indices as sample()'s loop
    const vistos = new Set();
    for (let i = Math.max(0, largo - repeatLastN); i < largo; i++) {
      const id = i < a.length ? a[i] : b[i - a.length];
      if (!Number.isInteger(id)) return null;
      ventana.push(id);
      if (id >= 0 && id < vocab && !vistos.has(id)) { vistos.add(id); S.push(id); }
    }
  }
  if (S.length > TOPK_P_MAX) return null;
  if (S.length && ((repeatPenalty !== 1 && !(Number.isFinite(repeatPenalty) && repeatPenalty !== 0)) ||
      (presence && !Number.isFinite(presence)))) return null;
  const M = K + S.length;
  if (M > TOPK_M_MAX) return null;
  return { vocab, K, M, S: Uint32Array.from(S), penaliza, ventana };
}

// The device record (u32 words) as { ids, bits, bitsS }, or { motivo } when the
// whole vector must be read (leeSalidaTopK, topk.js:100-111). `trozos` is the
// number of chunks the call used and `serie` its serial number.
function leeSalidaTopK(u, plan, trozos, serie) {
  if (serie !== undefined && u[4] !== serie) return { motivo: 'serie' };
  const n = u[0], avisos = u[1];
  if (avisos !== 0) return { motivo: avisos & 2 ? 'NaN' : 'no cupo' };
  if (u[2] !== plan.S.length || u[3] !== trozos || n > TOPK_CAP) return { motivo: 'cabecera' };
  const ini = TOPK_CABECERA + TOPK_P_MAX;
  const ids = new Uint32Array(n), bits = new Uint32Array(n);
  for (let q = 0; q < n; q++) { ids[q] = u[ini + 2 * q]; bits[q] = u[ini + 2 * q + 1]; }
  return { ids, bits, bitsS: u.slice(TOPK_CABECERA, TOPK_CABECERA + plan.S.length) };
}

// The token from the candidates (muestraCandidatos, topk.js:116-155): `ids` /
// `bits` the device's candidates (raw f32 bits), `bitsS` the raw logits of
// plan.S in its order. Null when what came back is not coherent.
function muestraCandidatos(plan, ids, bits, bitsS, opts) {
  const n = ids.length;
  if (bits.length !== n || bitsS.length !== plan.S.length) return null;
  if (n < Math.min(plan.M, plan.vocab)) return null;
  const valor = new Map();
  for (let q = 0; q < n; q++) {
    if (ids[q] >= plan.vocab || valor.has(ids[q])) return null;
    valor.set(ids[q], bits[q]);
  }
  for (let i = 0; i < plan.S.length; i++) {
    const prev = valor.get(plan.S[i]);
    if (prev !== undefined && prev !== bitsS[i]) return null;
    valor.set(plan.S[i], bitsS[i]);
  }
  const orden = Uint32Array.from(valor.keys()).sort();
  const sub = new Float32Array(orden.length);
  const subBits = new Uint32Array(sub.buffer);
  const pos = new Map();
  for (let j = 0; j < orden.length; j++) {
    subBits[j] = valor.get(orden[j]);
    pos.set(orden[j], j);
  }
  // the window as positions in the handful, same order; ids outside the
  // vocabulary become -1, which sample() skips as it skipped them
  let previos = null;
  if (plan.penaliza) {
    previos = plan.ventana.map((id) => (pos.has(id) ? pos.get(id) : -1));
  }
  const j = sample(sub, Object.assign({}, opts, { previos }));
  return orden[j];
}

module.exports = {
  TOPK_M_MAX, TOPK_P_MAX, TOPK_CAP, TOPK_CABECERA,
  uniforme, topKIndices, sample, planTopK, leeSalidaTopK, muestraCandidatos,
};
