'use strict';
// JavaScript host of the MI355X quantized matrix-product path: the operator
// objects of Elffuss Engine (createQuantOps, createGemvOps, createGemm2Ops,
// createTopKGPU) and the repack helpers of repack.js / kernels.bloques.wgsl.js,
// with the same call shapes, over the N-API addon (elffuss_amd.node) and the
// C ABI of include/elffuss_amd.h. A drop-in for device.js's WebGPU buffers
// and dispatches on this path only.
//
// Semantics kept from the reference:
//   * operations record work and return without waiting (ops.js:667-710); the
//     Promises they return resolve once the launch is enqueued, and only
//     readback() waits for the device (device.js:165-200);
//   * a fast path that does not apply returns null and the caller falls back
//     (ops.gemv.js:13-21, ops.gemm2.js:5-8);
//   * contract violations throw an Error (ops.js:767-771, 850-852;
//     repack.js:268-286) — here with the library's message and a `code`.
// Written for Node >= 12 (ES2019, CommonJS).

const path = require('path');

const native = require(path.join(__dirname, 'elffuss_amd.node'));
const muestreo = require(path.join(__dirname, 'muestreo.js'));

const STATUS = { NOT_APPLICABLE: 1, E_INVALID: -1, E_TYPE: -2, E_SHAPE: -3, E_MARK: -4, E_BOUNDS: -5, E_DEVICE: -6 };
const OPT = {
  GEMV_MAX_TOKENS: 1, GEMM_MIN_TOKENS: 2, GEMV_KERNEL: 3, SPLIT_CONFIG: 4,
  SPLIT_MIN_TOKENS: 5, GEMM_CONFIG: 6, GEMM_SPLIT: 7, SPLIT_SLICES: 8,
};
const GEMV_MODE = { SECTIONS: 1, SWIGLU: 2 };
const TOPK = { M_MAX: 192, P_MAX: 128, CAP: 256, CABECERA: 8, N_MAX: 1 << 24, POR_TROZO: 4096 };

// ---- types (gguf.js:51-64, kernels.wgsl.js QUANT_TYPES) --------------------
const TYPE_NAMES = ['Q8_0', 'Q8_0R', 'Q4_K', 'Q6_K', 'Q2_K', 'IQ2_XXS'];
const QUANT_TYPES = {};
for (const name of TYPE_NAMES) {
  const code = native.typeFromName(name);
  const g = native.geometry(code);
  QUANT_TYPES[name] = { name, code, blockElems: g.blockElems, blockBytes: g.blockBytes,
    table: name === 'IQ2_XXS' ? 'IQ2XXS' : null };
}

function quantInfo(type) {
  const i = QUANT_TYPES[type];
  if (!i) {
    const e = new Error(`tipo de cuantización no soportado: «${type}»`);
    e.code = STATUS.E_TYPE;
    throw e;
  }
  return i;
}

// ---- device and buffers (device.js / ops.js ctx) ----------------------------

class DeviceBuffer {
  constructor(device, size, label) {
    this.device = device;
    this.size = size;
    this.label = label || '';
    this._h = native.bufAlloc(device._ctx, size);
    this._alive = true;
  }
  // Like GPUBuffer.destroy(), safe with work already submitted and without a
  // wait: the memory goes back in stream order (eff_buf_retire), after the
  // work enqueued before on the context's stream.
  destroy() {
    if (this._alive) {
      native.bufRetire(this.device._ctx, this._h);
      this._alive = false;
    }
  }
}

// The HIP device context standing in for requestDevice() (device.js:66-139).
function requestDevice(opts) {
  const o = opts || {};
  const ctx = native.init(o.device || 0);
  const device = {
    _ctx: ctx,
    // the library's defaults (include/elffuss_amd.h); setOption keeps this in step
    _opts: { 1: 8, 2: 64, 3: 0, 4: 0, 5: 0, 6: 0, 7: 0, 8: 0 },
    features: new Set(['shader-f16']),
    limits: { maxStorageBufferBindingSize: 2 ** 32, maxComputeWorkgroupStorageSize: 163840 },
    createBuffer(desc) {
      return new DeviceBuffer(device, desc.size, desc.label);
    },
    queue: {
      // queue.writeBuffer(buffer, offset, data[, dataOffset, size])
      writeBuffer(buf, offset, data, dataOffset, size) {
        let view = data;
        if (dataOffset !== undefined || size !== undefined) {
          const bytes = ArrayBuffer.isView(data)
            ? new Uint8Array(data.buffer, data.byteOffset, data.byteLength) : new Uint8Array(data);
          const el = ArrayBuffer.isView(data) && data.BYTES_PER_ELEMENT ? data.BYTES_PER_ELEMENT : 1;
          const start = (dataOffset || 0) * el;
          const len = size !== undefined ? size * el : bytes.byteLength - start;
          view = bytes.subarray(start, start + len);
        }
        native.bufWrite(ctx, buf._h, offset, view);
      },
      onSubmittedWorkDone() {
        native.sync(ctx);
        return Promise.resolve();
      },
    },
    setOption(option, value) {
      native.setOption(ctx, option, value);
      device._opts[option] = value;
    },
    option(option) {
      return device._opts[option];
    },
    stats() {
      return native.stats(ctx);
    },
    destroy() {
      native.shutdown(ctx);
    },
  };
  return Promise.resolve(device);
}

// Device -> host copy; waits for the work enqueued before it (device.js:165).
function readback(device, buf, offset, size) {
  const off = offset || 0;
  const n = size === undefined ? buf.size - off : size;
  return native.bufReadAsync(device._ctx, buf._h, off, n);
}

// The ops context and its buffer pool (ops.js:233-307). Buffers are lent by
// size class (bytes rounded up to 256) and live until recycle() (the end of a
// token) or recycleDesde(marca, ...vivos) (between layers); returned buffers
// go back to their class and are lent again without touching the device.
// Reuse is safe without waiting because every operation is enqueued on the
// one stream, in order: a buffer lent again is written after the operations
// that read it in its previous life. A class that nobody asked for during more
// than POZO_RESPIRO tokens is destroyed (ops.js:264-279). Each handout gets a
// fresh number in `marcaDe` (the reference's marca de reparto): a key for
// anything derived from a buffer that must not survive its reuse.
const POZO_RESPIRO = 2;

function createContext(device) {
  const ctx = {
    device,
    scratch: [],              // { buf, size } lent since the last recycle, in order
    scratchFree: new Map(),   // size -> [buf]
    marcaDe: new WeakMap(),
    picoBytes: 0,
    vivosBytes: 0,
    _usoTalla: new Map(),     // size -> last token it was lent in
    _tokenPozo: 0,
  };
  let reparto = 0;
  ctx.alloc = function (bytes, label) {
    const size = Math.max(4, Math.ceil(bytes / 256) * 256);
    const free = ctx.scratchFree.get(size);
    let buf = free && free.pop();
    if (!buf) buf = device.createBuffer({ size, label });
    ctx._usoTalla.set(size, ctx._tokenPozo);
    ctx.marcaDe.set(buf, ++reparto);
    ctx.scratch.push({ buf, size });
    ctx.vivosBytes += size;
    if (ctx.vivosBytes > ctx.picoBytes) ctx.picoBytes = ctx.vivosBytes;
    return buf;
  };
  const devuelve = (e) => {
    if (!ctx.scratchFree.has(e.size)) ctx.scratchFree.set(e.size, []);
    ctx.scratchFree.get(e.size).push(e.buf);
  };
  // Everything lent goes back to the pool; the model calls it after a token.
  ctx.recycle = function () {
    for (const e of ctx.scratch) devuelve(e);
    ctx.scratch = [];
    ctx.vivosBytes = 0;
    ctx._tokenPozo++;
    for (const [size, lista] of ctx.scratchFree) {
      const uso = ctx._usoTalla.has(size) ? ctx._usoTalla.get(size) : 0;
      if (ctx._tokenPozo - uso <= POZO_RESPIRO) continue;
      for (const b of lista) b.destroy();
      ctx.scratchFree.delete(size);
      ctx._usoTalla.delete(size);
    }
  };
  // What was lent from position `marca` of ctx.scratch on goes back, except
  // the buffers in `vivos` (recycling between layers, ops.js:283-307).
  ctx.recycleDesde = function (marca, ...vivos) {
    const guardar = new Set(vivos);
    const quedan = [];
    for (let i = marca; i < ctx.scratch.length; i++) {
      const e = ctx.scratch[i];
      if (guardar.has(e.buf)) { quedan.push(e); continue; }
      devuelve(e);
      ctx.vivosBytes -= e.size;
    }
    ctx.scratch.length = marca;
    for (const e of quedan) ctx.scratch.push(e);
  };
  // A buffer lent by the last alloc() of this size goes back at once (an
  // operation that found it does not apply after lending its output).
  ctx.suelta = function (buf) {
    for (let i = ctx.scratch.length - 1; i >= 0; i--) {
      if (ctx.scratch[i].buf !== buf) continue;
      const e = ctx.scratch.splice(i, 1)[0];
      ctx.vivosBytes -= e.size;
      devuelve(e);
      return;
    }
  };
  // Records what `fn` enqueues into a HIP graph, to replay it per token: the
  // MI355X form of ctx.batch (ops.js:311-332), whose one submit per batch is
  // here one graph launch per replay, with the host's per-launch cost paid
  // once at recording. `fn` (async, device work only: no readback, no upload)
  // runs first eagerly once, a rehearsal that creates the pool's buffers and
  // the library's scratch for these shapes and whose outputs the first replay
  // overwrites, and is then recorded. The buffers it takes from the pool
  // belong to the recording until destroy(); its inputs stay where they
  // were, so new values are written into the same buffers before each
  // lanza(). Resolves to { salida (what the recorded run of fn returned),
  // nodos, lanza(), destroy() }.
  ctx.grabaGrafo = async function (fn) {
    if (ctx._grabando) throw new Error('grabaGrafo: ya hay una grabación abierta');
    const marca = ctx.scratch.length;
    await fn();
    ctx.recycleDesde(marca);
    // a prepared x from before the recording would be read, not prepared, by
    // the recorded products, and stale once x is written between replays
    if (ctx.memoX) ctx.memoX.olvida();
    native.graphBegin(device._ctx);
    ctx._grabando = true;
    let salida;
    try {
      salida = await fn();
    } catch (e) {
      try { native.graphDestroy(native.graphEnd(device._ctx)); } catch (_) { /* the recording is gone */ }
      ctx._grabando = false;
      ctx.recycleDesde(marca);
      throw e;
    }
    ctx._grabando = false;
    const g = native.graphEnd(device._ctx);
    const propios = ctx.scratch.splice(marca);
    for (const e of propios) ctx.vivosBytes -= e.size;
    let vivo = true;
    return {
      salida,
      nodos: native.graphNodes(g),
      lanza() {
        if (!vivo) throw new Error('grabaGrafo: el grafo ya se destruyó');
        native.graphLaunch(device._ctx, g);
      },
      destroy() {
        if (!vivo) return;
        vivo = false;
        native.graphDestroy(g);
        for (const e of propios) devuelve(e);
      },
    };
  };
  // Destroys every pooled and lent buffer (end of the session).
  ctx.destroy = function () {
    for (const e of ctx.scratch) e.buf.destroy();
    for (const lista of ctx.scratchFree.values()) for (const b of lista) b.destroy();
    ctx.scratch = [];
    ctx.scratchFree.clear();
    ctx._usoTalla.clear();
    ctx.vivosBytes = 0;
  };
  return ctx;
}

// ---- repacked layout (repack.js, kernels.bloques.wgsl.js) ---------------------

const TIPOS_R = new Set(['Q8_0R']);
const TIPO_R = Object.freeze({ Q8_0: 'Q8_0R' });
const TIPO_GGUF = Object.freeze({ Q8_0R: 'Q8_0' });
const R_CODE = QUANT_TYPES.Q8_0R.code;

function checkR(tipo, what) {
  if (tipo !== 'Q8_0R' && tipo !== 'Q8_0') throw new Error(`${what}: tipo sin formato reordenado: «${tipo}»`);
}
function bytesReordenado(tipo, nBloques) { checkR(tipo, 'bytesReordenado'); return native.bufferMath(0, R_CODE, nBloques); }
function bytesBufferR(tipo, nBloques) { checkR(tipo, 'bytesBufferR'); return native.bufferMath(1, R_CODE, nBloques); }
function bloquesDeBuffer(tipo, bytes) { checkR(tipo, 'bloquesDeBuffer'); return native.bufferMath(2, R_CODE, bytes); }
function escalasDesde(tipo, nBloques) { checkR(tipo, 'escalasDesde'); return native.bufferMath(3, R_CODE, nBloques); }

// reordena (repack.js:187-199): Q8_0 GGUF bytes -> Q8_0R, into `dst` if given.
function reordena(tipo, src, nBloques, dst) {
  checkR(tipo, 'reordena');
  const need = bytesReordenado(tipo, nBloques);
  if (dst && dst.byteLength < need) throw new Error(`reordena: el destino mide ${dst.byteLength} y hacen falta ${need}`);
  const out = native.repack(R_CODE, src, nBloques, dst ? dst.byteLength : bytesBufferR(tipo, nBloques));
  if (dst) { new Uint8Array(dst.buffer, dst.byteOffset, dst.byteLength).set(out); return dst; }
  return out;
}

// vuelveAlGGUF (repack.js:204-219).
function vuelveAlGGUF(tipo, src, nBloques) {
  checkR(tipo, 'vuelveAlGGUF');
  return native.unrepack(R_CODE, src, nBloques);
}

// marcaBufferR (repack.js:241-251): the mark lives with the device buffer.
function marcaBufferR(buf, tipoR, nBloques) {
  if (!TIPOS_R.has(tipoR)) throw new Error(`marcaBufferR: «${tipoR}» no es un tipo reordenado`);
  if (!(nBloques > 0) || nBloques % 1 !== 0) throw new Error(`marcaBufferR: número de bloques inválido: ${nBloques}`);
  const esperado = bytesBufferR(tipoR, nBloques);
  if (buf.size !== esperado || native.bufMarkR(buf._h, R_CODE, nBloques) !== 0) {
    throw new Error(`marcaBufferR: «${buf.label || '?'}» mide ${buf.size} bytes y un ${tipoR} de ` +
      `${nBloques} bloques tiene que medir ${esperado}`);
  }
  return buf;
}

// bloquesR (repack.js:256-259).
function bloquesR(buf) {
  return native.bufBlocksR(buf._h);
}

// compruebaBufferR (repack.js:268-286).
function compruebaBufferR(tipo, buf, opts, que) {
  const o = opts || {};
  const bloques = o.bloques || 0, porFila = o.porFila || 0;
  const q = que || 'lector';
  const n = bloquesR(buf);
  if (n === undefined) {
    throw new Error(`${q} ${tipo}: el buffer «${buf.label || '?'}» no lleva la marca de un tensor reordenado`);
  }
  if (!TIPOS_R.has(tipo)) throw new Error(`${q}: el buffer «${buf.label || '?'}» guarda un Q8_0R y se iba a leer como ${tipo}`);
  if (bloques > n) throw new Error(`${q} ${tipo}: la llamada lee ${bloques} bloques y el tensor de «${buf.label || '?'}» tiene ${n}`);
  if (porFila > 0 && n % porFila !== 0) throw new Error(`${q} ${tipo}: el tensor (${n} bloques) no son filas enteras de ${porFila} bloques`);
  return n;
}

// creaBufferR (repack.js:293-306).
function creaBufferR(device, t, tipoR) {
  const nBloques = t.nElements / 32;
  const buf = device.createBuffer({ size: bytesBufferR(tipoR, nBloques), label: t.name });
  return marcaBufferR(buf, tipoR, nBloques);
}

// ---- load path (gguf.js:97-111, model.js:141-330, repack.js:69-84, 308-345) ---

// [block elements, block bytes] of the tensor types a load accepts: the GGUF
// types with a kernel here, and the float types a model carries beside them
// (norm weights, biases), which go up as plain bytes (gguf.js:51-64).
const GEOMETRIA_CARGA = { F32: [1, 4], F16: [1, 2] };
for (const name of TYPE_NAMES) {
  if (!TIPOS_R.has(name)) GEOMETRIA_CARGA[name] = [QUANT_TYPES[name].blockElems, QUANT_TYPES[name].blockBytes];
}

// Bytes of a tensor: whole blocks along dims[0] times the other dims
// (tensorBytes, gguf.js:104-111); 0 for a type the load does not accept.
function tensorBytes(dims, typeName) {
  const g = GEOMETRIA_CARGA[typeName];
  if (!g) return 0;
  let n = (dims[0] / g[0]) * g[1];
  for (let i = 1; i < dims.length; i++) n *= dims[i];
  return n;
}

// The descriptor that travels with a repacked buffer: a copy with the internal
// type, the file's type kept beside it (comoReordenado, repack.js:78-80).
function comoReordenado(t, tipoR) {
  return Object.assign({}, t, { typeName: tipoR, typeNameGGUF: t.typeName });
}

function incompleto(que, pedidos, llegaron) {
  return new Error(`${que}: pedidos ${pedidos} bytes y llegaron ${llegaron}`);
}

// subeReordenadoPorTrozos (repack.js:318-345): a Q8_0 tensor too large for
// one read goes up in chunks of whole blocks, an even number per chunk as the
// reference cuts them, each repacked on the host and written to its quants and
// scales regions of the marked buffer by the library (eff_buf_write_r).
// `cuenta(msLeer, msSubir, bytes)` is called once per chunk.
async function subeReordenadoPorTrozos(o) {
  const { device, ranged, t, buf, tipoR } = o;
  if (!TIPOS_R.has(tipoR)) throw new Error(`subeReordenadoPorTrozos: «${tipoR}» no es un tipo reordenado`);
  const ahora = o.ahora || Date.now;
  const cuenta = o.cuenta || (() => {});
  const B = QUANT_TYPES.Q8_0.blockBytes;
  const N = t.nElements / QUANT_TYPES.Q8_0.blockElems;
  const porTrozo = Math.max(2, 2 * Math.floor(o.trozo / (2 * B)));
  for (let b0 = 0; b0 < N; b0 += porTrozo) {
    const nb = Math.min(porTrozo, N - b0);
    const t0 = ahora();
    const raw = await ranged.slice(t.start + b0 * B, nb * B);
    const t1 = ahora();
    // A short chunk would go up as weights without a single error.
    if (raw.byteLength !== nb * B) throw incompleto(`trozo incompleto en «${t.name}»`, nb * B, raw.byteLength);
    native.bufWriteR(device._ctx, buf._h, R_CODE, b0, raw);
    cuenta(t1 - t0, ahora() - t1, nb * B);
  }
}

// The weight upload of loadModel (model.js:141-330) over a tensor table
// ({name, typeName, dims, nElements, nBytes, start} per tensor, as parseGGUF
// gives it) and a ranged handle ({size, slice(offset, length) -> Promise of
// an ArrayBuffer}):
//   * every type must have a kernel (or be F32/F16) before a byte moves;
//   * tensors that follow each other in the file are read together, in spans
//     of up to `tramo` bytes (default 128 MiB); a larger tensor is read alone
//     in chunks of `trozo` bytes (default 32 MiB);
//   * each tensor gets its own buffer with 4 bytes of slack after the data,
//     zero like the rest of a new buffer;
//   * with `reorden` (the __ELFFUSS_REPACK switch, read once per load) Q8_0
//     tensors go up repacked as Q8_0R into marked buffers, and their
//     descriptor says Q8_0R.
// Resolves to { pesos: Map name -> { buf, t }, stats }.
async function cargaTensores(device, ranged, tensores, opciones) {
  const o = opciones || {};
  const onProgress = o.onProgress || (() => {});
  const conReorden = o.reorden === true;
  const TRAMO = Math.max(1, Math.floor(o.tramo || 128 * 1048576));
  const TROZO = Math.max(1, Math.floor(o.trozo || 32 * 1048576));
  const ahora = o.ahora || (() => (typeof performance !== 'undefined' ? performance.now() : Date.now()));
  const limite = device.limits.maxStorageBufferBindingSize;

  const sinKernel = new Map();
  for (const t of tensores) {
    if (!GEOMETRIA_CARGA[t.typeName] && !sinKernel.has(t.typeName)) sinKernel.set(t.typeName, t.name);
  }
  if (sinKernel.size) {
    throw new Error('el fichero trae tipos sin kernel: ' +
      Array.from(sinKernel, ([k, n]) => `${k} (p.ej. «${n}»)`).join(', '));
  }

  const tramos = [];
  for (const t of tensores) {
    if (t.nBytes > limite) throw new Error(`«${t.name}» son ${t.nBytes} bytes y el límite de binding es ${limite}`);
    const ult = tramos[tramos.length - 1];
    // Only a tensor that starts where the previous one ends joins its span:
    // padding between them would otherwise become part of a weight.
    if (ult && t.start === ult.fin && ult.fin - ult.ini + t.nBytes <= TRAMO) {
      ult.fin += t.nBytes;
      ult.ts.push(t);
    } else {
      tramos.push({ ini: t.start, fin: t.start + t.nBytes, ts: [t] });
    }
  }

  const pesos = new Map();
  const stats = { msLeer: 0, msSubir: 0, trozos: 0, tramos: tramos.length, reordenados: 0, bytes: 0 };
  const total = tensores.reduce((n, t) => n + t.nBytes, 0);
  const avanza = (n, nombre) => { stats.bytes += n; onProgress(stats.bytes, total, nombre); };
  const conHolgura = (t) => device.createBuffer({ size: Math.ceil((t.nBytes + 4) / 4) * 4, label: t.name });
  const tipoRDe = (t) => (conReorden && TIPO_R[t.typeName]) || null;

  for (const tr of tramos) {
    const largo = tr.fin - tr.ini;
    if (largo > TRAMO) {
      const t = tr.ts[0];
      const tipoR = tipoRDe(t);
      if (tipoR) {
        const buf = creaBufferR(device, t, tipoR);
        await subeReordenadoPorTrozos({
          device, ranged, t, buf, tipoR, trozo: TROZO, ahora,
          cuenta: (leer, subir, n) => {
            stats.msLeer += leer; stats.msSubir += subir; stats.trozos++;
            avanza(n, t.name);
          },
        });
        pesos.set(t.name, { buf, t: comoReordenado(t, tipoR) });
        stats.reordenados++;
        continue;
      }
      const buf = conHolgura(t);
      for (let off = 0; off < t.nBytes; off += TROZO) {
        const len = Math.min(TROZO, t.nBytes - off);
        const t0 = ahora();
        const raw = await ranged.slice(t.start + off, len);
        const t1 = ahora();
        if (raw.byteLength !== len) throw incompleto(`trozo incompleto en «${t.name}»`, len, raw.byteLength);
        device.queue.writeBuffer(buf, off, raw);
        stats.msLeer += t1 - t0; stats.msSubir += ahora() - t1; stats.trozos++;
        avanza(len, t.name);
      }
      pesos.set(t.name, { buf, t });
      continue;
    }

    const t0 = ahora();
    const span = new Uint8Array(await ranged.slice(tr.ini, largo));
    stats.msLeer += ahora() - t0; stats.trozos++;
    if (span.byteLength !== largo) throw incompleto(`tramo incompleto desde ${tr.ini}`, largo, span.byteLength);
    for (const t of tr.ts) {
      const tipoR = tipoRDe(t);
      const t1 = ahora();
      const bytes = span.subarray(t.start - tr.ini, t.start - tr.ini + t.nBytes);
      let buf;
      if (tipoR) {
        buf = creaBufferR(device, t, tipoR);
        native.bufWriteR(device._ctx, buf._h, R_CODE, 0, bytes);
        stats.reordenados++;
      } else {
        buf = conHolgura(t);
        device.queue.writeBuffer(buf, 0, bytes);
      }
      stats.msSubir += ahora() - t1;
      avanza(t.nBytes, t.name);
      pesos.set(t.name, { buf, t: tipoR ? comoReordenado(t, tipoR) : t });
    }
  }
  return { pesos, stats };
}

// ---- operators ---------------------------------------------------------------

// createGemvOps (ops.gemv.js:44-221): the decode GEMV, null when it does not
// apply. It applies where the reference's GEMV2 does (`prepara`,
// ops.gemv.js:111-135): the types of GEMV2_TIPOS that exist here (Q8_0,
// Q8_0R, Q6_K; kernels.gemv.wgsl.js:83-91), 1 to GEMV2_MAX_TOKENS = 3 tokens
// (kernels.gemv.wgsl.js:79), k a whole number of blocks and, for Q8_0R, a
// buffer whose mark passes compruebaBufferR (else null, and quant.matmul
// throws with its reason). `deps.ampliado` widens it to every type of this
// library and, for matmul, to 8 tokens. Applicability is decided before
// anything is lent from the pool.
const GEMV2_TIPOS = new Set(['Q8_0', 'Q8_0R', 'Q6_K']);
const GEMV2_MAX_TOKENS = 3;

function createGemvOps(device, deps) {
  const ctx = deps.ctx;
  const ampliado = deps.ampliado === true;
  const hechos = { matmul: 0, gateUp: 0, secciones: 0 };
  // The type's entry when the call applies, else null (ops.gemv.js:111-135).
  const prepara = (tipo, k, t, maxT, bufs, filas) => {
    const i = QUANT_TYPES[tipo];
    if (!i || !(ampliado || GEMV2_TIPOS.has(tipo))) return null;
    if (!Number.isInteger(t) || t < 1 || t > maxT) return null;
    if (!(k > 0) || k % i.blockElems !== 0) return null;
    for (let j = 0; j < bufs.length; j++) {
      if (!(filas[j] >= 1) || !bufs[j] || !(bufs[j].size > 0)) return null;
      if (TIPOS_R.has(tipo)) {
        try {
          compruebaBufferR(tipo, bufs[j], { bloques: filas[j] * (k / i.blockElems) }, 'gemv2');
        } catch (_) {
          return null;
        }
      }
    }
    return i;
  };
  return {
    matmul(tipo, wBuf, xBuf, rows, k, tokens) {
      const t = tokens === undefined ? 1 : tokens;
      const i = prepara(tipo, k, t, ampliado ? 8 : GEMV2_MAX_TOKENS, [wBuf], [rows]);
      if (!i) return Promise.resolve(null);
      const y = ctx.alloc(rows * t * 4, 'matmul.y');
      const r = native.qgemv(device._ctx, i.code, wBuf._h, xBuf._h, y._h, rows, k, t);
      if (r === null) { ctx.suelta(y); return Promise.resolve(null); }
      hechos.matmul++;
      return Promise.resolve(y);
    },
    // silu(W_gate·x)·(W_up·x) in one launch (ops.gemv.js:166-190).
    gateUp(tipo, wGate, wUp, xBuf, rows, k, tokens) {
      const t = tokens === undefined ? 1 : tokens;
      const i = prepara(tipo, k, t, GEMV2_MAX_TOKENS, [wGate, wUp], [rows, rows]);
      if (!i) return Promise.resolve(null);
      const y = ctx.alloc(rows * t * 4, 'swiglu.out');
      const r = native.qgemvMulti(device._ctx, i.code, GEMV_MODE.SWIGLU, [wGate._h, wUp._h], xBuf._h, [y._h],
        [rows, rows], k, t);
      if (r === null) { ctx.suelta(y); return Promise.resolve(null); }
      hechos.gateUp++;
      return Promise.resolve(y);
    },
    // 2 to 4 matrices sharing x, each with its rows and its output, in one
    // launch; the outputs in the order of the weights (ops.gemv.js:192-215).
    secciones(tipo, ws, xBuf, filas, k, tokens) {
      const t = tokens === undefined ? 1 : tokens;
      const n = ws.length;
      if (n < 2 || n > 4 || filas.length !== n) return Promise.resolve(null);
      const i = prepara(tipo, k, t, GEMV2_MAX_TOKENS, ws, filas);
      if (!i) return Promise.resolve(null);
      const ys = filas.map((f) => ctx.alloc(f * t * 4, 'matmul.y'));
      const r = native.qgemvMulti(device._ctx, i.code, GEMV_MODE.SECTIONS, ws.map((w) => w._h), xBuf._h,
        ys.map((y) => y._h), filas, k, t);
      if (r === null) { for (let j = ys.length - 1; j >= 0; j--) ctx.suelta(ys[j]); return Promise.resolve(null); }
      hechos.secciones++;
      return Promise.resolve(ys);
    },
    despachados() { return Object.assign({}, hechos); },
    rechazados() { return []; },
  };
}

// createFusionOps, the part on this path (ops.fusion.js:154-170): the
// embedding gather fused with the first layer's RMS norm.
const TIPOS_GATHER_NORMA = new Set(['Q8_0', 'Q2_K', 'Q4_K', 'Q6_K', 'Q8_0R']);
function createFusionOps(device, deps) {
  const ctx = deps.ctx;
  return {
    gatherNorma(type, wBuf, idsBuf, wNorm, dim, tokens, eps) {
      const i = QUANT_TYPES[type];
      if (!i || !TIPOS_GATHER_NORMA.has(type)) throw new Error(`gather+norma: tipo «${type}» sin lector de bloque`);
      if (dim % i.blockElems !== 0) throw new Error(`gather+norma ${type}: dim=${dim} no es múltiplo de ${i.blockElems}`);
      if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { porFila: dim / i.blockElems }, 'gather+norma');
      const x = ctx.alloc(tokens * dim * 4, 'embd');
      const nrm = ctx.alloc(tokens * dim * 4, 'fusion.nrm');
      native.gatherNorm(device._ctx, i.code, wBuf._h, idsBuf._h, wNorm._h, eps, x._h, nrm._h, dim, tokens);
      return Promise.resolve({ x, nrm });
    },
  };
}

// createGemm2Ops (ops.gemm2.js:259-303): the prefill GEMM, null when it does
// not apply. The plan follows planGemm2 (ops.gemm2.js:82-126): the fp16 GEMM
// takes Q8_0 and Q8_0R (GEMM2_TIPOS, kernels.gemm2.wgsl.js:51; Q4_0 has no
// kernel here), k a multiple of 32, tokens >= the DRIFT threshold (the GEMM
// min option, __ELFFUSS_DRIFT_DESDE, default 64) and rows a multiple of 16.
const GEMM2_TIPOS = new Set(['Q8_0', 'Q8_0R']);

// Prepared activations with a memo (aF16, ops.gemm2.js:151-196): the same
// activation feeds several products in a row (the norm's output q, k, v; the
// FFN's gate and up), and the preparation is the same operation on the same
// bytes, so reusing it changes no bit. The key is the pool's allocation mark
// of x (ctx.marcaDe), not the buffer: a buffer lent again gets a new mark. A
// preparation is reused only while its own buffer is still lent under the
// mark it was made with (a returned one could be lent to the same call as
// its output). The library gives the bytes and an id of the layout a product
// reads (eff_gemm_x_layout, eff_qmatmul_x_layout): a preparation serves every
// product whose layout id, tokens and k match — the fp16 x of the GEMM, the
// hi/lo parts of the split-x product. One memo per pool, shared by gemm2 and
// quant.matmul; four entries, oldest dropped first.
function memoPreparados(ctx) {
  if (ctx.memoX) return ctx.memoX;
  const prestado = (buf) => ctx.scratch.some((e) => e.buf === buf);
  const memo = [];
  ctx.memoX = {
    // the prepared x for `lay` ({bytes, layout}); `prepara(xp)` fills a new one
    toma(xBuf, lay, tokens, k, label, prepara) {
      const marca = ctx.marcaDe.get(xBuf);
      if (marca !== undefined) {
        for (let i = memo.length - 1; i >= 0; i--) {
          const m = memo[i];
          if (m.marca === marca && m.layout === lay.layout && m.tokens === tokens && m.k === k &&
              ctx.marcaDe.get(m.xp) === m.marcaXp && prestado(m.xp)) return m.xp;
        }
      }
      const xp = ctx.alloc(lay.bytes, label);
      prepara(xp);
      if (marca !== undefined) {
        memo.push({ marca, layout: lay.layout, tokens, k, xp, marcaXp: ctx.marcaDe.get(xp) });
        if (memo.length > 4) memo.shift();
      }
      return xp;
    },
    olvida() { memo.length = 0; },
  };
  return ctx.memoX;
}

function createGemm2Ops(ctx) {
  const device = ctx.device;
  const desde = () => device.option(OPT.GEMM_MIN_TOKENS);
  const memo = memoPreparados(ctx);
  function aF16(code, xBuf, rows, k, tokens, lote) {
    const lay = native.gemmXLayout(device._ctx, code, rows, k, tokens, lote);
    if (lay === null) return null;
    return memo.toma(xBuf, lay, tokens, k, 'gemm2.x',
      (xh) => native.gemmPrepareX(device._ctx, code, xBuf._h, xh._h, rows, k, tokens, lote));
  }
  const ops = {
    // What this shape would run (null: the caller's usual path).
    plan(type, rows, k, tokens) {
      const i = QUANT_TYPES[type];
      if (!i || !GEMM2_TIPOS.has(type) || k % 32 !== 0 || !(tokens >= 1)) return null;
      if (!(tokens >= desde()) || rows % 16 !== 0) return null;
      return { via: 'mfma-f16', type, bpr: k / i.blockElems, lote: tokens };
    },
    // Empties the x -> fp16 memo (for benches: so that one measurement does
    // not save conversions another one pays, ops.gemm2.js:265-266).
    olvida() { memo.olvida(); },
    matmul(type, wBuf, xBuf, rows, k, tokens) {
      if (tokens < 4 && tokens < desde()) return Promise.resolve(null);
      const pl = ops.plan(type, rows, k, tokens);
      if (!pl) return Promise.resolve(null);
      const i = QUANT_TYPES[type];
      if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { bloques: rows * pl.bpr }, 'gemm2');
      const xh = aF16(i.code, xBuf, rows, k, tokens, tokens);
      if (!xh) return Promise.resolve(null);
      const y = ctx.alloc(rows * tokens * 4, 'matmul.y');
      const r = native.qgemmPrepared(device._ctx, i.code, wBuf._h, xh._h, y._h, rows, k, tokens, tokens);
      return Promise.resolve(r === null ? null : y);
    },
    // The kernel's output for one token depends only on its x row and W,
    // summed in the order of the batch's configuration, so the tail is
    // reproducible whenever the batch has a plan.
    reproducible(type, rows, k, lote) { return ops.plan(type, rows, k, lote) !== null; },
    // The last-layer tail (ops.gemm2.js:282-303): `x1` is one row, the last
    // token of a batch of `lote`; computed with the batch's plan (same kernel,
    // tile and k order), it gives the bits of that token's row in the batch.
    cola(type, wBuf, x1, rows, k, lote) {
      const pl = ops.plan(type, rows, k, lote);
      if (!pl) return Promise.resolve(null);
      const i = QUANT_TYPES[type];
      if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { bloques: rows * pl.bpr }, 'gemm2');
      const xh = aF16(i.code, x1, rows, k, 1, lote);
      if (!xh) return Promise.resolve(null);
      const y = ctx.alloc(rows * 4, 'matmul.y');
      const r = native.qgemmPrepared(device._ctx, i.code, wBuf._h, xh._h, y._h, rows, k, 1, lote);
      return Promise.resolve(r === null ? null : y);
    },
  };
  return ops;
}

// createQuantOps (ops.js:748-1142). opts: { ctx, gemvAmpliado } (the
// latter widens quant.gemv, see createGemvOps).
function createQuantOps(device, opts) {
  const o = opts || {};
  const ctx = o.ctx || createContext(device);
  const gemv = createGemvOps(device, { ctx, ampliado: o.gemvAmpliado === true });
  const gemm2 = createGemm2Ops(ctx);
  const memo = memoPreparados(ctx);
  return {
    // Whole tensor -> f32, bit-exact with the reference decoders (ops.js:813-823).
    dequant(type, wBuf, nBlocks) {
      const i = quantInfo(type);
      if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { bloques: nBlocks }, 'dequant');
      const out = ctx.alloc(nBlocks * i.blockElems * 4, 'dequant.out');
      native.dequant(device._ctx, i.code, wBuf._h, out._h, nBlocks);
      return Promise.resolve(out);
    },
    // Rows ids[t] of a quantized table (the embeddings) as f32 [tokens][dim]
    // (ops.js:1104-1118); throws when dim is not a multiple of the block.
    gather(type, wBuf, idsBuf, dim, tokens) {
      const i = quantInfo(type);
      if (dim % i.blockElems !== 0) throw new Error(`gather ${type}: dim=${dim} no es múltiplo de ${i.blockElems}`);
      if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { porFila: dim / i.blockElems }, 'gather');
      const dst = ctx.alloc(tokens * dim * 4, 'embd');
      native.gather(device._ctx, i.code, wBuf._h, idsBuf._h, dst._h, dim, tokens);
      return Promise.resolve(dst);
    },
    // Y[tokens][rows] = W . X (ops.js:827-1101); throws when k is not a
    // multiple of the block, or for an unmarked repacked buffer. Where the
    // router's path reads a prepared x (the split-x product, the fp16 GEMM),
    // the preparation comes from the pool's memo: the products of one
    // activation prepare it once (the same bits as preparing it per call).
    matmul(type, wBuf, xBuf, rows, k, tokens) {
      const t = tokens === undefined ? 1 : tokens;
      const i = quantInfo(type);
      if (k % i.blockElems !== 0) throw new Error(`matmul ${type}: k=${k} no es múltiplo de ${i.blockElems}`);
      if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { bloques: rows * (k / i.blockElems) }, 'matmul');
      const y = ctx.alloc(rows * t * 4, 'matmul.y');
      // (one token: every path reads x itself; from 2 the router says which
      // prepared x its path reads, if any)
      const lay = t >= 2 ? native.qmatmulXLayout(device._ctx, i.code, rows, k, t) : null;
      if (lay === null) {
        native.qmatmul(device._ctx, i.code, wBuf._h, xBuf._h, y._h, rows, k, t);
      } else {
        const xp = memo.toma(xBuf, lay, t, k, 'matmul.x',
          (p) => native.qmatmulPrepareX(device._ctx, i.code, xBuf._h, p._h, rows, k, t));
        native.qmatmulPrepared(device._ctx, i.code, wBuf._h, xp._h, y._h, rows, k, t);
      }
      return Promise.resolve(y);
    },
    // Y = W . X for Q8_0 with the reference CPU path's arithmetic (8-bit x
    // blocks and integer block dots, cpu.js:350-381): the bits cpu-kernels.js
    // gives, for a caller that needs the GPU and CPU backends to agree; null
    // for the other types (the CPU path has no kernel for them,
    // cpu-trabajo.js:31). Not in the reference's quant ops, whose GPU path
    // is f32 (as quant.matmul here).
    matmulCPU(type, wBuf, xBuf, rows, k, tokens) {
      const t = tokens === undefined ? 1 : tokens;
      const i = quantInfo(type);
      if (k % i.blockElems !== 0) throw new Error(`matmul ${type}: k=${k} no es múltiplo de ${i.blockElems}`);
      if (type !== 'Q8_0') return Promise.resolve(null);
      const y = ctx.alloc(rows * t * 4, 'matmul.y');
      native.qmatmulCpuPath(device._ctx, i.code, wBuf._h, xBuf._h, y._h, rows, k, t);
      return Promise.resolve(y);
    },
    // Empties the memo of prepared activations (gemm2.olvida()).
    olvida() { memo.olvida(); },
    // The IQ2_XXS grid is part of the library (no upload needed).
    prepare(types) {
      for (const t of new Set(types)) quantInfo(t);
      return Promise.resolve();
    },
    upload(array, label) {
      const buf = ctx.alloc(array.byteLength, label || 'x');
      device.queue.writeBuffer(buf, 0, array);
      return buf;
    },
    ctx,
    gemv,
    gemm2,
  };
}

// createTopKGPU (ops.topk.js:42-190): candidatos() returns the exact top-M by
// (value desc, index asc) of one logits vector plus the raw logits of the
// penalised ids, or null when the device result must not be used; muestrea()
// is the whole step (plan, candidates, sample() on the handful) and returns
// the token sample() would give over the whole vector, or null. cabeza() and
// muestreaCabeza() do the same from the head's weights and x, computing the
// logits on the way (one call for the GEMV and the top-k).
const estadisticasTopK = { gpu: 0, respaldo: 0, motivos: {} };
const ahoraMs = () => (typeof performance !== 'undefined' ? performance.now() : Date.now());

function createTopKGPU(device, ctx) {
  const out = device.createBuffer({ size: native.topkOutBytes(), label: 'topk.out' });
  let serie = 0;
  const stats = { gpu: 0, respaldo: 0, motivos: {} };
  const respaldo = (motivo) => {
    for (const s of [stats, estadisticasTopK]) {
      s.respaldo++;
      s.motivos[motivo] = (s.motivos[motivo] || 0) + 1;
    }
    return null;
  };
  async function candidatos(logits, base, vocab, plan) {
    if (vocab >= TOPK.N_MAX) return respaldo('vocabulario');
    serie = ((serie + 1) >>> 0) || 1;
    const esta = serie;
    const S = plan.S || new Uint32Array(0);
    const r = native.topk(device._ctx, logits._h, base, vocab, plan.M, S, esta, out._h);
    if (r === null) return respaldo('no aplica');
    const u = new Uint32Array(await readback(device, out, 0, out.size));
    const c = muestreo.leeSalidaTopK(u, { S }, Math.ceil(vocab / TOPK.POR_TROZO), esta);
    return c.motivo ? respaldo(c.motivo) : c;
  }
  // The head (model.js:1145-1177: the output projection of one token, then
  // candidatos() over its logits) as one call, eff_qgemv_topk. Resolves to
  // { logits, candidatos }: the logits always (a pooled buffer), the
  // candidates as candidatos() gives them, or null (then the caller reads the
  // logits as before).
  async function cabeza(type, wBuf, xBuf, vocab, k, plan) {
    const i = quantInfo(type);
    if (k % i.blockElems !== 0) throw new Error(`matmul ${type}: k=${k} no es múltiplo de ${i.blockElems}`);
    if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { bloques: vocab * (k / i.blockElems) }, 'matmul');
    const logits = ctx.alloc(vocab * 4, 'matmul.y');
    const soloLogits = (motivo) => {
      native.qmatmul(device._ctx, i.code, wBuf._h, xBuf._h, logits._h, vocab, k, 1);
      return { logits, candidatos: respaldo(motivo) };
    };
    if (vocab >= TOPK.N_MAX) return soloLogits('vocabulario');
    serie = ((serie + 1) >>> 0) || 1;
    const esta = serie;
    const S = plan.S || new Uint32Array(0);
    const r = native.qgemvTopk(device._ctx, i.code, wBuf._h, xBuf._h, logits._h, vocab, k, plan.M, S, esta, out._h);
    if (r === null) return soloLogits('no aplica');   // nothing was enqueued
    const u = new Uint32Array(await readback(device, out, 0, out.size));
    const c = muestreo.leeSalidaTopK(u, { S }, Math.ceil(vocab / TOPK.POR_TROZO), esta);
    return { logits, candidatos: c.motivo ? respaldo(c.motivo) : c };
  }
  return {
    stats,
    candidatos,
    cabeza,
    // `opts` as for sample() without `previos`, which comes in two halves
    // (the prompt and the generated ids). Resolves to { id, msLectura,
    // msMuestreo }, or null: then the caller reads the whole vector.
    async muestrea(logits, base, vocab, opts, previosA, previosB) {
      const t0 = ahoraMs();
      const plan = muestreo.planTopK(vocab, opts, previosA, previosB);
      if (!plan) return respaldo('muestreo sin tope');
      const c = await candidatos(logits, base, vocab, plan);
      if (!c) return null;
      const t1 = ahoraMs();
      const id = muestreo.muestraCandidatos(plan, c.ids, c.bits, c.bitsS, opts);
      if (id === null) return respaldo('incoherente');
      stats.gpu++; estadisticasTopK.gpu++;
      return { id, msLectura: t1 - t0, msMuestreo: ahoraMs() - t1 };
    },
    // muestrea() over the head: resolves to { logits, id, msLectura,
    // msMuestreo }, id null when the caller has to sample the logits itself.
    async muestreaCabeza(type, wBuf, xBuf, vocab, k, opts, previosA, previosB) {
      const t0 = ahoraMs();
      const plan = muestreo.planTopK(vocab, opts, previosA, previosB);
      if (!plan) {
        const i = quantInfo(type);
        if (k % i.blockElems !== 0) throw new Error(`matmul ${type}: k=${k} no es múltiplo de ${i.blockElems}`);
        if (TIPOS_R.has(type)) compruebaBufferR(type, wBuf, { bloques: vocab * (k / i.blockElems) }, 'matmul');
        const logits = ctx.alloc(vocab * 4, 'matmul.y');
        native.qmatmul(device._ctx, i.code, wBuf._h, xBuf._h, logits._h, vocab, k, 1);
        respaldo('muestreo sin tope');
        return { logits, id: null };
      }
      const { logits, candidatos: c } = await cabeza(type, wBuf, xBuf, vocab, k, plan);
      if (!c) return { logits, id: null };
      const t1 = ahoraMs();
      const id = muestreo.muestraCandidatos(plan, c.ids, c.bits, c.bitsS, opts);
      if (id === null) {
        respaldo('incoherente');
        return { logits, id: null };
      }
      stats.gpu++; estadisticasTopK.gpu++;
      return { logits, id, msLectura: t1 - t0, msMuestreo: ahoraMs() - t1 };
    },
    destroy() { out.destroy(); },
  };
}

module.exports = {
  native, STATUS, OPT, GEMV_MODE, TOPK, QUANT_TYPES, quantInfo,
  requestDevice, readback, createContext,
  createQuantOps, createGemvOps, GEMV2_TIPOS, GEMV2_MAX_TOKENS, createGemm2Ops, GEMM2_TIPOS, createFusionOps, createTopKGPU, estadisticasTopK, TIPOS_GATHER_NORMA,
  TIPOS_R, TIPO_R, TIPO_GGUF, bytesReordenado, bytesBufferR, bloquesDeBuffer, escalasDesde,
  reordena, vuelveAlGGUF, marcaBufferR, bloquesR, compruebaBufferR, creaBufferR,
  tensorBytes, comoReordenado, subeReordenadoPorTrozos, cargaTensores,
  sample: muestreo.sample, topKIndices: muestreo.topKIndices, uniforme: muestreo.uniforme,
  planTopK: muestreo.planTopK, leeSalidaTopK: muestreo.leeSalidaTopK, muestraCandidatos: muestreo.muestraCandidatos,
  quantize: (type, f32) => native.quantize(quantInfo(type).code, f32),
  fillNormal: (seed, sigma, n) => native.fillNormal(seed, sigma, n),
};
