'use strict';
// GPU run of the JavaScript load path: reads a tensor table and a data file
// written by tests/test_gpu_load.py, loads them through cargaTensores with and
// without the repack switch, and writes every device buffer back to disk for
// the Python side to compare byte for byte.
const assert = require('assert');
const fs = require('fs');
const path = require('path');
const eff = require(path.join(__dirname, '..', '..', 'elffuss-engine_amd', 'js', 'index.js'));

// A ranged handle over a file ({size, slice(offset, length)}), as the engine
// builds one over a File or an HTTP server; `corto` drops the last byte of
// every read of more than `corto` bytes.
function rangedDe(file, corto) {
  const fd = fs.openSync(file, 'r');
  const size = fs.fstatSync(fd).size;
  return {
    size,
    slice(off, len) {
      let n = Math.max(0, Math.min(len, size - off));
      if (corto && n > corto) n -= 1;
      const b = Buffer.alloc(n);
      fs.readSync(fd, b, 0, n, off);
      return Promise.resolve(b.buffer.slice(b.byteOffset, b.byteOffset + n));
    },
    close() { fs.closeSync(fd); },
  };
}

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
  const ranged = rangedDe(path.join(dir, meta.file));
  const x = leeF32(path.join(dir, meta.gemv.x));
  const xBuf = ops.upload(x, 'x');
  const out = {};
  for (const reorden of [false, true]) {
    const modo = reorden ? 'r' : 'plano';
    const prog = [];
    const { pesos, stats } = await eff.cargaTensores(device, ranged, meta.tensores, {
      reorden, tramo: meta.tramo, trozo: meta.trozo, onProgress: (u, tot, n) => prog.push([u, tot, n]),
    });
    const o = { stats, prog, tensores: {} };
    for (const t of meta.tensores) {
      const { buf, t: d } = pesos.get(t.name);
      const bytes = new Uint8Array(await eff.readback(device, buf, 0, buf.size));
      fs.writeFileSync(path.join(dir, `${modo}.${t.name}.bin`), bytes);
      const n = eff.bloquesR(buf);
      o.tensores[t.name] = { size: buf.size, typeName: d.typeName, typeNameGGUF: d.typeNameGGUF || null,
        bloquesR: n === undefined ? null : n };
      // the file's descriptor is left as it was
      assert.strictEqual(t.typeName, meta.tensores.find((u) => u.name === t.name).typeName);
    }
    const g = pesos.get(meta.gemv.name);
    const y = await ops.matmul(g.t.typeName, g.buf, xBuf, meta.gemv.rows, meta.gemv.k, 1);
    o.gemv = Array.from(new Float32Array(await eff.readback(device, y, 0, meta.gemv.rows * 4)));
    out[modo] = o;
    for (const { buf } of pesos.values()) buf.destroy();
  }

  // tensorBytes agrees with the table for every tensor
  for (const t of meta.tensores) assert.strictEqual(eff.tensorBytes(t.dims, t.typeName), t.nBytes);
  assert.strictEqual(eff.tensorBytes([256], 'Q5_K'), 0);

  // a type without a kernel stops the load before a byte moves
  const conQ5 = meta.tensores.concat([Object.assign({}, meta.tensores[0], { name: 'otro', typeName: 'Q5_K' })]);
  await assert.rejects(eff.cargaTensores(device, ranged, conQ5, {}), /sin kernel: Q5_K \(p\.ej\. «otro»\)/);
  // a short read is an error, in a span and in a chunk
  const corto = rangedDe(path.join(dir, meta.file), 100);
  await assert.rejects(eff.cargaTensores(device, corto, meta.tensores.slice(0, 2), { tramo: meta.tramo, trozo: meta.trozo }),
    /tramo incompleto/);
  const grande = meta.tensores.find((t) => t.name === meta.gemv.name);
  await assert.rejects(eff.cargaTensores(device, corto, [grande], { tramo: meta.tramo, trozo: meta.trozo }),
    /trozo incompleto/);
  await assert.rejects(eff.cargaTensores(device, corto, [grande], { reorden: true, tramo: meta.tramo, trozo: meta.trozo }),
    /trozo incompleto/);
  corto.close();
  // chunks past the tensor, and a buffer without the mark
  const bR = eff.creaBufferR(device, grande, 'Q8_0R');
  const N = grande.nElements / 32;
  assert.throws(() => eff.native.bufWriteR(device._ctx, bR._h, eff.QUANT_TYPES.Q8_0R.code, N - 1, new Uint8Array(68)),
    (e) => e.code === eff.STATUS.E_BOUNDS);
  const sinMarca = device.createBuffer({ size: eff.bytesBufferR('Q8_0R', N), label: 'sin marca' });
  assert.throws(() => eff.native.bufWriteR(device._ctx, sinMarca._h, eff.QUANT_TYPES.Q8_0R.code, 0, new Uint8Array(34)),
    (e) => e.code === eff.STATUS.E_MARK);
  await assert.rejects(eff.subeReordenadoPorTrozos({ device, ranged, t: grande, buf: bR, tipoR: 'Q8_0', trozo: 1000 }),
    /no es un tipo reordenado/);
  bR.destroy();
  sinMarca.destroy();
  ranged.close();

  fs.writeFileSync(path.join(dir, 'out.json'), JSON.stringify(out));
  device.destroy();
  console.log('shim_carga ok');
}
main().catch((e) => { console.error(e); process.exit(1); });
