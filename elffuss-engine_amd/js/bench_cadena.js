'use strict';
// Host-side cost of the JavaScript drop-in in a decode-style loop: per token,
// an 8 KiB x upload, a chain of `ops` quant.matmul calls (each one's output
// the next one's input, Q4_K 2048 x 2048, 1 token), one readback of the last
// output and ctx.recycle(), as the engine's forward does per token
// (model.js mm() over ops.js:827-1101, recycle at the end of the token).
// Two ways: every call issued eagerly, and the token's chain recorded once
// (ctx.grabaGrafo, the HIP-graph form of ctx.batch) and replayed per token.
// Prints one JSON line: wall microseconds per token and per operation.
//   node bench_cadena.js [tokens] [ops]
const path = require('path');
const eff = require(path.join(__dirname, 'index.js'));

async function main() {
  const tokens = parseInt(process.argv[2] || '200', 10);
  const porToken = parseInt(process.argv[3] || '30', 10);
  const rows = 2048, k = 2048;
  const device = await eff.requestDevice();
  const ops = eff.createQuantOps(device);
  const w = eff.quantize('Q4_K', eff.fillNormal(1, 0.02, rows * k));
  const wBuf = device.createBuffer({ size: Math.ceil((w.length + 4) / 4) * 4, label: 'w' });
  device.queue.writeBuffer(wBuf, 0, w);
  const x0 = eff.fillNormal(2, 1.0, k);
  const ahora = () => Number(process.hrtime.bigint()) / 1e3;
  const token = async () => {
    let x = ops.upload(x0, 'x');
    for (let i = 0; i < porToken; i++) x = await ops.matmul('Q4_K', wBuf, x, rows, k, 1);
    const v = new Float32Array(await eff.readback(device, x, 0, 16));
    ops.ctx.recycle();
    return v[0];
  };
  for (let i = 0; i < 10; i++) await token();   // warm-up: pool classes filled, kernels loaded
  const before = device.stats();
  let t0 = ahora();
  let chk = 0;
  for (let i = 0; i < tokens; i++) chk += await token();
  const us = ahora() - t0;
  const after = device.stats();

  // the same chain recorded once and replayed: x written into the recorded
  // input buffer, one launch of the recording, the readback
  const xIn = device.createBuffer({ size: k * 4, label: 'xin' });
  const g = await ops.ctx.grabaGrafo(async () => {
    let x = xIn;
    for (let i = 0; i < porToken; i++) x = await ops.matmul('Q4_K', wBuf, x, rows, k, 1);
    return x;
  });
  const tokenGrafo = async () => {
    device.queue.writeBuffer(xIn, 0, x0);
    g.lanza();
    const v = new Float32Array(await eff.readback(device, g.salida, 0, 16));
    ops.ctx.recycle();
    return v[0];
  };
  let chkG = 0;
  for (let i = 0; i < 10; i++) await tokenGrafo();
  t0 = ahora();
  for (let i = 0; i < tokens; i++) chkG += await tokenGrafo();
  const usG = ahora() - t0;
  const out = {
    tokens, ops_per_token: porToken, us_per_token: us / tokens, us_per_op: us / (tokens * porToken),
    graph: { us_per_token: usG / tokens, us_per_op: usG / (tokens * porToken), nodes: g.nodos,
      same_result: chkG === chk },
    gemv_launches: after.gemv - before.gemv, pool_peak_bytes: ops.ctx.picoBytes, finite: Number.isFinite(chk),
  };
  g.destroy();
  xIn.destroy();
  ops.ctx.destroy();
  wBuf.destroy();
  device.destroy();
  console.log(JSON.stringify(out));
}
main().catch((e) => { console.error(e); process.exit(1); });
