'use strict';
// Host-side cost of the JavaScript drop-in in a decode-style loop: per token,
// an 8 KiB x upload, a chain of `ops` quant.matmul calls (each one's output
// the next one's input, Q4_K 2048 x 2048, 1 token), one readback of the last
// output and ctx.recycle(), as the engine's forward does per token
// (model.js mm() over ops.js:827-1101, recycle at the end of the token).
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
  const t0 = ahora();
  let chk = 0;
  for (let i = 0; i < tokens; i++) chk += await token();
  const us = ahora() - t0;
  const after = device.stats();
  const out = {
    tokens, ops_per_token: porToken, us_per_token: us / tokens, us_per_op: us / (tokens * porToken),
    gemv_launches: after.gemv - before.gemv, pool_peak_bytes: ops.ctx.picoBytes, finite: Number.isFinite(chk),
  };
  ops.ctx.destroy();
  wBuf.destroy();
  device.destroy();
  console.log(JSON.stringify(out));
}
main().catch((e) => { console.error(e); process.exit(1); });
