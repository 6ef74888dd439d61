'use strict';
// Draw-level outputs of the host sampler for tests/test_js.py: uniforme(seed)
// for a list of seeds, and sample() over the cases of a JSON file. The Python
// side computes the expected values with its own mulberry32 and softmax CDF.
const fs = require('fs');
const path = require('path');
const eff = require(path.join(__dirname, '..', '..', 'elffuss-engine_amd', 'js', 'muestreo.js'));

const dir = process.argv[2];
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'sorteo.json'), 'utf8'));
const out = { uniforme: meta.seeds.map((s) => eff.uniforme(s)), tokens: [] };
for (const c of meta.cases) {
  out.tokens.push(eff.sample(Float32Array.from(c.logits), c.opts));
}
fs.writeFileSync(path.join(dir, 'sorteo_out.json'), JSON.stringify(out));
console.log('shim_sorteo ok');
