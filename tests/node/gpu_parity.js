'use strict';
// Runs registry kernels through the Node host on the GPU: reads a manifest of cases (inputs as raw
// little-endian files) from argv[2], writes every output to <dir>/<case>.out. The Python side
// (tests/test_node_host.py) builds the inputs and checks the outputs against the oracle.
const fs = require('fs');
const path = require('path');
const h = require(path.join(__dirname, '..', '..', 'gemma4-webgpu-engine_amd', 'host', 'index.js'));

const dir = process.argv[2];
const manifest = JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
h.setDevice(0);
function load(file, kind) {
  const buf = fs.readFileSync(path.join(dir, file));
  const b = new h.DeviceBuffer(buf.length, kind);
  b.upload(new Uint8Array(buf.buffer, buf.byteOffset, buf.length));
  return b;
}
for (const c of manifest.cases) {
  console.log(`node case ${c.name} (${c.kernel})`);
  const inputs = {};
  for (const [name, spec] of Object.entries(c.inputs)) inputs[name] = load(spec.file, h.KIND[spec.kind]);
  const output = new h.DeviceBuffer(c.output.bytes, h.KIND[c.output.kind]);
  output.fill(0x7b);  // sentinel: unwritten outputs cannot pass
  if (c.kernel === 'plan') {
    const items = c.items.map(it => ({
      wq: inputs[it.wq], scales: inputs[it.scales], x: inputs[it.x], dst: output, bits: it.bits,
      k: it.k, numRows: it.numRows, inScale: it.inScale, outScale: it.outScale,
    }));
    const plan = new h.GemvPlan(items);
    plan.launch();
    h.synchronize();
    plan.destroy();
  } else {
    h.bind(c.kernel, { inputs, output, params: c.params });
    h.synchronize();
  }
  fs.writeFileSync(path.join(dir, `${c.name}.out`), Buffer.from(output.download()));
  output.free();
  for (const b of Object.values(inputs)) b.free();
}
console.log('node gpu cases done');
