'use strict';
// Writes every registry case of the Node host (inputs, params, expected) under argv[2] so the
// Python side can hold the JS known answers to the C oracle (tests/test_node_host.py). No device.
const fs = require('fs');
const path = require('path');
const h = require(path.join(__dirname, '..', '..', 'gemma4-webgpu-engine_amd', 'host', 'index.js'));

const dir = process.argv[2];
const index = [];
for (const name of h.kernelNames()) {
  h.KERNELS[name].cases.forEach((c, ci) => {
    const tag = `${name}.${ci}`;
    const inputs = {};
    for (const key of Object.keys(c.inputs)) {
      const v = c.inputs[key];
      if (!ArrayBuffer.isView(v)) continue;
      const file = `${tag}.${key}`;
      fs.writeFileSync(path.join(dir, file), Buffer.from(v.buffer, v.byteOffset, v.byteLength));
      inputs[key] = { file, type: v.constructor.name };
    }
    const file = `${tag}.expected`;
    fs.writeFileSync(path.join(dir, file), Buffer.from(c.expected.buffer, c.expected.byteOffset, c.expected.byteLength));
    index.push({ kernel: name, case: c.name, params: c.params, inputs,
      expected: { file, type: c.expected.constructor.name } });
  });
}
fs.writeFileSync(path.join(dir, 'cases.json'), JSON.stringify(index));
console.log(`dumped ${index.length} cases`);
