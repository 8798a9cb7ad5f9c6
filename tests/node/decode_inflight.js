'use strict';
// Two decode steps in flight through the Node host: the model is filled on the device from a spec
// (argv[2]/spec.json: tensor names, shapes and seeds of the seeded synthetic model; rope tables as
// files), then step t and step t + 1 are enqueued back to back on one stream, the second reading
// the next-token buffer the first writes, with the positions set in stream order. Only then does
// the host wait, on asynchronous downloads. Outputs go to <dir>/*.out for the Python side.
const fs = require('fs');
const path = require('path');
const h = require(path.join(__dirname, '..', '..', 'gemma4-webgpu-engine_amd', 'host', 'index.js'));

async function main() {
  const dir = process.argv[2];
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));
  h.setDevice(0);
  const stream = new h.Stream();
  const bufs = {};
  for (const t of spec.tensors) {
    const n = t.shape.reduce((a, b) => a * b, 1);
    if (t.kind === 'u8') {
      bufs[t.name] = new h.DeviceBuffer(n, h.KIND.i8);
      h.addon().fillHashU8(bufs[t.name].addr, n, t.seed, stream.handle);
    } else if (t.kind === 'f32') {
      bufs[t.name] = new h.DeviceBuffer(4 * n, h.KIND.f32);
      h.addon().fillHashF32(bufs[t.name].addr, n, t.seed, t.lo, t.hi, stream.handle);
    } else {  // a host table (rope)
      const b = fs.readFileSync(path.join(dir, t.file));
      bufs[t.name] = h.DeviceBuffer.from(new Float32Array(b.buffer, b.byteOffset, b.length / 4));
    }
  }
  const addr = name => (bufs[name] ? bufs[name].addr : 0);
  const weights = {};
  for (const f of spec.model_fields) weights[f] = addr(f);
  weights.layer = [];
  for (let l = 0; l < spec.shape.layers; ++l) {
    const L = { layer_scalar: spec.layer_scalar[l] };
    for (const f of spec.layer_fields) L[f] = addr(`l${l}.${f}`);
    weights.layer.push(L);
  }
  const dec = new h.Decoder(spec.shape, weights);
  for (let p = 0; p < spec.shape.kv_producers; ++p) {
    const kv = dec.kv(p);
    h.addon().fillHashF32(kv.k, spec.kv_elems, spec.kv_seeds[p], -spec.kv_amplitude,
      spec.kv_amplitude, stream.handle);
  }
  const tokens = h.DeviceBuffer.from(new Int32Array(spec.tokens));
  const next0 = new h.DeviceBuffer(4 * spec.shape.batch, h.KIND.i32);
  const next1 = new h.DeviceBuffer(4 * spec.shape.batch, h.KIND.i32);
  // both steps enqueued before any wait: the second reads next0 on the device. Step t's logits
  // are requested (downloadAsync) before step t + 1 is enqueued, and step t + 1 rewrites the same
  // buffer: the copy must hold step t's values, so it has to be ordered at the call.
  const logits = dec.buffer('logits');
  const hidden = dec.buffer('hidden');
  dec.setPosition(spec.pos, stream);
  dec.step(tokens, next0, stream);
  const lg0p = h.addon().downloadAsync(logits.addr, logits.bytes, stream.handle);
  dec.setPosition(spec.pos + 1, stream);
  dec.step(next0, next1, stream);
  const [a, b, lg0, lg, hd] = await Promise.all([
    next0.downloadAsync(stream), next1.downloadAsync(stream), lg0p,
    h.addon().downloadAsync(logits.addr, logits.bytes, stream.handle),
    h.addon().downloadAsync(hidden.addr, hidden.bytes, stream.handle)]);
  fs.writeFileSync(path.join(dir, 'logits0.out'), Buffer.from(lg0));
  fs.writeFileSync(path.join(dir, 'next0.out'), Buffer.from(a));
  fs.writeFileSync(path.join(dir, 'next1.out'), Buffer.from(b));
  fs.writeFileSync(path.join(dir, 'logits1.out'), Buffer.from(lg));
  fs.writeFileSync(path.join(dir, 'hidden1.out'), Buffer.from(hd));
  dec.destroy();
  stream.destroy();
  console.log('decode in flight done');
}
main().catch(e => { console.error(e); process.exit(1); });
