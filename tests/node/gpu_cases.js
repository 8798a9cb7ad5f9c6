'use strict';
// Every registry kernel's known-answer cases on the GPU through the Node host (runCases, on a
// stream of its own), qgemv-4bit's again on the tile8u geometry, then the asynchronous boundary: a bind enqueued on a stream and read back by
// downloadAsync, with the event loop shown to run while the device works. Prints one JSON line.
const path = require('path');
const h = require(path.join(__dirname, '..', '..', 'gemma4-webgpu-engine_amd', 'host', 'index.js'));

async function main() {
  h.setDevice(0);
  const stream = new h.Stream();
  const results = h.runCases(null, stream);
  const failed = results.filter(r => !r.ok);
  console.log(`registry cases: ${results.length} run, ${failed.length} failed`);
  // async: the config-0 shape on the stream, awaited without blocking the loop
  const c = h.KERNELS['qgemv-4bit'].cases[1];
  const inputs = {};
  for (const k of Object.keys(c.inputs)) inputs[k] = h.DeviceBuffer.from(c.inputs[k]);
  const out = new h.DeviceBuffer(c.expected.byteLength, h.KIND.i8);
  out.fill(0x7b, stream);
  h.bind('qgemv-4bit', { inputs, output: out, params: c.params, stream });
  let ticks = 0;
  const timer = setInterval(() => { ticks += 1; }, 0);
  const pending = out.downloadAsync(stream);
  const got = new Int8Array(await pending);
  await stream.synchronizeAsync();
  clearInterval(timer);
  let asyncOk = got.every((v, i) => v === c.expected[i]);
  // the same bind captured into a graph and replayed (the reference's cached per-token encode)
  const graph = new h.Graph(stream, () => h.bind('qgemv-4bit', { inputs, output: out, params: c.params, stream }));
  for (let rep = 0; rep < 3; ++rep) {
    out.fill(0x7b, stream);
    graph.launch();
    const again = new Int8Array(await out.downloadAsync(stream));
    asyncOk = asyncOk && again.every((v, i) => v === c.expected[i]);
  }
  graph.destroy();
  // qgemv-4bit's known-answer cases (exact-grid fixtures: every order is exact) on the tile8u
  // geometry: the row-layout wq repacked into the eight-row tile layout, bound under
  // setGemvInner(4, 'tile8u'); the split is refused there, as the reference's generator does
  let tileOk = true;
  h.setGemvInner(4, 'tile8u');
  try {
    for (const tc of h.KERNELS['qgemv-4bit'].cases) {
      const ins = {};
      for (const key of Object.keys(tc.inputs)) ins[key] = h.DeviceBuffer.from(tc.inputs[key]);
      const tw = new h.DeviceBuffer(h.tile8uBytes(tc.params.k, tc.params.numRows), h.KIND.f32);
      h.tile8uRepack(ins.wq, tw, tc.params.k, tc.params.numRows, stream);
      const o = new h.DeviceBuffer(tc.expected.byteLength, tc.expected instanceof Int8Array ? h.KIND.i8 : h.KIND.f32);
      o.fill(0x7b, stream);
      h.bind('qgemv-4bit', { inputs: { wq: tw, scales: ins.scales, x: ins.x }, output: o, params: tc.params, stream });
      const got = new Uint8Array(await o.downloadAsync(stream));
      const want = new Uint8Array(tc.expected.buffer, tc.expected.byteOffset, tc.expected.byteLength);
      const same = got.every((v, i) => v === want[i]);
      if (!same) console.log(`tile8u case ${tc.name} differs`);
      tileOk = tileOk && same;
      let refused = false;
      try {
        h.bind('qgemv-4bit-split', { inputs: ins, output: o, params: { ...tc.params, kSplits: 2 }, stream });
      } catch (e) {
        refused = /tile8u has no K split/.test(e.message);
      }
      tileOk = tileOk && refused;
      Object.values(ins).forEach(b => b.free());
      tw.free();
      o.free();
    }
  } finally {
    h.setGemvInner(4, 'classic');
  }
  console.log(`tile8u geometry: ${tileOk ? 'ok' : 'FAILED'}`);
  // a refused copy (a NULL address, refused on the host when the copy is enqueued at the call)
  // throws with the library's message
  let rejected = null;
  try {
    await h.addon().downloadAsync(0, 64, stream.handle);
  } catch (e) {
    rejected = e.message;
  }
  Object.values(inputs).forEach(b => b.free());
  out.free();
  stream.destroy();
  console.log(JSON.stringify({ cases: results.length, failed, asyncOk, tileOk, rejected: rejected !== null }));
  if (failed.length || !asyncOk || !tileOk || rejected === null) process.exit(1);
}
main().catch(e => { console.error(e); process.exit(1); });
