'use strict';
// CPU checks of the Node host (no device calls): registry names and refusals, the execute.ts
// routing mirror, and the split planner's known answers (tableSplit.ts:13-77).
const assert = require('assert');
const path = require('path');
const h = require(path.join(__dirname, '..', '..', 'gemma4-webgpu-engine_amd', 'host', 'index.js'));

function throwsWith(fn, fragment) {
  let msg = null;
  try { fn(); } catch (e) { msg = e.message; }
  assert.ok(msg !== null, `expected a throw containing "${fragment}"`);
  assert.ok(msg.includes(fragment), `"${msg}" does not contain "${fragment}"`);
}

// registry
for (const n of ['qgemv-4bit', 'qgemv-8bit', 'qgemv-4bit-m2', 'qgemm-4bit', 'qmatmul-8bit',
  'qkv-batch-4bit', 'gate-up-batch-4bit', 'qgemv-merge', 'qgemv-exact-merge', 'ple-gather-4bit',
  'ple-gather-4bit-sliced', 'qgemv-4bit-gelu', 'qgemv-8bit-gelu', 'qgemv-4bit-gelu-exact-split'])
  assert.ok(h.kernelNames().includes(n), n);
throwsWith(() => h.bind('qgemv-4bit-gelu', { inputs: { wq: { addr: 1 } }, output: {}, params: {} }), 'needs inputs named wq, scales, gate, up');
throwsWith(() => h.bind('qgemv-3bit', { inputs: {}, output: {}, params: {} }), 'no registered kernel named qgemv-3bit');
throwsWith(() => h.bind('qgemv-4bit', { inputs: { wq: { addr: 1 } }, output: {}, params: {} }), 'needs inputs named wq, scales, x');
throwsWith(() => h.bind('ple-gather-4bit-sliced', { inputs: { codes: { addr: 1, bytes: 4480 }, scales: { addr: 1 }, ids: { addr: 1 } }, output: { addr: 1 }, params: { slots: 4 } }), 'naming a non empty vocabulary range');
throwsWith(() => h.bind('gate-up-batch-4bit', { inputs: { x: {} }, output: {}, params: { outputIndex: 5 } }), 'invalid batch output index');
// C-side refusals before any device call (qgemv.ts:1305-1310 wording)
const fake = { addr: 4096, bytes: 4096, kind: h.KIND.f16 };
throwsWith(() => h.bind('qgemv-4bit', { inputs: { wq: fake, scales: fake, x: fake }, output: { addr: 4096, kind: h.KIND.i8 }, params: { k: 100, numRows: 8, inScale: 0.05, outScale: 0.1 } }), 'qgemv-4bit needs K a multiple of 256, got 100');
throwsWith(() => h.bind('qgemv-4bit-m2', { inputs: { wq: fake, scales: fake, x: fake }, output: { addr: 4096, kind: h.KIND.i8 }, params: { k: 256, numRows: 8, cols: 3, inScale: 0.05, outScale: 0.1 } }), 'needs params.cols in 1..2, got 3');

// routing (execute.ts:372-430)
const dec = { mode: 'gemv', tokens: 1 }, ver = { mode: 'gemv', tokens: 2 }, pre = { mode: 'gemm', tokens: 64 };
assert.strictEqual(h.matmulKernel(dec, 'qgemv-4bit'), 'qgemv-4bit');
assert.strictEqual(h.matmulKernel(ver, 'qgemv-4bit'), 'qgemv-4bit-m2');
assert.strictEqual(h.matmulKernel(pre, 'qgemv-4bit'), 'qgemm-4bit');
assert.strictEqual(h.matmulKernel({ mode: 'gemm', tokens: 1, singleTokenGemm: true }, 'qgemv-4bit'), 'qgemm-4bit-single');
assert.strictEqual(h.matmulKernel({ mode: 'gemm', tokens: 8, prefillGemm4Tile: 4 }, 'qgemv-4bit'), 'qgemm-4bit-prefill4');
assert.strictEqual(h.pleKernel(dec, 'qmatmul-8bit'), 'qgemv-8bit');
assert.strictEqual(h.pleKernel(ver, 'qmatmul-8bit'), 'qgemv-8bit-m2');
assert.strictEqual(h.pleKernel(pre, 'qmatmul-8bit'), 'qmatmul-8bit');
throwsWith(() => h.gemvWide({ mode: 'gemv', tokens: 3 }, 'qgemv-4bit'), 'a verify pass carries at most 2 positions, got 3');
const lp = h.linearParams({ mode: 'gemv', tokens: 2, scalars: { 'l0.q_proj.input_activation_scale': 0.05 } }, 'l0.q_proj', 1536, 2048);
assert.deepStrictEqual(lp, { k: 1536, numRows: 2048, inScale: 0.05, outScale: 0, cols: 2 });
assert.strictEqual(h.linearParams(pre, 'm', 1536, 6144).mCols, 64);

// planner known answers: 1 GiB limit -> first slice 1,073,694,720 bytes (tableSplit.ts:68-77)
const table = { rows: 262144, rowBytes: 4480, maxStorageBuffersPerShaderStage: 10 };
const gib = h.planTableSplit(Object.assign({}, table, { maxStorageBufferBindingSize: 2 ** 30, maxBufferSize: 2 ** 30, maxSliceBytes: 2 ** 30 }));
assert.strictEqual(gib.slices.length, 2);
assert.strictEqual(gib.slices[0].byteLength, 1073694720);
assert.strictEqual(gib.slices[1].rowCount, 262144 - 239664);
const floor = h.planTableSplit(Object.assign({}, table, { maxStorageBufferBindingSize: 128 * 2 ** 20, maxBufferSize: 2 ** 32 }));
assert.strictEqual(floor.slices.length, 9);
const big = h.planTableSplit(Object.assign({}, table, { maxStorageBufferBindingSize: 2 ** 32, maxBufferSize: 2 ** 32, maxSliceBytes: 2 ** 32 }));
assert.strictEqual(big.single, true);
const five = h.planTableSplit(Object.assign({}, table, { maxStorageBufferBindingSize: 2 ** 30, maxBufferSize: 2 ** 30 }));
assert.deepStrictEqual(five.slices.map(s => s.rowCount), [59904, 59904, 59904, 59904, 22528]);
assert.strictEqual(h.sliceForRow(five.slices, 59903), 0);
assert.strictEqual(h.sliceForRow(five.slices, 59904), 1);
assert.strictEqual(h.sliceForRow(five.slices, 262144), -1);
const disp = h.slicedGatherDispatches(five, 64);
assert.strictEqual(disp.length, 5);
assert.deepStrictEqual(disp[4].params, { slots: 64, sliceStartRow: 4 * 59904, sliceRowCount: 22528 });
// planGatherSplit (tableSplit.ts:257-287): nine code slices and one scale buffer at the floor
const ple = h.planGatherSplit('ple', 262144, 4480, 35, { maxStorageBufferBindingSize: 128 * 2 ** 20,
  maxBufferSize: 128 * 2 ** 20, maxStorageBuffersPerShaderStage: 10 });
assert.strictEqual(ple.codes.slices.length, 9);
assert.strictEqual(ple.scales.totalBytes, 36700160);
assert.strictEqual(ple.scalesSingle, true);
const tinyLim = h.planGatherSplit('ple', 262144, 4480, 35, { maxStorageBufferBindingSize: 16 * 2 ** 20,
  maxBufferSize: 16 * 2 ** 20, maxStorageBuffersPerShaderStage: 10 });
assert.strictEqual(tinyLim.scalesSingle, false);
assert.ok(tinyLim.note.includes('NOT fit in one binding'));

// every registry entry carries known-answer cases (registry.ts:106: at least one, or it is not
// registered), each with inputs, params and an expected output
for (const name of h.kernelNames()) {
  const k = h.KERNELS[name];
  assert.ok(Array.isArray(k.cases) && k.cases.length >= 1, name);
  for (const c of k.cases) {
    assert.ok(c.name && c.inputs && c.params && ArrayBuffer.isView(c.expected), `${name}/${c.name}`);
    assert.ok(c.expected.length > 0, `${name}/${c.name}`);
  }
}
// the gelu cases saturate tanh, so their expected codes are not all zero
assert.ok(h.KERNELS['qgemv-4bit-gelu'].cases[0].expected.some(v => v !== 0));
assert.ok(h.KERNELS['ple-gather-4bit-sliced'].cases[0].expected.some(v => v !== 0));
assert.strictEqual(typeof h.Stream, 'function');
assert.strictEqual(typeof h.Decoder, 'function');
console.log('node host cpu checks ok');
