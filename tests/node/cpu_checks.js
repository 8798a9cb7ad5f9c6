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
  'ple-gather-4bit-sliced', 'qgemv-4bit-gelu', 'qgemv-8bit-gelu', 'qgemv-4bit-gelu-exact-split',
  'qgemv-4bit-gelu-m2', 'qgemv-8bit-gelu-m2', 'ple-gate-split', 'ple-fold-projection', 'gelu-mul'])
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

// the PLE split pair and the wide gelu forms refuse with the reference's messages (pleSplit.ts:
// 11-15, 58-59; qgemvWide.ts:522-526; execute.ts:881) before any device call
const f32b = { addr: 4096, bytes: 4096, kind: h.KIND.f32 };
throwsWith(() => h.setPleGateSplits(3), 'PLE splits must be 1, 2, 4 or 8');
throwsWith(() => h.bind('ple-gate-split', { inputs: { wq: fake, scales: fake, x: f32b }, output: f32b, params: { k: 1536, numRows: 250, inScale: 0.05 } }), 'PLE split row count must be divisible by four');
throwsWith(() => h.bind('ple-gate-split', { inputs: { wq: fake, scales: fake, x: f32b }, output: f32b, params: { k: 1536, numRows: 256, inScale: 0 } }), 'PLE split needs calibrated input');
throwsWith(() => h.bind('ple-fold-projection', { inputs: { wq: fake, scales: fake, gate: f32b, up: f32b }, output: f32b, params: {} }), 'needs inputs named wq, scales, gate, up, gateScales');
throwsWith(() => h.bind('qgemv-8bit-gelu-m2', { inputs: { wq: fake, scales: fake, gate: f32b, up: f32b }, output: { addr: 4096, kind: h.KIND.i8 }, params: { k: 256, numRows: 8, cols: 3, inScale: 0.05, outScale: 0.1 } }), 'needs params.cols in 1..2, got 3');
throwsWith(() => h.bind('gelu-mul', { inputs: { gate: f32b, up: f32b }, output: f32b, params: { count: 6 } }), 'gelu-mul needs params.count a positive multiple of 4, got 6');
assert.strictEqual(h.pleGateSplits(), 1);

// the 4-bit geometry's inner loop (qgemv.ts:146, 239-241): classic by default, tile8u selectable,
// anything else refused; the tile layout's size is ceil(N / 8) tiles of K words
assert.strictEqual(h.gemvInner(4), 'classic');
throwsWith(() => h.setGemvInner(4, 'tile16u'), 'inner must be classic or tile8u');
throwsWith(() => h.setGemvInner(2, 'tile8u'), 'bits must be 4 or 8');
h.setGemvInner(4, 'tile8u');
assert.strictEqual(h.gemvInner(4), 'tile8u');
h.setGemvInner(4, 'classic');
assert.strictEqual(h.tile8uBytes(1536, 77), 10 * 1536 * 4);

// every name a plan binds on the projection path is registered (plan.ts:487-665 through
// execute.ts's resolution): a decode step with the split PLE gate and the producer down split, a
// verify pass of two tokens, batched projections, and a prefill chunk; and what resolveStep
// refuses is refused the same way
const planned = (geometry, options, slices) => {
  const names = h.planProjectionKernels(geometry, options, slices);
  for (const n of names) assert.ok(h.kernelNames().includes(n), `${n} (${JSON.stringify(options)}, tokens ${geometry.tokens})`);
  return names;
};
const splitPle = planned({ mode: 'gemv', tokens: 1 }, { pleGateKSplits: 2, producerDownKSplits: 2 }, 5);
for (const n of ['ple-gate-split', 'ple-fold-projection', 'qgemv-4bit-gelu-exact-split', 'qgemv-exact-merge', 'ple-gather-4bit-sliced', 'qgemv-4bit'])
  assert.ok(splitPle.includes(n), n);
const verify = planned({ mode: 'gemv', tokens: 2 }, {}, 1);
for (const n of ['qgemv-4bit-m2', 'qgemv-8bit-m2', 'qgemv-4bit-gelu-m2', 'qgemv-8bit-gelu-m2', 'ple-gather-4bit'])
  assert.ok(verify.includes(n), n);
assert.ok(!verify.includes('qgemv-4bit'));
const batched = planned({ mode: 'gemv', tokens: 1 }, { batchProjections: true, pleGateKSplits: 8 });
for (const n of ['qkv-batch-4bit', 'gate-up-batch-4bit', 'qgemv-4bit-gelu', 'ple-fold-projection'])
  assert.ok(batched.includes(n), n);
const prefill = planned({ mode: 'gemm', tokens: 64 }, { pleGateKSplits: 2 });
for (const n of ['qgemm-4bit', 'qmatmul-8bit', 'gelu-mul']) assert.ok(prefill.includes(n), n);
assert.ok(!prefill.includes('ple-gate-split'));  // prefill never splits (plan.ts:633)
planned({ mode: 'gemv', tokens: 2 }, { attnKSplits: 2 });  // the wide pass drops the q/k/v split
throwsWith(() => h.planProjectionKernels({ mode: 'gemv', tokens: 2 }, { pleGateKSplits: 2 }), 'PLE split needs one token');
throwsWith(() => h.planProjectionKernels({ mode: 'gemv', tokens: 2 }, { producerDownKSplits: 2 }), 'producer split needs one token');
throwsWith(() => h.planProjectionKernels({ mode: 'gemv', tokens: 2 }, { batchProjections: true }), 'batched projections require a single token');
// the PLE split kernels' cases follow the active split count (pleSplit.ts:43-49)
h.setPleGateSplits(8);
assert.strictEqual(h.KERNELS['ple-gate-split'].cases[0].expected.length, 8 * 8);
assert.ok(h.KERNELS['ple-fold-projection'].cases[0].name.includes('fold-8'));
h.setPleGateSplits(1);
assert.strictEqual(h.KERNELS['ple-gate-split'].cases[0].expected.length, 8 * 2);

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
for (const n of ['qgemv-4bit-gelu-m2', 'qgemv-8bit-gelu-m2', 'ple-fold-projection', 'gelu-mul'])
  for (const c of h.KERNELS[n].cases) assert.ok(c.expected.some(v => v !== 0), `${n}/${c.name}`);
assert.ok(h.KERNELS['ple-gather-4bit-sliced'].cases[0].expected.some(v => v !== 0));
assert.strictEqual(typeof h.Stream, 'function');
assert.strictEqual(typeof h.Decoder, 'function');
console.log('node host cpu checks ok');
