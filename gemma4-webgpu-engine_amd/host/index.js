'use strict';
/*
 * Node host of the g4w8a8 C ABI: the reference's operator seam (src/kernels/registry.ts:108-119,
 * Kernel.bind) and the pure host pieces that feed it (src/execute.ts:349-430 linearParams / routing,
 * src/tableSplit.ts planTableSplit / sliceForRow, src/kernels/embedGather.ts:403-419 sliced
 * dispatches), written for Node 12 (ES2019, CommonJS). The kernels run on MI355X through the N-API
 * addon g4w8a8.node, which links libg4w8a8.so; there is no JavaScript or CPU fallback, so a missing
 * addon fails here, loudly.
 *
 * Buffers are device allocations: { addr, bytes, kind } (kind: KIND.f32 / f16 / i8 / i32). Kernel
 * params use the reference's names (k, numRows, inScale, outScale, cols, mCols, rows0.., slots,
 * sliceStartRow, sliceRowCount, ...). bind() enqueues and returns; synchronize() waits.
 */
const path = require('path');

let addon = null;
function g4() {
  if (addon === null) {
    const file = path.join(__dirname, 'g4w8a8.node');
    try {
      addon = require(file);
    } catch (e) {
      throw new Error(`g4w8a8: the N-API addon ${file} did not load (${e.message}); build it with ` +
        '`make -C gemma4-webgpu-engine_amd/host` after the library. There is no fallback.');
    }
  }
  return addon;
}

const KIND = { f32: 0, f16: 1, i8: 2, i32: 3 };
const KIND_OF_ARRAY = new Map([
  [Float32Array, KIND.f32], [Uint16Array, KIND.f16], [Int8Array, KIND.i8], [Uint8Array, KIND.i8],
  [Int32Array, KIND.i32],
]);

/** A device allocation owned by the caller (the reference's BufferManager owns buffers the same way). */
class DeviceBuffer {
  constructor(bytes, kind) {
    this.bytes = bytes;
    this.kind = kind === undefined ? KIND.i8 : kind;
    this.addr = g4().malloc(Math.max(1, bytes));
  }

  /** Upload a typed array; `kind` defaults from the array type (Uint16Array = f16 bits). */
  static from(array, kind) {
    const k = kind === undefined ? KIND_OF_ARRAY.get(array.constructor) : kind;
    if (k === undefined) throw new TypeError('DeviceBuffer.from: pass a kind for this array type');
    const b = new DeviceBuffer(array.byteLength, k);
    g4().upload(b.addr, array);
    return b;
  }

  upload(array) { g4().upload(this.addr, array); }
  download() { return g4().download(this.addr, this.bytes); }
  fill(byte) { g4().fill(this.addr, byte, this.bytes); }
  free() {
    if (this.addr) g4().free(this.addr);
    this.addr = 0;
  }
}

function need(inputs, names, who) {
  for (const n of names) {
    if (!inputs[n]) throw new Error(`${who} needs inputs named ${names.join(', ')}`);
  }
}
function num(params, key, dflt) {
  const v = params[key];
  return v === undefined || v === null ? dflt : v;
}

// ---- the registry seam ------------------------------------------------------------------------

function gemvKernel(bits, wide) {
  return ({ inputs, output, params }) => {
    need(inputs, ['wq', 'scales', 'x'], `qgemv-${bits}bit`);
    g4().qgemv(bits, inputs.wq.addr, inputs.scales.addr, inputs.x.addr, inputs.x.kind, output.addr,
      output.kind, num(params, 'k', 0), num(params, 'numRows', 0), wide ? num(params, 'cols', 1) : 1,
      num(params, 'inScale', 0), num(params, 'outScale', 0));
  };
}

function gemmKernel(bits) {
  return ({ inputs, output, params }) => {
    need(inputs, ['wq', 'scales', 'x'], bits === 4 ? 'qgemm-4bit' : 'qmatmul-8bit');
    g4().qgemm(bits, inputs.wq.addr, inputs.scales.addr, inputs.x.addr, inputs.x.kind, output.addr,
      output.kind, num(params, 'k', 0), num(params, 'numRows', 0), num(params, 'mCols', 1),
      num(params, 'inScale', 0), num(params, 'outScale', 0));
  };
}

// qkv-batch-4bit / gate-up-batch-4bit (projectionBatch.ts:85-128): the bound output is projection
// `outputIndex`; the others arrive as inputs out0.. .
function batchKernel(count) {
  return ({ inputs, output, params }) => {
    const outIndex = num(params, 'outputIndex', count - 1);
    if (outIndex < 0 || outIndex >= count) throw new Error('invalid batch output index');
    const idx = Array.from({ length: count }, (_, i) => i);
    const ws = idx.map(i => inputs[`w${i}`]);
    const ss = idx.map(i => inputs[`s${i}`]);
    const outs = idx.map(i => (i === outIndex ? output : inputs[`out${i}`]));
    if (!inputs.x || ws.concat(ss, outs).some(b => !b)) {
      throw new Error('batched projection is missing an input buffer');
    }
    g4().projectionBatch(4, count, ws.map(b => b.addr), ss.map(b => b.addr), inputs.x.addr,
      inputs.x.kind, outs.map(b => b.addr), output.kind, idx.map(i => num(params, `rows${i}`, 0)),
      idx.map(i => num(params, `inScale${i}`, 0)), idx.map(i => num(params, `outScale${i}`, 0)),
      num(params, 'k', 0));
  };
}

function splitKernel(bits) {
  return ({ inputs, output, params }) => {
    need(inputs, ['wq', 'scales', 'x'], `qgemv-${bits}bit-split`);
    g4().qgemvSplit(bits, inputs.wq.addr, inputs.scales.addr, inputs.x.addr, inputs.x.kind,
      output.addr, num(params, 'k', 0), num(params, 'numRows', 0), num(params, 'kSplits', 1),
      num(params, 'exact', 0) ? 1 : 0, num(params, 'inScale', 0));
  };
}

// qgemv-4bit-gelu / qgemv-8bit-gelu (qgemv.ts:1668-1696) and the gelu exact split (exactSplit.ts:
// 19-31): gate and up bound in place of x, upOffset selecting the per-layer row.
function geluKernel(bits, split) {
  const who = split ? `qgemv-${bits}bit-gelu-exact-split` : `qgemv-${bits}bit-gelu`;
  return ({ inputs, output, params }) => {
    need(inputs, ['wq', 'scales', 'gate', 'up'], who);
    const head = [bits, inputs.wq.addr, inputs.scales.addr, inputs.gate.addr, inputs.gate.kind,
      inputs.up.addr, inputs.up.kind, num(params, 'upOffset', 0), output.addr];
    const scales = [num(params, 'gateScale', 0), num(params, 'upScale', 0)];
    if (split) {
      g4().qgemvGeluSplit(...head, num(params, 'k', 0), num(params, 'numRows', 0),
        num(params, 'kSplits', 1), 1, num(params, 'inScale', 0), ...scales);
    } else {
      g4().qgemvGelu(...head, output.kind, num(params, 'k', 0), num(params, 'numRows', 0),
        num(params, 'inScale', 0), num(params, 'outScale', 0), ...scales);
    }
  };
}

const PLE_COLS = 8960; // PLE_ROW_VALUES (quant.ts:35-37)
const PLE_GROUP_SIZE = 256;

function gatherKernel(sliced) {
  const who = sliced ? 'ple-gather-4bit-sliced' : 'ple-gather-4bit';
  return ({ inputs, output, params }) => {
    need(inputs, ['codes', 'scales', 'ids'], who);
    const cols = num(params, 'cols', PLE_COLS);
    const group = num(params, 'groupSize', PLE_GROUP_SIZE);
    const slots = num(params, 'slots', 0) || 1;
    let start = 0;
    let count = Math.floor(inputs.codes.bytes / (cols / 2));
    if (sliced) {
      start = params.sliceStartRow;
      count = params.sliceRowCount;
      if (start === undefined || count === undefined || !(count > 0)) {
        throw new Error(`${who} needs params sliceStartRow and sliceRowCount naming a non empty vocabulary range`);
      }
    }
    g4().pleGather(inputs.codes.addr, inputs.scales.addr, inputs.scales.kind, inputs.ids.addr,
      output.addr, output.kind, slots, cols, group, cols / group, sliced ? 1 : 0, start, count);
  };
}

const KERNELS = {
  'qgemv-4bit': gemvKernel(4, false),
  'qgemv-8bit': gemvKernel(8, false),
  'qgemv-4bit-m2': gemvKernel(4, true),
  'qgemv-8bit-m2': gemvKernel(8, true),
  'qgemm-4bit': gemmKernel(4),
  'qgemm-4bit-single': gemmKernel(4),
  'qgemm-4bit-prefill4': gemmKernel(4),
  'qmatmul-8bit': gemmKernel(8),
  'qkv-batch-4bit': batchKernel(3),
  'gate-up-batch-4bit': batchKernel(2),
  'qgemv-4bit-gelu': geluKernel(4, false),
  'qgemv-8bit-gelu': geluKernel(8, false),
  'qgemv-4bit-gelu-exact-split': geluKernel(4, true),
  'qgemv-4bit-split': splitKernel(4),
  'qgemv-8bit-split': splitKernel(8),
  'qgemv-merge': ({ inputs, output, params }) => {
    if (!inputs.part) throw new Error('qgemv-merge needs an input named part');
    g4().qgemvMerge(inputs.part.addr, output.addr, output.kind, num(params, 'numRows', 0),
      num(params, 'kSplits', 0), num(params, 'outScale', 0));
  },
  'qgemv-exact-merge': ({ inputs, output, params }) => {
    need(inputs, ['part', 'scales'], 'qgemv-exact-merge');
    g4().qgemvExactMerge(inputs.part.addr, inputs.scales.addr, output.addr, output.kind,
      num(params, 'numRows', 0), num(params, 'kSplits', 0), num(params, 'inScale', 0),
      num(params, 'outScale', 0));
  },
  'ple-gather-4bit': gatherKernel(false),
  'ple-gather-4bit-sliced': gatherKernel(true),
};

/** Run registry kernel `name` with the reference's bind input ({inputs, output, params}). */
function bind(name, input) {
  const run = KERNELS[name];
  if (!run) throw Object.assign(new Error(`gemma4 engine: no registered kernel named ${name}`), { status: 2 });
  run(input);
  return { kernel: name };
}

// ---- pure host mirrors (execute.ts:349-430) ------------------------------------------------------

const GEMV_WIDE_COLS = 2; // qgemvWide.ts:71

/** linearParams (execute.ts:350-369): a missing calibration scalar reads 0 (uncalibrated). */
function linearParams(geometry, module, k, numRows) {
  const scalar = name => (geometry.scalars && geometry.scalars[name] !== undefined ? geometry.scalars[name] : 0);
  const params = {
    k,
    numRows,
    inScale: scalar(`${module}.input_activation_scale`),
    outScale: scalar(`${module}.output_activation_scale`),
  };
  if (geometry.mode === 'gemm') params.mCols = geometry.tokens;
  else if (geometry.tokens > 1) params.cols = geometry.tokens;
  return params;
}

/** gemvWide (execute.ts:383-390): a verify pass over more than one position takes the -m2 form. */
function gemvWide(geometry, kernel) {
  if (geometry.mode !== 'gemv' || geometry.tokens === 1 || !kernel.startsWith('qgemv-')) return kernel;
  if (geometry.tokens > GEMV_WIDE_COLS) {
    throw new Error(`gemma4 engine: a verify pass carries at most ${GEMV_WIDE_COLS} positions, got ${geometry.tokens}`);
  }
  return `${kernel}-m${GEMV_WIDE_COLS}`;
}

/** pleKernel (execute.ts:372-375): the I8 family is the GEMV on a decode step, the matmul over a chunk. */
function pleKernel(geometry, stepKernel) {
  if (stepKernel !== 'qmatmul-8bit') return gemvWide(geometry, stepKernel);
  return geometry.mode === 'gemv' ? gemvWide(geometry, 'qgemv-8bit') : stepKernel;
}

/** matmulKernel (execute.ts:406-430) for the projection families on this path. */
function matmulKernel(geometry, stepKernel) {
  if (geometry.mode === 'gemm') {
    const kernel = stepKernel.startsWith('qgemv-') ? stepKernel.replace('qgemv-', 'qgemm-') : stepKernel;
    if (geometry.tokens === 1 && geometry.singleTokenGemm === true && kernel === 'qgemm-4bit') {
      return `${kernel}-single`;
    }
    if (geometry.tokens > 1 && geometry.prefillGemm4Tile === 4 && kernel === 'qgemm-4bit') {
      return 'qgemm-4bit-prefill4';
    }
    return kernel;
  }
  return gemvWide(geometry, stepKernel);
}

// ---- the split planner (tableSplit.ts) ----------------------------------------------------------

/** planTableSplit (tableSplit.ts:125-215), computed by the library (pure host code). */
function planTableSplit(input) { return g4().planTableSplit(input); }

/** sliceForRow (tableSplit.ts:218-223): the slice index carrying `row`, or -1. */
function sliceForRow(slices, row) {
  for (const s of slices) if (row >= s.startRow && row < s.startRow + s.rowCount) return s.index;
  return -1;
}

/** slicedGatherDispatches (embedGather.ts:403-419): one sliced gather per slice of the plan. */
function slicedGatherDispatches(plan, slots) {
  return plan.slices.map(s => ({
    kernel: 'ple-gather-4bit-sliced',
    slice: s.index,
    params: { slots, sliceStartRow: s.startRow, sliceRowCount: s.rowCount },
  }));
}

// ---- launches beyond the registry ---------------------------------------------------------------

/** A device-resident grouped GEMV over any number of projections (g4_qgemv_plan_*). */
class GemvPlan {
  constructor(items) {
    this.handle = g4().qgemvPlanCreate(items.map(it => ({
      wq: it.wq.addr, scales: it.scales.addr, x: it.x.addr, dst: it.dst.addr, bits: it.bits,
      xKind: it.x.kind, outKind: it.dst.kind, k: it.k, numRows: it.numRows, inScale: it.inScale,
      outScale: it.outScale,
    })));
  }

  launch() { g4().qgemvPlanLaunch(this.handle); }
  destroy() {
    if (this.handle) g4().qgemvPlanDestroy(this.handle);
    this.handle = 0;
  }
}

module.exports = {
  KIND,
  DeviceBuffer,
  KERNELS,
  kernelNames: () => Object.keys(KERNELS),
  bind,
  linearParams,
  gemvWide,
  pleKernel,
  matmulKernel,
  planTableSplit,
  sliceForRow,
  slicedGatherDispatches,
  GemvPlan,
  kernelForShape: (bits, m, n, k) => g4().kernelForShape(bits, m, n, k),
  deviceCount: () => g4().deviceCount(),
  setDevice: d => g4().setDevice(d),
  synchronize: () => g4().synchronize(),
  pleGatherSplit: (...args) => g4().pleGatherSplit(...args),
  addon: g4,
};
