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

  upload(array, stream) { g4().upload(this.addr, array, streamHandle(stream)); }
  download(stream) { return g4().download(this.addr, this.bytes, streamHandle(stream)); }
  /** Promise<ArrayBuffer>: the copy waits on a worker thread, after the stream's queued work. */
  downloadAsync(stream) { return g4().downloadAsync(this.addr, this.bytes, streamHandle(stream)); }
  fill(byte, stream) { g4().fill(this.addr, byte, this.bytes, streamHandle(stream)); }
  free() {
    if (this.addr) g4().free(this.addr);
    this.addr = 0;
  }
}

/** A stream argument as the addon takes it: a Stream, a raw handle, or undefined (default). */
function streamHandle(stream) {
  if (stream === undefined || stream === null) return 0;
  return typeof stream === 'number' ? stream : stream.handle;
}

/**
 * A HIP stream (runtime.ts's queue). Work enqueued on one stream runs in order; synchronize()
 * blocks, synchronizeAsync() returns a Promise and leaves the event loop free.
 */
class Stream {
  constructor() { this.handle = g4().streamCreate(); }
  synchronize() { g4().streamSynchronize(this.handle); }
  synchronizeAsync() { return g4().synchronizeAsync(this.handle); }
  destroy() {
    if (this.handle) g4().streamDestroy(this.handle);
    this.handle = 0;
  }
}

/** A captured sequence of enqueues on a stream, replayed with one launch (the cached encode). */
class Graph {
  constructor(stream, record) {
    this.stream = stream;
    g4().graphBeginCapture(stream.handle);
    let ok = false;
    try {
      record();
      ok = true;
    } finally {
      const h = g4().graphEndCapture(stream.handle);
      this.handle = ok ? h : 0;
      if (!ok && h) g4().graphDestroy(h);
    }
  }

  launch(stream) { g4().graphLaunch(this.handle, streamHandle(stream || this.stream)); }
  destroy() {
    if (this.handle) g4().graphDestroy(this.handle);
    this.handle = 0;
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

// GemvGeometry.inner per bit width (qgemv.ts:146, 239-241; setGemvGeometry in the device profile):
// 'tile8u' makes the 4-bit pipeline the tile loop (qgemv.ts:440), whose wq is the eight-row tile
// layout (tile8uRepack). The 8-bit family has no tile loop and keeps the classic one.
const gemvInnerOf = { 4: 'classic', 8: 'classic' };
function gemvInner(bits) { return gemvInnerOf[bits]; }
function setGemvInner(bits, inner) {
  if (!(bits in gemvInnerOf)) throw new Error(`gemv geometry: bits must be 4 or 8, got ${bits}`);
  if (inner !== 'classic' && inner !== 'tile8u') {
    throw new Error(`gemv geometry: inner must be classic or tile8u on this build, got ${inner}`);
  }
  gemvInnerOf[bits] = inner;
}
const tile8u = bits => bits === 4 && gemvInnerOf[4] === 'tile8u';
function tile8uBytes(k, numRows) { return Math.ceil(numRows / 8) * k * 4; }
function tile8uRepack(wq, tileWq, k, numRows, stream) {
  g4().tile8uRepack(wq.addr, tileWq.addr, k, numRows, streamHandle(stream));
}
// qgemv-4bit (up null) or qgemv-4bit-gelu on the tile8u geometry (qgemv.ts:870-1015)
function qgemvTile8u(tileWq, scales, x, up, upOffsetElems, output, params, stream) {
  g4().qgemvTile8u(tileWq.addr, scales.addr, x.addr, x.kind, up ? up.addr : 0, up ? up.kind : 0,
    upOffsetElems, output.addr, output.kind, num(params, 'k', 0), num(params, 'numRows', 0),
    num(params, 'inScale', 0), num(params, 'outScale', 0), num(params, 'gateScale', 0),
    num(params, 'upScale', 0), streamHandle(stream));
}

function gemvKernel(bits, wide) {
  return ({ inputs, output, params, stream }) => {
    need(inputs, ['wq', 'scales', 'x'], `qgemv-${bits}bit`);
    if (!wide && tile8u(bits)) {
      qgemvTile8u(inputs.wq, inputs.scales, inputs.x, null, 0, output, params, stream);
      return;
    }
    g4().qgemv(bits, inputs.wq.addr, inputs.scales.addr, inputs.x.addr, inputs.x.kind, output.addr,
      output.kind, num(params, 'k', 0), num(params, 'numRows', 0), wide ? num(params, 'cols', 1) : 1,
      num(params, 'inScale', 0), num(params, 'outScale', 0), streamHandle(stream));
  };
}

function gemmKernel(bits) {
  return ({ inputs, output, params, stream }) => {
    need(inputs, ['wq', 'scales', 'x'], bits === 4 ? 'qgemm-4bit' : 'qmatmul-8bit');
    g4().qgemm(bits, inputs.wq.addr, inputs.scales.addr, inputs.x.addr, inputs.x.kind, output.addr,
      output.kind, num(params, 'k', 0), num(params, 'numRows', 0), num(params, 'mCols', 1),
      num(params, 'inScale', 0), num(params, 'outScale', 0), streamHandle(stream));
  };
}

// qkv-batch-4bit / gate-up-batch-4bit (projectionBatch.ts:85-128): the bound output is projection
// `outputIndex`; the others arrive as inputs out0.. .
function batchKernel(count) {
  return ({ inputs, output, params, stream }) => {
    const outIndex = num(params, 'outputIndex', count - 1);
    if (outIndex < 0 || outIndex >= count) throw new Error('invalid batch output index');
    const idx = Array.from({ length: count }, (_, i) => i);
    const ws = idx.map(i => inputs[`w${i}`]);
    const ss = idx.map(i => inputs[`s${i}`]);
    const outs = idx.map(i => (i === outIndex ? output : inputs[`out${i}`]));
    if (!inputs.x || ws.concat(ss, outs).some(b => !b)) {
      throw new Error('batched projection is missing an input buffer');
    }
    g4().projectionBatch(4, ws.map(b => b.addr), ss.map(b => b.addr), inputs.x.addr,
      inputs.x.kind, outs.map(b => b.addr), output.kind, idx.map(i => num(params, `rows${i}`, 0)),
      idx.map(i => num(params, `inScale${i}`, 0)), idx.map(i => num(params, `outScale${i}`, 0)),
      num(params, 'k', 0), streamHandle(stream));
  };
}

function splitKernel(bits) {
  return ({ inputs, output, params, stream }) => {
    need(inputs, ['wq', 'scales', 'x'], `qgemv-${bits}bit-split`);
    if (tile8u(bits)) throw new Error('qgemv-4bit tile8u has no K split yet');
    g4().qgemvSplit(bits, inputs.wq.addr, inputs.scales.addr, inputs.x.addr, inputs.x.kind,
      output.addr, num(params, 'k', 0), num(params, 'numRows', 0), num(params, 'kSplits', 1),
      num(params, 'exact', 0) ? 1 : 0, num(params, 'inScale', 0), streamHandle(stream));
  };
}

// qgemv-4bit-gelu / qgemv-8bit-gelu (qgemv.ts:1668-1696), their -m2 forms (qgemvWide.ts:660-709)
// and the gelu exact split (exactSplit.ts:19-31): gate and up bound in place of x. params.upOffset
// counts vec4s, as the reference's (qgemv.ts:398, execute.ts:886 layer * dim / 4); the addon takes
// elements.
function geluKernel(bits, split, wide) {
  const who = split ? `qgemv-${bits}bit-gelu-exact-split` : `qgemv-${bits}bit-gelu${wide ? '-m2' : ''}`;
  return ({ inputs, output, params, stream }) => {
    need(inputs, ['wq', 'scales', 'gate', 'up'], who);
    const head = [bits, inputs.wq.addr, inputs.scales.addr, inputs.gate.addr, inputs.gate.kind,
      inputs.up.addr, inputs.up.kind, 4 * num(params, 'upOffset', 0), output.addr];
    const scales = [num(params, 'gateScale', 0), num(params, 'upScale', 0)];
    if (split) {
      g4().qgemvGeluSplit(...head, num(params, 'k', 0), num(params, 'numRows', 0),
        num(params, 'kSplits', 1), 1, num(params, 'inScale', 0), ...scales, streamHandle(stream));
    } else if (!wide && tile8u(bits)) {
      qgemvTile8u(inputs.wq, inputs.scales, inputs.gate, inputs.up, 4 * num(params, 'upOffset', 0),
        output, params, stream);
    } else if (wide) {
      g4().qgemvGeluM2(...head, output.kind, num(params, 'k', 0), num(params, 'numRows', 0),
        num(params, 'cols', 0), num(params, 'inScale', 0), num(params, 'outScale', 0), ...scales,
        streamHandle(stream));
    } else {
      g4().qgemvGelu(...head, output.kind, num(params, 'k', 0), num(params, 'numRows', 0),
        num(params, 'inScale', 0), num(params, 'outScale', 0), ...scales, streamHandle(stream));
    }
  };
}

// pleGateSplits / setPleGateSplits (pleSplit.ts:10-15): the split count both PLE split kernels run,
// a module setting as in the reference (a device profile sets it); 1 runs as 2 (pleSplit.ts:16).
let pleSplits = 1;
function pleGateSplits() { return pleSplits; }
function setPleGateSplits(value) {
  if (![1, 2, 4, 8].includes(value)) throw new Error('PLE splits must be 1, 2, 4 or 8');
  pleSplits = value;
}
function pleActiveSplits() { return pleSplits === 1 ? 2 : pleSplits; }

// ple-gate-split (pleSplit.ts:50-63): exact 8-bit split partials, row-interleaved for the fold.
function pleGateSplitKernel({ inputs, output, params, stream }) {
  need(inputs, ['wq', 'scales', 'x'], 'ple-gate-split');
  g4().pleGateSplit(inputs.wq.addr, inputs.scales.addr, inputs.x.addr, inputs.x.kind, output.addr,
    num(params, 'k', 0), num(params, 'numRows', 0), pleSplits, num(params, 'inScale', 0),
    streamHandle(stream));
}

// ple-fold-projection (pleSplit.ts:64-84): gate (the partials), up, gateScales; gateInScale and
// gateOutScale are the gate linear's own scales.
function pleFoldProjectionKernel({ inputs, output, params, stream }) {
  need(inputs, ['wq', 'scales', 'gate', 'up', 'gateScales'], 'ple-fold-projection');
  g4().pleFoldProjection(inputs.wq.addr, inputs.scales.addr, inputs.gate.addr,
    inputs.gateScales.addr, pleSplits, num(params, 'gateInScale', 0),
    num(params, 'gateOutScale', 0), inputs.up.addr, inputs.up.kind, 4 * num(params, 'upOffset', 0),
    output.addr, output.kind, num(params, 'k', 0), num(params, 'numRows', 0),
    num(params, 'inScale', 0), num(params, 'outScale', 0), num(params, 'upScale', 0),
    streamHandle(stream));
}

// gelu-mul (geluMul.ts:250-278): the prefill chunk's separate pass over f32 gate and up.
function geluMulKernel({ inputs, output, params, stream }) {
  need(inputs, ['gate', 'up'], 'gelu-mul');
  g4().geluMulF32(inputs.gate.addr, inputs.up.addr, output.addr, num(params, 'count', 0),
    num(params, 'srqScale', 0), streamHandle(stream));
}

const PLE_COLS = 8960; // PLE_ROW_VALUES (quant.ts:35-37)
const PLE_GROUP_SIZE = 256;

function gatherKernel(sliced) {
  const who = sliced ? 'ple-gather-4bit-sliced' : 'ple-gather-4bit';
  return ({ inputs, output, params, stream }) => {
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
      output.addr, output.kind, slots, cols, group, cols / group, sliced ? 1 : 0, start, count,
      streamHandle(stream));
  };
}

const BINDS = {
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
  'qgemv-4bit-gelu-m2': geluKernel(4, false, true),
  'qgemv-8bit-gelu-m2': geluKernel(8, false, true),
  'qgemv-4bit-gelu-exact-split': geluKernel(4, true),
  'gelu-mul': geluMulKernel,
  'ple-gate-split': pleGateSplitKernel,
  'ple-fold-projection': pleFoldProjectionKernel,
  'qgemv-4bit-split': splitKernel(4),
  'qgemv-8bit-split': splitKernel(8),
  'qgemv-merge': ({ inputs, output, params, stream }) => {
    if (!inputs.part) throw new Error('qgemv-merge needs an input named part');
    g4().qgemvMerge(inputs.part.addr, output.addr, output.kind, num(params, 'numRows', 0),
      num(params, 'kSplits', 0), num(params, 'outScale', 0), streamHandle(stream));
  },
  'qgemv-exact-merge': ({ inputs, output, params, stream }) => {
    need(inputs, ['part', 'scales'], 'qgemv-exact-merge');
    g4().qgemvExactMerge(inputs.part.addr, inputs.scales.addr, output.addr, output.kind,
      num(params, 'numRows', 0), num(params, 'kSplits', 0), num(params, 'inScale', 0),
      num(params, 'outScale', 0), streamHandle(stream));
  },
  'ple-gather-4bit': gatherKernel(false),
  'ple-gather-4bit-sliced': gatherKernel(true),
};

// ---- known-answer cases (registry.ts:72-119: a kernel without cases is not registered) --------
//
// The reference's cases name manifest entries its excluded scripts generated; none ship. These are
// built from the reference's own fixture recipes instead (qgemv.ts:1365-1388: activations on the
// 1/8 grid, the scales 0.1875 / 0.015625 / 0.0625, ten rows against a workgroup of four, eleven
// columns against a tile of eight), so every product, sum and scale is a short dyadic rational
// that f32 holds exactly: the expected outputs below are computed in JS doubles with no rounding
// to argue about, and every case gates at zero (tolAbs 0, the registry's default).

function rng(seed) {  // mulberry32: deterministic case inputs
  let t = seed >>> 0;
  return () => {
    t = (t + 0x6D2B79F5) >>> 0;
    let r = Math.imul(t ^ (t >>> 15), 1 | t);
    r = (r + Math.imul(r ^ (r >>> 7), 61 | r)) ^ r;
    return ((r ^ (r >>> 14)) >>> 0) / 4294967296;
  };
}
function randInt(next, lo, hi) { return lo + Math.floor(next() * (hi - lo + 1)); }
const f32 = Math.fround;
/** srqCodes (quant.ts:309-334) on exact quotients: round half to even, clamp to int8. */
function snap(v, s) {
  const q = v / s;
  let r = Math.round(q);
  if (Math.abs(q % 1) === 0.5 && r % 2 !== 0) r -= 1;
  return Math.max(-128, Math.min(127, r));
}
const GRID_SCALES = [0.1875, 0.015625, 0.0625];

/** Weights (packed bytes and codes), scales and x [cols][k] on the grid. */
function gridOperands(seed, bits, rows, k, cols) {
  const next = rng(seed);
  const codes = new Int8Array(rows * k);
  for (let i = 0; i < codes.length; ++i) codes[i] = bits === 4 ? randInt(next, -8, 7) : randInt(next, -127, 127);
  let wq;
  if (bits === 4) {
    wq = new Uint8Array(rows * k / 2);
    for (let i = 0; i < wq.length; ++i) wq[i] = ((codes[2 * i] + 8) & 15) | (((codes[2 * i + 1] + 8) & 15) << 4);
  } else {
    wq = new Uint8Array(codes.buffer.slice(0));
  }
  const scales = new Float32Array(rows);
  for (let r = 0; r < rows; ++r) scales[r] = GRID_SCALES[r % 3];
  const x = new Float32Array(cols * k);
  for (let i = 0; i < x.length; ++i) x[i] = randInt(next, -16, 16) / 8;
  return { codes, wq, scales, x };
}

/** qgemvOracle (qgemv.ts:1131-1176) on the grid: dst[col * rows + row], f32 (q * out) or int8 q. */
function gridExpected(op, rows, k, cols, inScale, outScale, kind) {
  const out = kind === KIND.i8 ? new Int8Array(cols * rows) : new Float32Array(cols * rows);
  for (let c = 0; c < cols; ++c) {
    for (let r = 0; r < rows; ++r) {
      let sum = 0;
      for (let i = 0; i < k; ++i) {
        const x = op.x[c * k + i];
        sum += op.codes[r * k + i] * (inScale !== 0 ? snap(x, inScale) : x);
      }
      const y = f32(f32((inScale !== 0 ? inScale : 1) * op.scales[r]) * sum);
      const q = outScale !== 0 ? snap(y, outScale) : null;
      out[c * rows + r] = kind === KIND.i8 ? q : (q === null ? y : q * outScale);
    }
  }
  return out;
}

function linearCase(name, seed, bits, rows, k, cols, inScale, outScale, kind, paramsExtra) {
  const op = gridOperands(seed, bits, rows, k, cols);
  const params = Object.assign({ k, numRows: rows, inScale, outScale }, paramsExtra || {});
  return {
    name,
    inputs: { wq: op.wq, scales: op.scales, x: op.x },
    params,
    expected: gridExpected(op, rows, k, cols, inScale, outScale, kind),
    note: 'the qgemv.ts:1365-1388 exact-grid recipe: exact in f32, so it gates at zero',
  };
}

function linearCases(bits, colsParam, cols) {
  const k = bits === 4 ? 256 : 128;
  const extra = colsParam ? { [colsParam]: cols } : {};
  return [
    linearCase('grid-uncalibrated', 11 + bits, bits, 10, k, cols, 0, 0, KIND.f32, extra),
    linearCase('grid-srq-int8-out', 12 + bits, bits, 10, k, cols, 0.125, 0.0625, KIND.i8, extra),
    linearCase('grid-srq-f32-out', 13 + bits, bits, 10, k, cols, 0.125, 0.0625, KIND.f32, extra),
  ];
}

function batchCases(count) {
  const rows = 8;
  const k = 256;
  const pairs = [[0, 0], [0.125, 0.0625], [0.015625, 0]];
  const ops = Array.from({ length: count }, (_, i) => gridOperands(40 + i, 4, rows, k, 1));
  ops.forEach(op => op.x.set(ops[0].x));  // one x for every projection
  const out = [];
  for (let oi = 0; oi < count; ++oi) {
    const inputs = { x: ops[0].x };
    const params = { k, outputIndex: oi };
    for (let i = 0; i < count; ++i) {
      inputs[`w${i}`] = ops[i].wq;
      inputs[`s${i}`] = ops[i].scales;
      params[`rows${i}`] = rows;
      params[`inScale${i}`] = pairs[i][0];
      params[`outScale${i}`] = pairs[i][1];
      if (i !== oi) inputs[`out${i}`] = { bytes: rows * 4, kind: KIND.f32 };
    }
    out.push({
      name: `mixed-routing-output-${oi}`, inputs, params,
      expected: gridExpected(ops[oi], rows, k, 1, pairs[oi][0], pairs[oi][1], KIND.f32),
      note: 'projectionBatch.ts:130-150: uncalibrated, SRQ and clamped SRQ in one dispatch',
    });
  }
  return out;
}

/** The split band of qgemv.ts:521-548 (32-word iterations, the tail in the band past kIters). */
function splitBands(bits, k, splits, exact) {
  const cpw = bits === 4 ? 8 : 4;
  const kWords = k / cpw;
  const kIters = Math.floor(kWords / 32);
  const slots = kIters + (exact ? (kWords % 32 !== 0 ? 1 : 0) : 1);
  const per = Math.ceil(slots / splits);
  const bands = [];
  for (let s = 0; s < splits; ++s) {
    const lo = Math.min(s * per, slots);
    const hi = Math.min(lo + per, slots);
    let wLo = lo * 32;
    let wHi = Math.min(hi, kIters) * 32;
    if (hi > kIters) wHi = kWords;
    if (wLo > wHi) wLo = wHi;
    bands.push([wLo * cpw, wHi * cpw]);
  }
  return bands;
}

function splitCase(bits, exact) {
  const rows = 10;
  const k = bits === 4 ? 1024 : 512;
  const splits = 4;  // 1, 2, 4 or 8 (qgemv.ts:253)
  const op = gridOperands(60 + bits, bits, rows, k, 1);
  const inScale = 0.125;
  const bands = splitBands(bits, k, splits, exact);
  const part = new Float32Array(rows * splits);
  for (let r = 0; r < rows; ++r) {
    bands.forEach(([lo, hi], s) => {
      let sum = 0;
      for (let i = lo; i < hi; ++i) sum += op.codes[r * k + i] * snap(op.x[i], inScale);
      part[r * splits + s] = exact ? sum : f32(f32(inScale * op.scales[r]) * sum);
    });
  }
  return {
    name: exact ? 'grid-exact-partials' : 'grid-scaled-partials',
    inputs: { wq: op.wq, scales: op.scales, x: op.x },
    params: { k, numRows: rows, kSplits: splits, exact: exact ? 1 : 0, inScale },
    expected: part,
  };
}

function mergeCases(exact) {
  const rows = 10;
  const splits = 4;
  const next = rng(70);
  const part = new Float32Array(rows * splits);
  for (let i = 0; i < part.length; ++i) part[i] = exact ? randInt(next, -500, 500) : randInt(next, -64, 64) / 32;
  const scales = new Float32Array(rows).map((_, r) => GRID_SCALES[r % 3]);
  const expected = new Float32Array(rows);
  for (let r = 0; r < rows; ++r) {
    let t = 0;
    for (let s = 0; s < splits; ++s) t += part[r * splits + s];
    const y = exact ? f32(f32(0.125 * scales[r]) * t) : t;
    expected[r] = snap(y, 0.0625) * 0.0625;
  }
  const inputs = exact ? { part, scales } : { part };
  const params = exact ? { numRows: rows, kSplits: splits, inScale: 0.125, outScale: 0.0625 }
    : { numRows: rows, kSplits: splits, outScale: 0.0625 };
  return [{ name: exact ? 'integer-partials' : 'grid-partials', inputs, params, expected }];
}

/** gelu(g) is exact at g in {-8, -6, 0, 6, 8}: tanh saturates to +-1 in f32 (geluMul.ts:101-116). */
function geluCases(bits, split) {
  const rows = 10;
  const k = bits === 4 ? 512 : 256;
  const op = gridOperands(80 + bits, bits, rows, k, 1);
  const next = rng(81);
  const gate = new Float32Array(k).map(() => [-8, -6, 0, 6, 8][randInt(next, 0, 4)]);
  const up = new Float32Array(k).map(() => randInt(next, -8, 8) / 8);
  const act = new Float32Array(k).map((_, i) => (gate[i] > 0 ? gate[i] : 0) * up[i]);
  const inScale = 0.125;
  if (split) {
    const bands = splitBands(bits, k, 2, true);
    const part = new Float32Array(rows * 2);
    for (let r = 0; r < rows; ++r) {
      bands.forEach(([lo, hi], s) => {
        let sum = 0;
        for (let i = lo; i < hi; ++i) sum += op.codes[r * k + i] * snap(act[i], inScale);
        part[r * 2 + s] = sum;
      });
    }
    return [{ name: 'saturated-gelu-exact-partials', inputs: { wq: op.wq, scales: op.scales, gate, up },
      params: { k, numRows: rows, kSplits: 2, inScale }, expected: part }];
  }
  const geluOp = { codes: op.codes, scales: op.scales, x: act };
  return [{ name: 'saturated-gelu', inputs: { wq: op.wq, scales: op.scales, gate, up },
    params: { k, numRows: rows, inScale, outScale: 0.0625 },
    expected: gridExpected(geluOp, rows, k, 1, inScale, 0.0625, KIND.i8) }];
}

/** gelu-mul on the saturated grid (gelu exact at 0 and |g| >= 6), with and without the snap. */
function geluMulCases() {
  const count = 64;
  const next = rng(83);
  const gate = new Float32Array(count).map(() => [-8, -6, 0, 6, 8][randInt(next, 0, 4)]);
  const up = new Float32Array(count).map(() => randInt(next, -24, 24) / 16);
  // gelu(g) in f32 on this grid: g for g >= 6, +0 at 0, and 0.5 * g * (1 - 1) = -0 for g <= -6
  const gelu = g => (g > 0 ? g : (g < 0 ? -0 : 0));
  const v = new Float32Array(count).map((_, i) => gelu(gate[i]) * up[i]);
  return [0, 0.125].map(srqScale => ({
    name: `saturated-gelu-mul-srq-${srqScale}`, inputs: { gate, up }, params: { count, srqScale },
    expected: srqScale === 0 ? v : v.map(x => snap(x, srqScale) * srqScale),
    note: 'geluMul.ts:101-116 with the consumer snap; exact on this grid',
  }));
}

/** The -m2 gelu forms: every column on the saturated-gelu grid, calibrated and uncalibrated. */
function geluWideCases(bits) {
  const rows = 10;
  const k = bits === 4 ? 512 : 256;
  const cols = 2;
  const op = gridOperands(84 + bits, bits, rows, k, cols);
  const next = rng(85 + bits);
  const gate = new Float32Array(cols * k).map(() => [-8, -6, 0, 6, 8][randInt(next, 0, 4)]);
  const up = new Float32Array(cols * k).map(() => randInt(next, -8, 8) / 8);
  const act = new Float32Array(cols * k).map((_, i) => (gate[i] > 0 ? gate[i] : 0) * up[i]);
  const geluOp = { codes: op.codes, scales: op.scales, x: act };
  const inputs = { wq: op.wq, scales: op.scales, gate, up };
  return [
    { name: 'saturated-gelu-m2-srq', inputs, params: { k, numRows: rows, cols, inScale: 0.125, outScale: 0.0625 },
      expected: gridExpected(geluOp, rows, k, cols, 0.125, 0.0625, KIND.i8),
      note: 'qgemvWide.ts:20-27: column for column the one-column gelu GEMV' },
    { name: 'saturated-gelu-m2-uncalibrated', inputs, params: { k, numRows: rows, cols },
      expected: gridExpected(geluOp, rows, k, cols, 0, 0, KIND.f32),
      note: 'the f32 path over the unsnapped product, exact on the grid' },
  ];
}

/** ple-gate-split: integer partials of each split band, interleaved (row/4)*4n + s*4 + row%4. */
function pleGateSplitCases() {
  const rows = 8;
  const k = 512;
  const n = pleActiveSplits();
  const op = gridOperands(91, 8, rows, k, 1);
  const inScale = 0.125;
  const bands = splitBands(8, k, n, true);
  const part = new Float32Array(rows * n);
  for (let r = 0; r < rows; ++r) {
    bands.forEach(([lo, hi], sp) => {
      let sum = 0;
      for (let i = lo; i < hi; ++i) sum += op.codes[r * k + i] * snap(op.x[i], inScale);
      part[Math.floor(r / 4) * 4 * n + sp * 4 + (r % 4)] = sum;
    });
  }
  return [{ name: `grid-raw-partials-${n}`, inputs: { wq: op.wq, scales: op.scales, x: op.x },
    params: { k, numRows: rows, inScale }, expected: part,
    note: 'pleSplit.ts:17-23: the exact partials in the fold\'s vec4 layout' }];
}

/**
 * ple-fold-projection: integer partials whose folded gate is 0 or at least 6 in magnitude (gelu is
 * then exact in f32: tanh saturates under the 10 clamp), at gateInScale 0.125 and gateScales 0.5
 * (v = total / 16 exactly), with gateOutScale 0 and 0.125 (the reference's two cases,
 * pleSplit.ts:66-71); odd totals land the gate snap on ties. The up row is read at upOffset.
 */
function pleFoldCases() {
  const rows = 10;
  const k = 256;
  const n = pleActiveSplits();
  const op = gridOperands(93, 8, rows, k, 1);
  const next = rng(94);
  const totals = new Float32Array(k).map(() => {
    const c = randInt(next, 0, 2);
    return c === 0 ? 0 : (c === 1 ? 1 : -1) * randInt(next, 96, 250);
  });
  const part = new Float32Array(k * n);
  for (let i = 0; i < k; ++i) {
    const base = Math.floor(i / 4) * 4 * n + (i % 4);
    let rest = totals[i];
    for (let sp = 0; sp < n - 1; ++sp) {
      const piece = randInt(next, -20, 20);
      part[base + sp * 4] = piece;
      rest -= piece;
    }
    part[base + (n - 1) * 4] = rest;
  }
  const gateScales = new Float32Array(k).fill(0.5);
  const layerRow = 3;
  const upAll = new Float32Array(5 * k).map(() => randInt(next, -8, 8) / 8);
  const out = [];
  for (const gateOutScale of [0, 0.125]) {
    const act = new Float32Array(k).map((_, i) => {
      let v = totals[i] / 16;
      if (gateOutScale !== 0) v = snap(v, gateOutScale) * gateOutScale;
      const g = v >= 6 ? v : 0;  // gelu at |v| >= 6 and at 0, exact in f32
      return g * upAll[layerRow * k + i];
    });
    out.push({
      name: `grid-fold-${n}-gate-srq-${gateOutScale}`,
      inputs: { wq: op.wq, scales: op.scales, gate: part, up: upAll, gateScales },
      params: { k, numRows: rows, inScale: 0.125, outScale: 0.0625, upOffset: layerRow * k / 4,
        gateInScale: 0.125, gateOutScale },
      expected: gridExpected({ codes: op.codes, scales: op.scales, x: act }, rows, k, 1, 0.125, 0.0625, KIND.i8),
      note: 'pleSplit.ts:33-41 foldGate, then the qgemv-8bit-gelu prologue',
    });
  }
  return out;
}

function gatherCase(sliced) {
  const rows = 48;
  const cols = 512;
  const group = 256;
  const next = rng(90);
  const codes = new Uint8Array(rows * cols / 2).map(() => randInt(next, 0, 255));
  const scales = new Float32Array(rows * 2).map(() => [0.0078125, 0.015625, 0.005859375][randInt(next, 0, 2)]);
  const ids = new Int32Array([3, 40, 17, 47, 0, 3]);
  const start = 16;
  const count = 24;
  const expected = new Float32Array(ids.length * cols);
  ids.forEach((id, slot) => {
    if (sliced && !(id >= start && id < start + count)) return;  // not this slice's: untouched
    for (let c = 0; c < cols; ++c) {
      const b = codes[id * cols / 2 + (c >> 1)];
      const code = ((c & 1) ? b >> 4 : b & 15) - 8;
      expected[slot * cols + c] = code * f32(16 * scales[id * 2 + Math.floor(c / group)]);
    }
  });
  const table = sliced ? codes.slice(start * cols / 2, (start + count) * cols / 2) : codes;
  const params = { slots: ids.length, cols, groupSize: group };
  if (sliced) Object.assign(params, { sliceStartRow: start, sliceRowCount: count });
  return [{ name: sliced ? 'one-slice-owner-writes' : 'whole-table', inputs: { codes: table, scales, ids },
    params, expected, outputInit: sliced ? 'zero' : 'sentinel',
    note: 'embedGather.ts:149-152, 188-196: (code - 8) * f32(16 * scale), a non-owner writes nothing' }];
}

// The PLE split kernels' cases depend on the active split count (pleSplit.ts:43-49, 65-71 build
// them in getters for the same reason), so those two entries compute theirs when read.
const LIVE_CASES = {
  'ple-gate-split': pleGateSplitCases,
  'ple-fold-projection': pleFoldCases,
};
function registered(name, bind, cases, note) {
  if (cases !== null) return { name, bind, cases, note };
  return { name, bind, note, get cases() { return LIVE_CASES[name](); } };
}

const KERNELS = {
  'qgemv-4bit': registered('qgemv-4bit', BINDS['qgemv-4bit'], linearCases(4, null, 1)),
  'qgemv-8bit': registered('qgemv-8bit', BINDS['qgemv-8bit'], linearCases(8, null, 1)),
  'qgemv-4bit-m2': registered('qgemv-4bit-m2', BINDS['qgemv-4bit-m2'], linearCases(4, 'cols', 2)),
  'qgemv-8bit-m2': registered('qgemv-8bit-m2', BINDS['qgemv-8bit-m2'], linearCases(8, 'cols', 2)),
  'qgemm-4bit': registered('qgemm-4bit', BINDS['qgemm-4bit'], linearCases(4, 'mCols', 11)),
  'qgemm-4bit-single': registered('qgemm-4bit-single', BINDS['qgemm-4bit-single'], linearCases(4, 'mCols', 1)),
  'qgemm-4bit-prefill4': registered('qgemm-4bit-prefill4', BINDS['qgemm-4bit-prefill4'], linearCases(4, 'mCols', 40)),
  'qmatmul-8bit': registered('qmatmul-8bit', BINDS['qmatmul-8bit'], linearCases(8, 'mCols', 3)),
  'qkv-batch-4bit': registered('qkv-batch-4bit', BINDS['qkv-batch-4bit'], batchCases(3)),
  'gate-up-batch-4bit': registered('gate-up-batch-4bit', BINDS['gate-up-batch-4bit'], batchCases(2)),
  'qgemv-4bit-gelu': registered('qgemv-4bit-gelu', BINDS['qgemv-4bit-gelu'], geluCases(4, false)),
  'qgemv-8bit-gelu': registered('qgemv-8bit-gelu', BINDS['qgemv-8bit-gelu'], geluCases(8, false)),
  'qgemv-4bit-gelu-m2': registered('qgemv-4bit-gelu-m2', BINDS['qgemv-4bit-gelu-m2'], geluWideCases(4)),
  'qgemv-8bit-gelu-m2': registered('qgemv-8bit-gelu-m2', BINDS['qgemv-8bit-gelu-m2'], geluWideCases(8)),
  'qgemv-4bit-gelu-exact-split': registered('qgemv-4bit-gelu-exact-split',
    BINDS['qgemv-4bit-gelu-exact-split'], geluCases(4, true)),
  'gelu-mul': registered('gelu-mul', BINDS['gelu-mul'], geluMulCases()),
  'ple-gate-split': registered('ple-gate-split', BINDS['ple-gate-split'], null),
  'ple-fold-projection': registered('ple-fold-projection', BINDS['ple-fold-projection'], null),
  'qgemv-4bit-split': registered('qgemv-4bit-split', BINDS['qgemv-4bit-split'], [splitCase(4, false), splitCase(4, true)]),
  'qgemv-8bit-split': registered('qgemv-8bit-split', BINDS['qgemv-8bit-split'], [splitCase(8, false), splitCase(8, true)]),
  'qgemv-merge': registered('qgemv-merge', BINDS['qgemv-merge'], mergeCases(false)),
  'qgemv-exact-merge': registered('qgemv-exact-merge', BINDS['qgemv-exact-merge'], mergeCases(true)),
  'ple-gather-4bit': registered('ple-gather-4bit', BINDS['ple-gather-4bit'], gatherCase(false)),
  'ple-gather-4bit-sliced': registered('ple-gather-4bit-sliced', BINDS['ple-gather-4bit-sliced'], gatherCase(true)),
};

/**
 * Run registry kernel `name` with the reference's bind input ({inputs, output, params}, plus an
 * optional `stream`: a Stream or handle; the call only enqueues).
 */
function bind(name, input) {
  const k = KERNELS[name];
  if (!k) throw Object.assign(new Error(`gemma4 engine: no registered kernel named ${name}`), { status: 2 });
  k.bind(input);
  return { kernel: name };
}

function kindOfArray(a) {
  if (a instanceof Float32Array) return KIND.f32;
  if (a instanceof Int32Array) return KIND.i32;
  return KIND.i8;
}

/**
 * Runs every case of `name` (or of every kernel) on the device and compares the output bytes with
 * the expected ones (the registry's zero tolerance): [{kernel, case, ok, mismatches}].
 */
function runCases(name, stream) {
  const names = name ? [name] : Object.keys(KERNELS);
  const results = [];
  for (const n of names) {
    for (const c of KERNELS[n].cases) {
      const bufs = [];
      const inputs = {};
      for (const key of Object.keys(c.inputs)) {
        const v = c.inputs[key];
        const b = ArrayBuffer.isView(v) ? DeviceBuffer.from(v, kindOfArray(v))
          : new DeviceBuffer(v.bytes, v.kind);
        inputs[key] = b;
        bufs.push(b);
      }
      const output = new DeviceBuffer(c.expected.byteLength, kindOfArray(c.expected));
      bufs.push(output);
      output.fill(c.outputInit === 'zero' ? 0 : 0x7b, stream);
      bind(n, { inputs, output, params: c.params, stream });
      const got = new Uint8Array(output.download(stream));
      const want = new Uint8Array(c.expected.buffer, c.expected.byteOffset, c.expected.byteLength);
      let mismatches = 0;
      for (let i = 0; i < want.length; ++i) if (got[i] !== want[i]) mismatches += 1;
      results.push({ kernel: n, case: c.name, ok: mismatches === 0, mismatches });
      bufs.forEach(b => b.free());
    }
  }
  return results;
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

// ---- the plan's projection steps (plan.ts:487-665, 725-753, 775-785) -----------------------------
//
// The kernel names planLayer / planEmbed / planHead give the steps of the projection path, for the
// families this build serves (4-bit attention, MLP and head; the 8-bit PLE linears), and
// resolveStep's choice among them (execute.ts:566-600, 721-726, 765-895, 956-968). A caller can
// check that every name a plan under its options binds is registered here.

const PLAN_GEMV = { 4: 'qgemv-4bit', 8: 'qmatmul-8bit' };                 // plan.ts:369
const PLAN_GEMM = { 4: 'qgemm-4bit', 8: 'qmatmul-8bit' };                 // plan.ts:370
const PLAN_GEMV_GELU = { 4: 'qgemv-4bit-gelu', 8: 'qgemv-8bit-gelu' };    // plan.ts:433

/** planLayer's projection steps for one layer (plan.ts:487-640): {kernel, role, kSplits?}. */
function planLayerProjections(producer, mode, options) {
  const o = options || {};
  const mm = mode === 'gemv' ? PLAN_GEMV : PLAN_GEMM;
  const steps = [];
  const push = (kernel, role, extra) => steps.push(Object.assign({ kernel, role }, extra || {}));
  const fusedPrologue = mode === 'gemv' && o.attentionPrologue !== false;
  const attnSplit = fusedPrologue && (o.attnKSplits || 1) > 1;
  const proj = attnSplit ? 'qgemv-4bit-split' : mm[4];
  if (mode === 'gemv' && o.batchProjections && producer && !attnSplit) {
    push('qkv-batch-4bit', 'q_proj, k_proj, v_proj');
  } else {
    push(proj, 'q_proj');
    if (producer) {
      push(proj, 'k_proj');
      push(proj, 'v_proj');
    }
  }
  push(mm[4], 'o_proj');
  if (mode === 'gemv' && o.batchProjections) {
    push('gate-up-batch-4bit', 'gate_proj, up_proj');
  } else {
    push(mm[4], 'gate_proj');
    push(mm[4], 'up_proj');
  }
  if (mode === 'gemv') {
    if ((o.producerDownKSplits || 1) > 1) {
      push('qgemv-4bit-gelu-exact-split', 'producer down exact partials');
      push('qgemv-exact-merge', 'producer down exact fold', { kSplits: o.producerDownKSplits });
    } else {
      push(PLAN_GEMV_GELU[4], 'gelu down');
    }
  } else {
    push('gelu-mul', 'gelu times up');
    push(mm[4], 'down_proj');
  }
  const pleSplit = mode === 'gemv' && (o.pleGateKSplits || 1) > 1;
  push(pleSplit ? 'ple-gate-split' : mm[8], 'per_layer_input_gate');
  if (mode === 'gemv') {
    push(pleSplit ? 'ple-fold-projection' : PLAN_GEMV_GELU[8], 'gelu ple');
  } else {
    push('gelu-mul', 'gate times per layer row');
    push(mm[8], 'per_layer_projection');
  }
  return steps;
}

/** resolveStep's registry name for a projection step (execute.ts:566-895, 956-968); throws where it does. */
function resolveProjectionKernel(step, geometry) {
  const tokens = geometry.tokens;
  switch (step.role) {
    case 'q_proj, k_proj, v_proj':
    case 'gate_proj, up_proj':
      if (tokens !== 1) throw new Error('batched projections require a single token');
      return step.kernel;
    case 'q_proj':
    case 'k_proj':
    case 'v_proj': {
      const wide = geometry.mode === 'gemv' && tokens !== 1;  // attnUnsplitOnWide, execute.ts:396-403
      return matmulKernel(geometry, wide && step.kernel === 'qgemv-4bit-split' ? 'qgemv-4bit' : step.kernel);
    }
    case 'o_proj':
    case 'gate_proj':
    case 'up_proj':
    case 'down_proj':
      return matmulKernel(geometry, step.kernel);
    case 'producer down exact partials':
      if (tokens !== 1) throw new Error('producer split needs one token');
      return step.kernel;
    case 'producer down exact fold':
      return step.kernel;
    case 'gelu down':
      return gemvWide(geometry, step.kernel);
    case 'per_layer_input_gate':
    case 'per_layer_projection':
      return pleKernel(geometry, step.kernel);
    case 'gelu ple':
      if (step.kernel === 'ple-fold-projection') {
        if (tokens !== 1) throw new Error('PLE split needs one token');
        return step.kernel;
      }
      return gemvWide(geometry, step.kernel);
    case 'gelu times up':
    case 'gate times per layer row':
      return step.kernel;  // gelu-mul: the elementwise pass (g4_gelu_mul), not a projection
    case 'lm_head':
      return gemvWide(geometry, step.kernel);
    default:
      throw new Error(`gemma4 engine: no projection step with role ${step.role}`);
  }
}

/**
 * Every registry name one decode step (mode 'gemv') or prefill chunk ('gemm') binds on the
 * projection path under `options` (PlanOptions: batchProjections, producerDownKSplits,
 * pleGateKSplits, attnKSplits, attentionPrologue): the per-layer linears of producer and consumer
 * layers, the PLE gather (one sliced step per slice when `pleSlices` > 1, plan.ts:775-785) and
 * the head (plan.ts:745-753). Throws what resolveStep throws for an unservable combination.
 */
function planProjectionKernels(geometry, options, pleSlices) {
  const names = new Set();
  for (const producer of [true, false]) {
    for (const step of planLayerProjections(producer, geometry.mode, options)) {
      names.add(resolveProjectionKernel(step, geometry));
    }
  }
  names.add((pleSlices || 1) > 1 ? 'ple-gather-4bit-sliced' : 'ple-gather-4bit');
  if (geometry.mode === 'gemv') names.add(resolveProjectionKernel({ kernel: PLAN_GEMV[4], role: 'lm_head' }, geometry));
  return [...names];
}

// ---- the split planner (tableSplit.ts) ----------------------------------------------------------

/** planTableSplit (tableSplit.ts:125-215), computed by the library (pure host code). */
function planTableSplit(input) { return g4().planTableSplit(input); }

/**
 * planGatherSplit (tableSplit.ts:257-287): the packed codes and the f32 scales planned separately
 * under one device's limits; scalesSingle is what the sliced gather assumes.
 */
function planGatherSplit(name, rows, codeRowBytes, scalesPerRow, limits) {
  const plans = g4().planGatherSplit(rows, codeRowBytes, scalesPerRow, limits);
  plans.name = name;
  plans.note = plans.scalesSingle
    ? `${name} codes: ${plans.codes.slices.length} slice(s); ${name} scales: one buffer, which is what the gather kernel assumes.`
    : `${name} scales do NOT fit in one binding on this adapter, and the sliced gather addresses `
      + 'scales by the absolute vocabulary row, so this configuration is not served.';
  return plans;
}

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

/**
 * The native decode-step runner (include/g4decode.h) over a model already in device memory:
 * shape and weights use the C structs' field names (weights: device addresses, `layer` one object
 * per layer, optional `ple_slices` [{codes, start_row, row_count}] for a split PLE table).
 * step() and setPosition() only enqueue on the given stream, so several tokens' steps can be in
 * flight at once (the reference's lookahead, plan.ts:942-973): step t+1 reads the next-token
 * buffer step t writes, and the host awaits only its downloads.
 */
class Decoder {
  constructor(shape, weights) {
    this.shape = shape;
    this.handle = g4().decodeCreate(shape, weights);
  }

  setPosition(pos, stream) { g4().decodeSetPosition(this.handle, pos, streamHandle(stream)); }
  step(tokens, nextTokens, stream) {
    g4().decodeStep(this.handle, tokens.addr, nextTokens.addr, streamHandle(stream));
  }

  /** A named work buffer of the last step: {addr, bytes} ("logits", "hidden", "per_layer", ...). */
  buffer(name) { return g4().decodeBuffer(this.handle, name); }
  kv(layer) { return g4().decodeKv(this.handle, layer); }
  setStop(lastLayer) { g4().decodeSetStop(this.handle, lastLayer); }
  destroy() {
    if (this.handle) g4().decodeDestroy(this.handle);
    this.handle = 0;
  }
}

module.exports = {
  KIND,
  DeviceBuffer,
  KERNELS,
  kernelNames: () => Object.keys(KERNELS),
  bind,
  runCases,
  Stream,
  Graph,
  Decoder,
  planGatherSplit,
  linearParams,
  gemvWide,
  pleKernel,
  matmulKernel,
  planLayerProjections,
  resolveProjectionKernel,
  planProjectionKernels,
  pleGateSplits,
  setPleGateSplits,
  gemvInner,
  setGemvInner,
  tile8uBytes,
  tile8uRepack,
  qgemvTile8u,
  planTableSplit,
  sliceForRow,
  slicedGatherDispatches,
  GemvPlan,
  kernelForShape: (bits, m, n, k) => g4().kernelForShape(bits, m, n, k),
  deviceCount: () => g4().deviceCount(),
  setDevice: d => g4().setDevice(d),
  synchronize: () => g4().synchronize(),
  synchronizeAsync: stream => g4().synchronizeAsync(streamHandle(stream)),
  qgemmNoalloc: (...args) => g4().qgemmNoalloc(...args),
  pleGatherSplit: (...args) => g4().pleGatherSplit(...args),
  addon: g4,
};
