"""GPU parity of the registry kernels a verify pass and a split-PLE profile name:
ple-gate-split and ple-fold-projection (pleSplit.ts:17-84, plan.ts:633-636, execute.ts:855-890)
and the wide gelu GEMVs qgemv-4bit-gelu-m2 / qgemv-8bit-gelu-m2 (qgemvWide.ts:660-709, execute.ts
:382-390), each bit for bit against the pinned oracle: the split partials and int8 codes exactly,
and the fold at adversarial gate-snap quotients."""
import numpy as np
import pytest

import decode_oracle as d
import g4synth as syn
from snapcases import ADV_OUT, KA_SCALE, KA_VALUE, S_OUT

pytestmark = pytest.mark.gpu

F = np.float32
IN, OUT = syn.IN_SCALE, syn.OUT_SCALE
HIDDEN, PLE_DIM, LAYERS = 1536, 256, 35


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def u32(a):
    return np.ascontiguousarray(a, F).view(np.uint32)


def residual(seed, k=HIDDEN):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(k) * 2.0).astype(F)
    x[::97] = F(8.0)  # saturating outliers
    return x


@pytest.mark.parametrize("splits", [1, 2, 4, 8])
@pytest.mark.parametrize("x_kind", ["f32", "f16", "i8"])
def test_ple_gate_split_partials(gpu, oracle, splits, x_kind):
    print(f"ple-gate-split splits={splits} x={x_kind}", flush=True)
    n, k = PLE_DIM, HIDDEN
    w = syn.int8_weights("plesplit", "gate", n, k)
    s = syn.row_scales("plesplit", "gate_s", n)
    x = residual(splits)
    if x_kind == "f16":
        x = x.astype(np.float16)
        x_ref = x.astype(F)
        dx = dev(gpu, x)
    elif x_kind == "i8":
        codes = oracle.srq_codes(x, IN)
        x_ref = codes.astype(F) * F(IN)
        dx = dev(gpu, codes)
    else:
        x_ref = x
        dx = dev(gpu, x)
    active = 2 if splits == 1 else splits  # pleSplit.ts:16
    want = oracle.ple_gate_split(w, s, x_ref, n, k, active, IN)
    parts = gpu.DeviceBuffer.empty((n * active,), F)
    parts.fill(0x7B)
    gpu.ple_gate_split(dev(gpu, w), dev(gpu, s), dx, parts, k, n, splits, IN)
    assert np.array_equal(u32(parts.download()), u32(want))


def fold_expected(oracle, w, s, parts, gate_scales, splits, gin, gout, up_row, n, k):
    gate = oracle.ple_fold_gate(parts, k, splits, gate_scales, gin, gout)
    act = d.gelu_mul_f32_codes(gate, up_row, IN)
    xin = act.astype(F) * F(IN)
    assert np.array_equal(oracle.srq_codes(xin, IN), act)  # the codes survive the oracle's snap
    return oracle.qgemv(8, w, s, xin, n, k, IN, OUT)[2]


@pytest.mark.parametrize("splits", [2, 4, 8])
@pytest.mark.parametrize("gate_out", [0.0, float(OUT), 0.125])
def test_ple_fold_projection_after_gate_split(gpu, oracle, splits, gate_out):
    """The decode pair: the gate split over the residual, then the fold projection reading layer
    34's row of the per-layer input in place (upOffset = 34 * 64 vec4s, qgemv.ts:1801)."""
    print(f"ple-fold-projection splits={splits} gate_out={gate_out}", flush=True)
    layer = 34
    gw = syn.int8_weights("plesplit", "gate", PLE_DIM, HIDDEN)
    gs = syn.row_scales("plesplit", "gate_s", PLE_DIM)
    pw = syn.int8_weights("plesplit", "proj", HIDDEN, PLE_DIM)
    ps = syn.row_scales("plesplit", "proj_s", HIDDEN)
    x = residual(10 + splits)
    rng = np.random.default_rng(splits)
    ple_in = rng.uniform(-3, 3, LAYERS * PLE_DIM).astype(F)
    up_row = ple_in[layer * PLE_DIM:(layer + 1) * PLE_DIM]
    parts_ref = oracle.ple_gate_split(gw, gs, x, PLE_DIM, HIDDEN, splits, IN)
    want = fold_expected(oracle, pw, ps, parts_ref, gs, splits, IN, gate_out, up_row, HIDDEN,
                         PLE_DIM)
    # the same codes through the unsplit chain: the gate's f32 output, then qgemv-8bit-gelu
    y_gate = oracle.qgemv(8, gw, gs, x, PLE_DIM, HIDDEN, IN, gate_out)[0]
    act2 = d.gelu_mul_f32_codes(y_gate, up_row, IN)
    assert np.array_equal(oracle.qgemv(8, pw, ps, act2.astype(F) * F(IN), HIDDEN, PLE_DIM, IN,
                                       OUT)[2], want)
    dgs = dev(gpu, gs)
    parts = gpu.DeviceBuffer.empty((PLE_DIM * splits,), F)
    gpu.ple_gate_split(dev(gpu, gw), dgs, dev(gpu, x), parts, HIDDEN, PLE_DIM, splits, IN)
    dup = dev(gpu, ple_in)
    act = gpu.gelu_act(dup, up_offset=4 * layer * 64)
    dst = gpu.DeviceBuffer.empty((HIDDEN,), np.int8)
    dst.fill(0x7B)
    gpu.ple_fold_projection(dev(gpu, pw), dev(gpu, ps), parts, dgs, splits, IN, gate_out, act,
                            dst, PLE_DIM, HIDDEN, IN, OUT)
    assert np.array_equal(dst.download(), want)
    assert np.array_equal(u32(parts.download()), u32(parts_ref))
    # the Python registry mirror: upOffset in vec4s, the split count a module setting
    dst2 = gpu.DeviceBuffer.empty((HIDDEN,), np.int8)
    gpu.set_ple_gate_splits(splits)
    try:
        gpu.bind("ple-fold-projection",
                 {"wq": dev(gpu, pw), "scales": dev(gpu, ps), "gate": parts, "up": dup,
                  "gateScales": dgs}, dst2,
                 {"k": PLE_DIM, "numRows": HIDDEN, "inScale": IN, "outScale": OUT,
                  "upOffset": layer * PLE_DIM // 4, "gateInScale": IN, "gateOutScale": gate_out})
    finally:
        gpu.set_ple_gate_splits(1)
    assert np.array_equal(dst2.download(), want)


@pytest.mark.parametrize("case", ["adv-out", "known-answer", "ties"])
def test_ple_fold_gate_snap_adversarial(gpu, oracle, case):
    """Gate values planted on the quotients where rint(v * fl(1/s)) and rint(fl(v / s)) differ, on
    exact ties, and on the in-tree known answer: the fold's snap must take the IEEE divide."""
    print(f"ple-fold gate snap {case}", flush=True)
    splits, k, n = 4, PLE_DIM, HIDDEN
    pw = syn.int8_weights("plesplit", "proj", n, k)
    ps = syn.row_scales("plesplit", "proj_s", n)
    rng = np.random.default_rng(7)
    if case == "adv-out":
        vals = np.array([v for v in ADV_OUT] + [-v for v in ADV_OUT], F)
        gout, gin = float(S_OUT), 1.0
    elif case == "known-answer":
        vals = np.array([KA_VALUE, -KA_VALUE], F)
        gout, gin = float(KA_SCALE), 1.0
    else:
        vals = np.arange(-41, 42, 2, dtype=F)  # odd totals: at in * scale = 1/16, gout 1/8, halves
        gout, gin = 0.125, 0.125
    totals = vals[np.arange(k) % vals.size]
    gscale = np.full(k, 0.5 if case == "ties" else 1.0, F)
    parts = np.zeros(k * splits, F)
    # spread each total over the splits in integer-free pieces that sum exactly in f32 order
    for i in range(k):
        base = (i // 4) * 4 * splits + i % 4
        parts[base + 2 * 4] = totals[i]
    up = rng.uniform(-3, 3, k).astype(F)
    want = fold_expected(oracle, pw, ps, parts, gscale, splits, gin, gout, up, n, k)
    gate = oracle.ple_fold_gate(parts, k, splits, gscale, gin, gout)
    if case == "adv-out":  # the planted quotients really are the divergent ones
        q = (np.abs(vals).astype(F) / F(gout)).astype(F)
        assert np.any(np.rint(q) != np.rint(np.abs(vals) * (F(1) / F(gout))))
    assert np.unique(gate).size >= 2
    dst = gpu.DeviceBuffer.empty((n,), np.int8)
    dst.fill(0x7B)
    gpu.ple_fold_projection(dev(gpu, pw), dev(gpu, ps), dev(gpu, parts), dev(gpu, gscale), splits,
                            gin, gout, gpu.gelu_act(dev(gpu, up)), dst, k, n, IN, OUT)
    assert np.array_equal(dst.download(), want)


@pytest.mark.parametrize("bits,n,k,form", [(4, 1536, 6144, "f32"), (4, 1536, 6144, "codes"),
                                           (8, 1536, 256, "ple"), (8, 40, 1536, "f32")])
@pytest.mark.parametrize("cols", [1, 2])
def test_qgemv_gelu_m2_columns(gpu, oracle, bits, n, k, form, cols):
    """The draft-verify down_proj / per_layer_projection: every column is the one-column gelu GEMV
    over its own gate and up (qgemvWide.ts:20-27), here against the oracle's unfused chain."""
    print(f"qgemv-{bits}bit-gelu-m2 n={n} k={k} form={form} cols={cols}", flush=True)
    rng = np.random.default_rng(n + k + cols)
    w = syn.weights("gelu2", f"w{bits}_{n}_{k}", n, k, bits)
    s = syn.row_scales("gelu2", f"s{n}_{k}", n)
    if form == "codes":
        gate = rng.integers(-128, 128, (cols, k)).astype(np.int8)
        up = rng.integers(-128, 128, (cols, k)).astype(np.int8)
        acts = [d.gelu_mul_codes(gate[c], OUT, up[c], OUT, IN) for c in range(cols)]
    elif form == "ple":
        gate = rng.integers(-128, 128, (cols, k)).astype(np.int8)
        up = rng.uniform(-3, 3, (cols, k)).astype(F)
        acts = [d.gelu_mul_codes(gate[c], OUT, None, 0.0, IN, up_f32=up[c]) for c in range(cols)]
    else:
        gate = (rng.standard_normal((cols, k)) * 2.5).astype(F)
        up = (rng.standard_normal((cols, k)) * 1.5).astype(F)
        acts = [d.gelu_mul_f32_codes(gate[c], up[c], IN) for c in range(cols)]
    want = np.stack([oracle.qgemv(bits, w, s, a.astype(F) * F(IN), n, k, IN, OUT)[2] for a in acts])
    pad = 32  # up sits at an offset (elements) inside a wider buffer
    up_buf = np.concatenate([np.zeros(pad, up.dtype), up.reshape(-1), np.zeros(16, up.dtype)])
    dw, ds, dg, du = dev(gpu, w), dev(gpu, s), dev(gpu, gate), dev(gpu, up_buf)
    act = gpu.gelu_act(du, gate_scale=OUT, up_scale=OUT, up_offset=pad)
    dst = gpu.DeviceBuffer.empty((cols, n), np.int8)
    dst.fill(0x7B)
    gpu.qgemv_gelu_m2(bits, dw, ds, dg, act, dst, k, n, cols, IN, OUT)
    assert np.array_equal(dst.download(), want)
    # through the registry mirror, upOffset in vec4s
    dst2 = gpu.DeviceBuffer.empty((cols, n), np.int8)
    gpu.bind(f"qgemv-{bits}bit-gelu-m2", {"wq": dw, "scales": ds, "gate": dg, "up": du}, dst2,
             {"k": k, "numRows": n, "cols": cols, "inScale": IN, "outScale": OUT,
              "upOffset": pad // 4, "gateScale": OUT, "upScale": OUT})
    assert np.array_equal(dst2.download(), want)


@pytest.mark.parametrize("bits,cols", [(4, 1), (4, 2), (8, 2)])
def test_gelu_uncalibrated_on_the_exact_grid(gpu, oracle, bits, cols):
    """inScale 0: the f32 code dot over the unsnapped gelu(gate) * up (qgemv.ts:359-400). With
    gates where gelu is exact in f32 ({-8, -6, 0, 6, 8}: tanh saturates) and up on the 1/8 grid,
    every product and sum is exact, so the order cannot matter and the output is exact."""
    print(f"gelu uncalibrated bits={bits} cols={cols}", flush=True)
    n, k = 24, 512
    rng = np.random.default_rng(bits * 10 + cols)
    codes = rng.integers(-8, 8, (n, k)) if bits == 4 else rng.integers(-127, 128, (n, k))
    w = oracle.pack_matrix(bits, codes.astype(np.int8))
    s = np.array([0.1875, 0.015625, 0.0625] * (n // 3), F)
    gate = rng.choice(np.array([-8, -6, 0, 6, 8], F), (cols, k))
    up = (rng.integers(-8, 9, (cols, k)) / 8).astype(F)
    for g in (-8.0, -6.0, 0.0, 6.0, 8.0):
        assert d.gelu_tanh(g) == max(g, 0.0)
    act = np.maximum(gate, 0) * up
    want = np.stack([oracle.qgemv(bits, w, s, act[c], n, k, 0.0, 0.0)[0] for c in range(cols)])
    dst = gpu.DeviceBuffer.empty((cols, n), F)
    gpu.qgemv_gelu_m2(bits, dev(gpu, w), dev(gpu, s), dev(gpu, gate), gpu.gelu_act(dev(gpu, up)),
                      dst, k, n, cols, 0.0, 0.0)
    assert np.array_equal(u32(dst.download()), u32(want))
