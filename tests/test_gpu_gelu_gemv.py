"""GPU parity of the fused gelu prologue GEMVs (qgemv-4bit-gelu / qgemv-8bit-gelu, the gelu exact
split and plans with prologues; qgemv.ts:359-400, 1668-1696, exactSplit.ts:19-31) against the
oracle's unfused chain: gelu-mul codes (geluMul.ts, oracle/g4_decode_oracle.c) fed to the pinned
GEMV oracle. On calibrated sites the fused and unfused forms are bit for bit the same, which is
what the reference argues at qgemv.ts:362-368; every output here is compared exactly."""
import numpy as np
import pytest

import decode_oracle as d
import g4synth as syn

pytestmark = pytest.mark.gpu

IN, OUT = syn.IN_SCALE, syn.OUT_SCALE


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def operands(rng, k, form):
    """gate and up as the runner produces them (int8 codes on OUT) or as the reference's f32."""
    gc = rng.integers(-128, 128, k).astype(np.int8)
    uc = rng.integers(-128, 128, k).astype(np.int8)
    if form == "codes":
        act = d.gelu_mul_codes(gc, OUT, uc, OUT, IN)
        return gc, uc, act
    if form == "ple":  # int8 gate, f32 up row (the per-layer input)
        up = rng.uniform(-3, 3, k).astype(np.float32)
        return gc, up, d.gelu_mul_codes(gc, OUT, None, 0.0, IN, up_f32=up)
    g = rng.standard_normal(k).astype(np.float32) * np.float32(2.5)
    u = rng.standard_normal(k).astype(np.float32) * np.float32(1.5)
    return g, u, d.gelu_mul_f32_codes(g, u, IN)


def expected(oracle, bits, w, s, act, n, k):
    x = act.astype(np.float32) * np.float32(IN)  # round-trips to the same codes in the oracle's snap
    _, acc, codes = oracle.qgemv(bits, w, s, x, n, k, IN, OUT)
    return acc, codes


@pytest.mark.parametrize("bits,n,k,form", [(4, 1536, 6144, "codes"), (4, 96, 6144, "f32"),
                                           (8, 1536, 256, "ple"), (8, 40, 1536, "codes"),
                                           (4, 200, 512, "ple"), (4, 64, 2304, "f32")])
def test_qgemv_gelu_matches_unfused(gpu, oracle, bits, n, k, form):
    print(f"qgemv gelu bits={bits} n={n} k={k} form={form}", flush=True)
    rng = np.random.default_rng(n + k + bits)
    w = syn.weights("gelu", f"w{bits}_{n}_{k}", n, k, bits)
    s = syn.row_scales("gelu", f"s{n}_{k}", n)
    gate, up, act = operands(rng, k, form)
    _, want = expected(oracle, bits, w, s, act, n, k)
    dw, ds, dg = dev(gpu, w), dev(gpu, s), dev(gpu, gate)
    # the up operand sits at an offset inside a wider buffer, as a per-layer row does
    pad = 64
    up_buf = np.concatenate([np.zeros(pad, up.dtype), up, np.zeros(16, up.dtype)])
    du = dev(gpu, up_buf)
    a = gpu.gelu_act(du, gate_scale=OUT, up_scale=OUT, up_offset=pad)
    dst = gpu.DeviceBuffer.empty((n,), np.int8)
    dst.fill(0x7B)
    gpu.qgemv_gelu(bits, dw, ds, dg, a, dst, k, n, IN, OUT)
    assert np.array_equal(dst.download(), want)


@pytest.mark.parametrize("splits", [2, 4, 8])
def test_gelu_exact_split_and_fold(gpu, oracle, splits):
    """qgemv-4bit-gelu-exact-split: integer partials per K band; the exact fold gives the codes."""
    bits, n, k = 4, 1536, 6144
    rng = np.random.default_rng(splits)
    w = syn.weights("gelu", "down", n, k, bits)
    s = syn.row_scales("gelu", "down_s", n)
    gate, up, act = operands(rng, k, "codes")
    x = act.astype(np.float32) * np.float32(IN)
    want_parts = oracle.qgemv_split(bits, w, s, x, n, k, splits, True, IN)
    _, want_codes = expected(oracle, bits, w, s, act, n, k)
    dw, ds, dg, du = dev(gpu, w), dev(gpu, s), dev(gpu, gate), dev(gpu, up)
    a = gpu.gelu_act(du, gate_scale=OUT, up_scale=OUT)
    parts = gpu.DeviceBuffer.empty((n, splits), np.float32)
    gpu.qgemv_gelu_split(bits, dw, ds, dg, a, parts, k, n, splits, True, IN)
    got = parts.download()
    assert np.array_equal(got.view(np.uint32), want_parts.view(np.uint32))
    dst = gpu.DeviceBuffer.empty((n,), np.int8)
    gpu.qgemv_exact_merge(parts, ds, dst, n, splits, IN, OUT)
    assert np.array_equal(dst.download(), want_codes)


def test_plan_with_prologues(gpu, oracle):
    """A plan mixing a plain projection and two gelu-prologue ones (the runner's down_proj and
    per_layer_projection shapes), launched twice."""
    rng = np.random.default_rng(77)
    items, acts, wants, keep = [], [], [], []
    specs = [(4, 2048, 1536, None), (4, 1536, 6144, "codes"), (8, 1536, 256, "ple")]
    for i, (bits, n, k, form) in enumerate(specs):
        w = syn.weights("gelu", f"p{i}", n, k, bits)
        s = syn.row_scales("gelu", f"ps{i}", n)
        if form is None:
            xc = rng.integers(-128, 128, k).astype(np.int8)
            gate, act_codes, a = xc, xc, None
        else:
            gate, up, act_codes = operands(rng, k, form)
            du = dev(gpu, up)
            keep.append(du)
            a = gpu.gelu_act(du, gate_scale=OUT, up_scale=OUT)
        _, want = expected(oracle, bits, w, s, act_codes, n, k)
        dst = gpu.DeviceBuffer.empty((n,), np.int8)
        dst.fill(0x11)
        items.append(gpu.Gemv(dev(gpu, w), dev(gpu, s), dev(gpu, gate), dst, bits, k, n, IN, OUT))
        acts.append(a)
        wants.append(want)
    plan = gpu.GemvPlan(items, acts)
    for _ in range(2):
        plan.launch()
        gpu.synchronize()
        for it, want in zip(items, wants):
            assert np.array_equal(it.dst.download(), want)
    plan.close()


def test_gelu_refusals(gpu):
    L = gpu.lib()
    a = gpu.GeluAct(0x1000, gpu.KIND_F32, 0.1, 0.1, 0)
    import ctypes

    def call(**kw):
        args = dict(bits=4, k=512, n=16, ins=IN, gk=gpu.KIND_I8, act=a)
        args.update(kw)
        gpu._check(L.g4_qgemv_gelu(args["bits"], 0x1000, 0x1000, 0x1000, args["gk"],
                                   ctypes.byref(args["act"]), 0x1000, gpu.KIND_I8, args["k"],
                                   args["n"], args["ins"], OUT, None))
    with pytest.raises(gpu.G4Error, match="uncalibrated f32 path, which has no int8 input codes"):
        call(ins=0.0)  # an uncalibrated site takes the f32 gate, not codes
    with pytest.raises(gpu.G4Error, match="multiple of 256"):
        call(k=300)
    with pytest.raises(gpu.G4Error, match="gate must be f32 or int8"):
        call(gk=gpu.KIND_F16)
    with pytest.raises(gpu.G4Error, match="aligned"):
        call(act=gpu.GeluAct(0x1004, gpu.KIND_F32, 0.1, 0.1, 0))
    with pytest.raises(gpu.G4Error, match="gate and up"):
        call(act=gpu.GeluAct(None, gpu.KIND_F32, 0.1, 0.1, 0))
