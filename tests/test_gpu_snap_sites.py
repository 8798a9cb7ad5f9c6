"""Every SRQ snap site on the device against the oracle's IEEE divide, on inputs where the
reciprocal fast path alone would round the other way (tests/snapcases.py builds them).

Sites: the streaming GEMV's activation snap and output snap (M = 1), the generic GEMV (M = 2),
the small-M MFMA kernel's fused snap and epilogue (4- and 16-wave grids), quantize_rows and the
tile kernel's epilogue (M > 32, f32 and int8 codes in), the wide tile's grouped epilogue
(M >= 256), the standalone srq kernel, and the gelu prologue. Each site also runs the in-tree known answer srqCodes(-11.435039520263672,
0.6181102395057678) = -18 (quant.ts:324-329) as an activation and as an output.
Also here: uncalibrated qmatmul-8bit in the reference's serial vec4 f32 order
(pleMatmul.ts:212-222) against or_qmatmul8 on off-grid inputs."""
import numpy as np
import pytest

import decode_oracle as d
import g4synth as syn
import snapcases as sc

pytestmark = pytest.mark.gpu

F = np.float32


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(g4, shape, dtype):
    b = g4.DeviceBuffer.empty(shape, dtype)
    b.fill(0x7B)
    return b


def f32_equal(a, b):
    return np.array_equal(np.asarray(a, F).view(np.uint32), np.asarray(b, F).view(np.uint32))


def case(oracle, bits, m, n, k, mode, seed):
    """(w, scales, x f32 [m, k], in_scale, out_scale, oracle (y, acc, codes)) with adversarial
    activations planted in x and row scales tuned onto adversarial outputs."""
    g = np.random.default_rng(seed)
    w = syn.weights("snap", f"w{bits}_{n}_{k}", n, k, bits)
    s0 = syn.row_scales("snap", f"s{n}", n)
    if mode == "adv":
        sin, sout, vin, vout = sc.S_IN, sc.S_OUT, sc.ADV_IN, sc.ADV_OUT
        x = g.standard_normal((m, k)).astype(F) * F(2.0)
    else:  # the known answer, as an input code and as an output code
        sin, sout, vin, vout = sc.KA_SCALE, sc.KA_SCALE, [sc.KA_VALUE], [sc.KA_VALUE]
        x = g.standard_normal((m, k)).astype(F) * F(20.0)
    x = sc.plant(x, vin, every=5, offset=seed % 5)
    _, acc, _ = oracle.qgemm(bits, w, s0, x, n, k, m, sin, sout)
    s, tuned = sc.tune_row_scales(acc, s0, sin, vout)
    y, acc, codes = oracle.qgemm(bits, w, s, x, n, k, m, sin, sout)
    # the case must be adversarial at both kinds of site, or it pins nothing
    flat = x.reshape(-1)
    assert (sc.divide_code(flat, sin) != sc.recip_code(flat, sin)).sum() >= 8 or mode == "ka"
    assert (sc.divide_code(flat, sin) == -18).any() or mode == "adv"
    pre = (F(sin) * s)[None, :] * acc.astype(F)
    if mode == "adv":
        diff = sc.divide_code(pre, sout) != sc.recip_code(pre, sout)
        assert diff.sum() >= 4, "no adversarial output in the case"
    else:  # exact ties at -18.5 / 18.5, where an f64 divide would round away
        assert (np.abs(pre) == -sc.KA_VALUE).sum() >= 4, "no known-answer output in the case"
    return w, s, x, sin, sout, (y, acc, codes)


def check(got, want_tuple, out_kind, g4):
    y, acc, codes = want_tuple
    if out_kind == g4.KIND_I8:
        assert np.array_equal(got, codes), f"{int((got != codes).sum())} codes differ"
    elif out_kind == g4.KIND_I32:
        assert np.array_equal(got, acc), f"{int((got != acc).sum())} accumulators differ"
    else:
        assert f32_equal(got, y)


KINDS = [("i8", np.int8), ("i32", np.int32), ("f32", F)]


@pytest.mark.parametrize("mode", ["adv", "ka"])
@pytest.mark.parametrize("bits", [4, 8])
def test_stream_gemv_snap(gpu, oracle, bits, mode):
    """M = 1, f32 x, K = 1536: the streaming kernel's activation snap and output snap."""
    n, k = 1536, 1536
    w, s, x, sin, sout, want = case(oracle, bits, 1, n, k, mode, 11 + bits)
    assert gpu.kernel_for_shape(bits, 1, n, k).endswith("-stream")
    dw, ds, dx = dev(gpu, w), dev(gpu, s), dev(gpu, x[0])
    for name, dt in KINDS:
        print(f"stream bits={bits} mode={mode} out={name}", flush=True)
        dst = out_buf(gpu, (n,), dt)
        gpu.qgemv(bits, dw, ds, dx, dst, k, n, 1, sin, sout)
        check(dst.download()[None], want, dst.kind, gpu)


@pytest.mark.parametrize("mode", ["adv", "ka"])
def test_wide_gemv_snap(gpu, oracle, mode):
    """M = 2 (qgemv-4bit-m2): the generic GEMV's snap and epilogue."""
    n, k = 1024, 1536
    w, s, x, sin, sout, want = case(oracle, 4, 2, n, k, mode, 21)
    dw, ds, dx = dev(gpu, w), dev(gpu, s), dev(gpu, x)
    for name, dt in KINDS:
        print(f"wide mode={mode} out={name}", flush=True)
        dst = out_buf(gpu, (2, n), dt)
        gpu.qgemv(4, dw, ds, dx, dst, k, n, 2, sin, sout)
        check(dst.download(), want, dst.kind, gpu)


@pytest.mark.parametrize("mode", ["adv", "ka"])
@pytest.mark.parametrize("bits,m,n", [(4, 4, 6144), (4, 16, 1536), (4, 32, 6144), (8, 8, 1536),
                                      (8, 32, 256)])
def test_small_m_snap(gpu, oracle, bits, m, n, mode):
    """3 <= M <= 32: the small-M kernel's fused activation snap and its epilogue snap, on the
    4-wave grid (many blocks) and the 16-wave grid (no wider than the CU count)."""
    k = 1536
    w, s, x, sin, sout, want = case(oracle, bits, m, n, k, mode, 31 + m + bits)
    assert "small" in gpu.kernel_for_shape(bits, m, n, k)
    dw, ds, dx = dev(gpu, w), dev(gpu, s), dev(gpu, x)
    for name, dt in KINDS:
        print(f"small bits={bits} m={m} n={n} mode={mode} out={name}", flush=True)
        dst = out_buf(gpu, (m, n), dt)
        gpu.qgemm(bits, dw, ds, dx, dst, k, n, m, sin, sout)
        check(dst.download(), want, dst.kind, gpu)


@pytest.mark.parametrize("mode", ["adv", "ka"])
@pytest.mark.parametrize("bits", [4, 8])
def test_tile_snap(gpu, oracle, bits, mode):
    """M > 32: quantize_rows (f32 in) and the tile kernel's epilogue snap; int8 codes in take the
    natural-order tile kernel with the same epilogue."""
    m, n, k = 96, 1536, 1536
    w, s, x, sin, sout, want = case(oracle, bits, m, n, k, mode, 41 + bits)
    assert "tile" in gpu.kernel_for_shape(bits, m, n, k)
    dw, ds = dev(gpu, w), dev(gpu, s)
    codes = oracle.srq_codes(x.reshape(-1), sin).reshape(m, k)
    for src_name, src in (("f32", dev(gpu, x)), ("i8", dev(gpu, codes))):
        for name, dt in KINDS:
            print(f"tile bits={bits} mode={mode} x={src_name} out={name}", flush=True)
            dst = out_buf(gpu, (m, n), dt)
            gpu.qgemm(bits, dw, ds, src, dst, k, n, m, sin, sout)
            check(dst.download(), want, dst.kind, gpu)


@pytest.mark.parametrize("mode", ["adv", "ka"])
def test_wide_tile_snap(gpu, oracle, mode):
    """M >= 256 over a grid that fills the device: the 64 x 192 tile's grouped epilogue snap
    (one divide fallback per group of 4 outputs), f32 and int8 codes in."""
    m, n, k = 512, 6144, 512
    w, s, x, sin, sout, want = case(oracle, 4, m, n, k, mode, 47)
    assert gpu.kernel_for_shape(4, m, n, k) == "qgemm-4bit-mfma-wide"
    dw, ds = dev(gpu, w), dev(gpu, s)
    codes = oracle.srq_codes(x.reshape(-1), sin).reshape(m, k)
    for src_name, src in (("f32", dev(gpu, x)), ("i8", dev(gpu, codes))):
        for name, dt in KINDS:
            print(f"wide mode={mode} x={src_name} out={name}", flush=True)
            dst = out_buf(gpu, (m, n), dt)
            gpu.qgemm(4, dw, ds, src, dst, k, n, m, sin, sout)
            check(dst.download(), want, dst.kind, gpu)


def test_srq_quantize_snap(gpu, oracle):
    """The standalone srq kernel on planted adversarial values and the known answer."""
    g = np.random.default_rng(7)
    for s, vals in ((sc.S_IN, sc.ADV_IN), (sc.S_OUT, sc.ADV_OUT), (sc.KA_SCALE, [sc.KA_VALUE])):
        x = sc.plant(g.standard_normal(40_001).astype(F) * F(4.0), vals, every=3)
        codes = out_buf(gpu, (x.size,), np.int8)
        dx = dev(gpu, x)
        gpu.srq_quantize(dx, codes, x.size, s)
        want = oracle.srq_codes(x, s)
        assert np.array_equal(codes.download(), want)
        assert (sc.divide_code(x, s) != sc.recip_code(x, s)).any() or s == sc.KA_SCALE
    assert oracle.srq_codes(np.array([sc.KA_VALUE], F), sc.KA_SCALE)[0] == -18


@pytest.mark.parametrize("bits", [4, 8])
def test_gelu_prologue_snap(gpu, oracle, bits):
    """qgemv-4/8bit-gelu: gelu(gate) * up lands on the adversarial activations, so the prologue's
    snap must take the divide there."""
    n, k = 512, 1536
    g = np.random.default_rng(51 + bits)
    gate = g.uniform(0.5, 3.0, k).astype(F)
    gl = np.array([d.gelu_tanh(float(v)) for v in gate], F)
    targets = np.array(sc.ADV_IN + [-v for v in sc.ADV_IN], F)[np.arange(k) % 6]
    up = sc.solve_factor(gl, targets)
    hit = ~np.isnan(up)
    up[~hit] = g.standard_normal((~hit).sum()).astype(F)
    act = d.gelu_mul_f32_codes(gate, up, sc.S_IN)
    prod = gl * up
    assert (sc.divide_code(prod, sc.S_IN) != sc.recip_code(prod, sc.S_IN)).sum() >= 100
    w = syn.weights("snap", f"gw{bits}", n, k, bits)
    s = syn.row_scales("snap", "gs", n)
    x = act.astype(F) * F(sc.S_IN)  # round-trips to the same codes in the oracle's snap
    _, acc, codes = oracle.qgemv(bits, w, s, x, n, k, sc.S_IN, sc.S_OUT)
    # every device buffer stays referenced until its outputs are read back: a GeluAct holds only
    # the up buffer's address
    du, dw, ds, dg = dev(gpu, up), dev(gpu, w), dev(gpu, s), dev(gpu, gate)
    a = gpu.gelu_act(du)
    for name, dt in (("i8", np.int8), ("i32", np.int32)):
        dst = out_buf(gpu, (n,), dt)
        gpu.qgemv_gelu(bits, dw, ds, dg, a, dst, k, n, sc.S_IN, sc.S_OUT)
        want = codes if name == "i8" else acc
        assert np.array_equal(dst.download(), want), name


@pytest.mark.parametrize("m", [1, 3, 64])
def test_qmatmul8_uncalibrated_serial_order(gpu, oracle, m):
    """qmatmul-8bit with inScale 0 (pleMatmul.ts:212-222): per output, a serial loop over K/4
    words, each word's four products summed in order from 0, then added to the accumulator, all in
    f32. Off-grid f32 inputs make every partial round, so any other order shows."""
    n, k = 300, 1536
    g = np.random.default_rng(61 + m)
    w = syn.int8_weights("snap", "qm8", n, k)
    s = g.uniform(0.005, 0.02, n).astype(F)
    x = (g.standard_normal((m, k)) * 1.7).astype(F)
    want = oracle.qmatmul8(w, s, x, n, k, m, 0.0, 0.0)
    # the order matters on these inputs: a pairwise sum of the same products differs somewhere
    prods = w.view(np.int8)[None].astype(F) * x[:, None, :]
    pair = prods.reshape(m, n, -1, 2).sum(axis=3, dtype=F).sum(axis=2, dtype=F) * s[None]
    assert not f32_equal(pair, want)
    inputs = {"wq": dev(gpu, w), "scales": dev(gpu, s), "x": dev(gpu, x)}
    for out_scale in (0.0, float(F(0.1))):
        dst = out_buf(gpu, (m, n), F)
        gpu.bind("qmatmul-8bit", inputs, dst,
                 {"k": k, "numRows": n, "mCols": m, "inScale": 0.0, "outScale": out_scale})
        want = oracle.qmatmul8(w, s, x, n, k, m, 0.0, out_scale)
        assert f32_equal(dst.download(), want), out_scale
