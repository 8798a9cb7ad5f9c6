"""GPU parity of qgemv-4bit's tile8u geometry (qgemv.ts:870-1015) through the C ABI: the repack
into the eight-row tile layout against numpy, and g4_qgemv_tile8u against or_qgemv_tile8u bit for
bit, on both paths (calibrated int8 codes, uncalibrated f32 in the loop's own order), every input
and output kind, ragged row counts, and the gelu prologue; then through the registry seam with the
4-bit geometry's inner loop set to tile8u."""
import numpy as np
import pytest

import decode_oracle as d
import g4synth as syn

pytestmark = pytest.mark.gpu

IN, OUT = syn.IN_SCALE, syn.OUT_SCALE


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def tile_layout(oracle, w, n, k):
    """numpy: word [t][k] holds row 8t + r's unsigned code at bits 4r (rows past n: code 8)."""
    u = oracle.unpack(4, w.reshape(-1), n * k).reshape(n, k).astype(np.int64) + 8
    tiles = (n + 7) // 8
    pad = np.full((tiles * 8, k), 8, np.int64)
    pad[:n] = u
    pad = pad.reshape(tiles, 8, k)
    words = np.zeros((tiles, k), np.uint64)
    for r in range(8):
        words |= pad[:, r, :].astype(np.uint64) << np.uint64(4 * r)
    return words.astype(np.uint32)


def repacked(gpu, w, n, k):
    dw = dev(gpu, w)
    tw = gpu.DeviceBuffer(gpu.tile8u_bytes(k, n), np.uint32)
    gpu.tile8u_repack(dw, tw, k, n)
    return tw


@pytest.mark.parametrize("n,k", [(77, 512), (16, 256), (1536, 1536)])
def test_repack_layout(gpu, oracle, n, k):
    print(f"tile8u repack n={n} k={k}", flush=True)
    w = syn.int4_weights("t8", f"r{n}_{k}", n, k)
    got = repacked(gpu, w, n, k).download().reshape(-1, k)
    assert np.array_equal(got, tile_layout(oracle, w, n, k))


@pytest.mark.parametrize("n,k", [(77, 256), (1536, 1536), (200, 6144), (24, 16384)])
@pytest.mark.parametrize("x_kind", ["f32", "f16", "i8"])
def test_calibrated(gpu, oracle, n, k, x_kind):
    print(f"tile8u calibrated n={n} k={k} x={x_kind}", flush=True)
    w = syn.int4_weights("t8", f"c{n}_{k}", n, k)
    s = syn.row_scales("t8", f"c{n}_{k}", n)
    x = syn.activations("t8", f"x{k}", 1, k, outlier_frac=0.01)[0].astype(np.float32)
    if x_kind == "f16":
        x = x.astype(np.float16)
        xin = x
    elif x_kind == "i8":
        xin = oracle.srq_codes(x, IN)
    else:
        xin = x
    x32 = x.astype(np.float32) if x_kind != "i8" else xin.astype(np.float32) * np.float32(IN)
    want_f, want_c = oracle.qgemv_tile8u(w, s, x32, n, k, IN, OUT)
    classic_f, _, _ = oracle.qgemv(4, w, s, x32, n, k, IN, OUT)
    assert np.array_equal(want_f.view(np.uint32), classic_f.view(np.uint32))
    tw, ds, dx = repacked(gpu, w, n, k), dev(gpu, s), dev(gpu, xin)
    for kind, want in (("f32", want_f), ("i8", want_c)):
        dst = gpu.DeviceBuffer.empty((n,), np.float32 if kind == "f32" else np.int8)
        dst.fill(0x7B)
        gpu.qgemv_tile8u(tw, ds, dx, dst, k, n, IN, OUT)
        got = dst.download()
        if kind == "f32":
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())
        else:
            assert np.array_equal(got, want), int((got != want).sum())


@pytest.mark.parametrize("n,k", [(77, 256), (1536, 1536), (64, 6144)])
@pytest.mark.parametrize("out_scale", [0.0, OUT])
def test_uncalibrated_f32_order(gpu, oracle, n, k, out_scale):
    print(f"tile8u f32 n={n} k={k} out={out_scale}", flush=True)
    w = syn.int4_weights("t8", f"u{n}_{k}", n, k)
    s = syn.row_scales("t8", f"u{n}_{k}", n)
    rng = np.random.default_rng(n + k)
    x = (rng.standard_normal(k) * 3.0).astype(np.float32)
    want, _ = oracle.qgemv_tile8u(w, s, x, n, k, 0.0, out_scale)
    dst = gpu.DeviceBuffer.empty((n,), np.float32)
    dst.fill(0x7B)
    gpu.qgemv_tile8u(repacked(gpu, w, n, k), dev(gpu, s), dev(gpu, x), dst, k, n, 0.0, out_scale)
    got = dst.download()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())


@pytest.mark.parametrize("calibrated", [True, False])
@pytest.mark.parametrize("gate_form", ["codes", "f32"])
def test_gelu_prologue(gpu, oracle, calibrated, gate_form):
    n, k = 96, 1536
    print(f"tile8u gelu calibrated={calibrated} gate={gate_form}", flush=True)
    rng = np.random.default_rng(7 + calibrated)
    w = syn.int4_weights("t8", "gelu", n, k)
    s = syn.row_scales("t8", "gelu", n)
    if gate_form == "codes":
        gc = rng.integers(-128, 128, k).astype(np.int8)
        g = gc.astype(np.float32) * np.float32(OUT)
        gate = gc
    else:
        g = (rng.standard_normal(k) * 2.5).astype(np.float32)
        gate = g
    up = (rng.standard_normal(k) * 1.5).astype(np.float32)
    vals = np.array([np.float32(d.gelu_tanh(float(g[i]))) * up[i] for i in range(k)], np.float32)
    in_scale = IN if calibrated else 0.0
    want, _ = oracle.qgemv_tile8u(w, s, vals, n, k, in_scale, OUT)
    pad = 64
    du = dev(gpu, np.concatenate([np.zeros(pad, np.float32), up, np.zeros(16, np.float32)]))
    act = gpu.gelu_act(du, gate_scale=OUT, up_offset=pad)
    dst = gpu.DeviceBuffer.empty((n,), np.float32)
    dst.fill(0x7B)
    gpu.qgemv_tile8u(repacked(gpu, w, n, k), dev(gpu, s), dev(gpu, gate), dst, k, n, in_scale, OUT,
                     act=act)
    got = dst.download()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())


def test_registry_routes_tile8u(gpu, oracle):
    """bind('qgemv-4bit') with the 4-bit geometry's inner loop set to tile8u reads the tile layout;
    back on the classic loop it reads the row layout; the split is refused as the reference does."""
    n, k = 256, 1536
    w = syn.int4_weights("t8", "reg", n, k)
    s = syn.row_scales("t8", "reg", n)
    x = syn.activations("t8", "reg", 1, k)[0].astype(np.float32)
    want, _, _ = oracle.qgemv(4, w, s, x, n, k, IN, OUT)
    ds, dx = dev(gpu, s), dev(gpu, x)
    out = gpu.DeviceBuffer.empty((n,), np.float32)
    params = {"k": k, "numRows": n, "inScale": IN, "outScale": OUT}
    try:
        gpu.set_gemv_inner(4, "tile8u")
        gpu.bind("qgemv-4bit", {"wq": repacked(gpu, w, n, k), "scales": ds, "x": dx}, out, params)
        assert np.array_equal(out.download().view(np.uint32), want.view(np.uint32))
        with pytest.raises(gpu.G4Error, match="tile8u has no K split"):
            gpu.bind("qgemv-4bit-split", {"wq": dev(gpu, w), "scales": ds, "x": dx},
                     gpu.DeviceBuffer.empty((n, 2), np.float32), dict(params, kSplits=2))
    finally:
        gpu.set_gemv_inner(4, "classic")
    out.fill(0)
    gpu.bind("qgemv-4bit", {"wq": dev(gpu, w), "scales": ds, "x": dx}, out, params)
    assert np.array_equal(out.download().view(np.uint32), want.view(np.uint32))


def test_refusals(gpu):
    t = gpu.DeviceBuffer(gpu.tile8u_bytes(512, 8), np.uint32)
    s = gpu.DeviceBuffer.empty((8,), np.float32)
    x = gpu.DeviceBuffer.empty((512,), np.float32)
    out = gpu.DeviceBuffer.empty((8,), np.float32)
    with pytest.raises(gpu.G4Error, match="multiple of 256"):
        gpu.qgemv_tile8u(t, s, x, out, 384, 8, IN, OUT)
    with pytest.raises(gpu.G4Error, match="calibrated outScale"):
        gpu.qgemv_tile8u(t, s, x, gpu.DeviceBuffer.empty((8,), np.int8), 512, 8, IN, 0.0)
    with pytest.raises(gpu.G4Error, match="inner must be"):
        gpu.set_gemv_inner(4, "tile16u")
