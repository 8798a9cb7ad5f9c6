"""GPU parity of the M-column linears on int8 MFMA (qgemm-4bit, qmatmul-8bit) against the oracle.

Config 2: the gate projection (N 6144, K 1536) with int4 weights and f16 activations carrying 1%
outliers at +-8 sigma, at M in {4, 8, 16, 128, 512, 2048}: every output is compared, at M = 2048
with f16 and with int8-code activations.
"""
import numpy as np
import pytest

import g4synth as syn

pytestmark = pytest.mark.gpu


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(g4, shape, dtype):
    b = g4.DeviceBuffer.empty(shape, dtype)
    b.fill(0x7B)
    return b


def f32_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def test_reference_case_m11_over_tile(gpu, oracle):
    # qgemm.ts:648-673: 8 rows, K 512, 11 columns, grid activations; plain and SRQ.
    g = np.random.default_rng(51)
    w = g.integers(0, 256, size=(8, 256), dtype=np.uint8)
    s = g.uniform(0.005, 0.02, 8).astype(np.float32)
    x = (g.integers(-64, 65, size=(11, 512)) / 8.0).astype(np.float32)
    for ins, outs in ((0.0, 0.0), (0.1875, 0.0625)):
        print(f"qgemm m11 in={ins}", flush=True)
        o = out_buf(gpu, (11, 8), np.float32)
        gpu.bind("qgemm-4bit", {"wq": dev(gpu, w), "scales": dev(gpu, s), "x": dev(gpu, x)}, o,
                 {"k": 512, "numRows": 8, "mCols": 11, "inScale": ins, "outScale": outs})
        want, _, _ = oracle.qgemm(4, w, s, x, 8, 512, 11, ins, outs)
        assert f32_equal(o.download(), want)


@pytest.fixture(scope="module")
def gate(gpu):
    n, k = syn.FFN, syn.HIDDEN
    w = syn.int4_weights("c2", "gate", n, k)
    s = syn.row_scales("c2", "gate", n)
    return n, k, w, s, dev(gpu, w), dev(gpu, s)


@pytest.mark.parametrize("m", [3, 4, 8, 16, 17, 32, 33, 128, 512])
def test_config2_gate_full_compare(gpu, oracle, gate, m):
    n, k, w, s, wb, sb = gate
    x = syn.activations("c2", f"x{m}", m, k, outlier_frac=0.01)
    print(f"config2 m={m} kernel={gpu.kernel_for_shape(4, m, n, k)}", flush=True)
    want, acc, codes = oracle.qgemm(4, w, s, x.astype(np.float32), n, k, m, syn.IN_SCALE,
                                    syn.OUT_SCALE)
    xb = dev(gpu, x)
    o8 = out_buf(gpu, (m, n), np.int8)
    gpu.qgemm(4, wb, sb, xb, o8, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
    assert np.array_equal(o8.download(), codes)
    o32 = out_buf(gpu, (m, n), np.int32)
    gpu.qgemm(4, wb, sb, xb, o32, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
    assert np.array_equal(o32.download(), acc)
    if m in (4, 128):
        of = out_buf(gpu, (m, n), np.float32)
        gpu.qgemm(4, wb, sb, xb, of, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
        assert f32_equal(of.download(), want)


@pytest.mark.parametrize("x_kind", ["f16", "i8"])
def test_config2_gate_m2048_full(gpu, oracle, gate, x_kind):
    """Every output of the M = 2048 gate call against the oracle: f16 activations (the snap pass,
    then the wide kernel on interleaved codes) and int8 codes (the wide kernel's NAT instantiation
    reading the caller's codes in place); int8 codes and int32 accumulators. As a size-independent
    property, a few columns also equal the GEMV kernel's answer for that column alone."""
    n, k, w, s, wb, sb = gate
    m = 2048
    x = syn.activations("c2", "x2048", m, k, outlier_frac=0.01)
    print(f"config2 m=2048 x={x_kind} kernel={gpu.kernel_for_shape(4, m, n, k)}", flush=True)
    _, acc, codes = oracle.qgemm(4, w, s, x.astype(np.float32), n, k, m, syn.IN_SCALE,
                                 syn.OUT_SCALE)
    xin = x if x_kind == "f16" else oracle.srq_codes(x.astype(np.float32), syn.IN_SCALE).reshape(m, k)
    xb = dev(gpu, xin)
    o8 = out_buf(gpu, (m, n), np.int8)
    gpu.qgemm(4, wb, sb, xb, o8, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
    got = o8.download()
    assert np.array_equal(got, codes)
    o32 = out_buf(gpu, (m, n), np.int32)
    gpu.qgemm(4, wb, sb, xb, o32, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
    assert np.array_equal(o32.download(), acc)
    for c in (0, 1000, m - 1):
        o1 = out_buf(gpu, (n,), np.int8)
        gpu.qgemv(4, wb, sb, dev(gpu, xin[c]), o1, k, n, 1, syn.IN_SCALE, syn.OUT_SCALE)
        assert np.array_equal(o1.download(), got[c])


@pytest.mark.parametrize("m,n,k", [(3, 256, 1536), (9, 1536, 256), (40, 1000, 1536),
                                   (130, 300, 6144), (200, 1536, 256)])
def test_qmatmul8_shapes(gpu, oracle, m, n, k):
    w = syn.int8_weights("q8", f"{m}x{n}x{k}", n, k)
    s = syn.row_scales("q8", f"{m}x{n}x{k}", n)
    x = syn.activations("q8", f"{m}x{n}x{k}", m, k)
    print(f"qmatmul8 m={m} n={n} k={k} kernel={gpu.kernel_for_shape(8, m, n, k)}", flush=True)
    want = oracle.qmatmul8(w, s, x.astype(np.float32), n, k, m, 0.05, 0.1)
    of = out_buf(gpu, (m, n), np.float32)
    gpu.bind("qmatmul-8bit", {"wq": dev(gpu, w), "scales": dev(gpu, s), "x": dev(gpu, x)}, of,
             {"k": k, "numRows": n, "mCols": m, "inScale": 0.05, "outScale": 0.1})
    assert f32_equal(of.download(), want)


@pytest.mark.parametrize("m,n", [(37, 1000), (129, 2047), (64, 128)])
def test_int4_partial_tiles(gpu, oracle, m, n):
    k = 2048
    w = syn.int4_weights("tiles", f"{m}x{n}", n, k)
    s = syn.row_scales("tiles", f"{m}x{n}", n)
    x = syn.activations("tiles", f"{m}x{n}", m, k)
    print(f"partial tiles m={m} n={n}", flush=True)
    _, acc, codes = oracle.qgemm(4, w, s, x.astype(np.float32), n, k, m, 0.05, 0.1)
    o32 = out_buf(gpu, (m, n), np.int32)
    gpu.qgemm(4, dev(gpu, w), dev(gpu, s), dev(gpu, x), o32, k, n, m, 0.05, 0.1)
    assert np.array_equal(o32.download(), acc)


def test_uncalibrated_gemm_grid_exact(gpu, oracle):
    g = np.random.default_rng(53)
    w = g.integers(0, 256, size=(64, 256), dtype=np.uint8)
    s = g.uniform(0.005, 0.02, 64).astype(np.float32)
    x = (g.integers(-64, 65, size=(5, 512)) / 8.0).astype(np.float32)
    want, _, _ = oracle.qgemm(4, w, s, x, 64, 512, 5, 0.0, 0.0625)
    of = out_buf(gpu, (5, 64), np.float32)
    gpu.qgemm(4, dev(gpu, w), dev(gpu, s), dev(gpu, x), of, 512, 64, 5, 0.0, 0.0625)
    assert f32_equal(of.download(), want)


@pytest.mark.parametrize("out_kind", ["f32", "i8", "i32"])
def test_tile_epilogue_kinds_m96(gpu, oracle, gate, out_kind):
    # The tile kernel's epilogue for every output kind, over a ragged last M tile (96 = 64 + 32)
    # and every column of the gate shape.
    n, k, w, s, wb, sb = gate
    m = 96
    x = syn.activations("c2", "epi96", m, k, outlier_frac=0.01)
    want, acc, codes = oracle.qgemm(4, w, s, x.astype(np.float32), n, k, m, syn.IN_SCALE,
                                    syn.OUT_SCALE)
    dt = {"f32": np.float32, "i8": np.int8, "i32": np.int32}[out_kind]
    o = out_buf(gpu, (m, n), dt)
    gpu.qgemm(4, wb, sb, dev(gpu, x), o, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
    got = o.download()
    if out_kind == "f32":
        assert f32_equal(got, want)
    elif out_kind == "i8":
        assert np.array_equal(got, codes)
    else:
        assert np.array_equal(got, acc)


def test_tile_int8_codes_in(gpu, oracle, gate):
    # Activation codes already snapped (x_kind int8) through the tile path equal the f16 path.
    n, k, w, s, wb, sb = gate
    m = 200
    x = syn.activations("c2", "codes200", m, k, outlier_frac=0.01)
    _, _, codes = oracle.qgemm(4, w, s, x.astype(np.float32), n, k, m, syn.IN_SCALE, syn.OUT_SCALE)
    xq = np.clip(np.rint(x.astype(np.float32) / np.float32(syn.IN_SCALE)), -128, 127).astype(np.int8)
    o8 = out_buf(gpu, (m, n), np.int8)
    gpu.qgemm(4, wb, sb, dev(gpu, xq), o8, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
    assert np.array_equal(o8.download(), codes)


@pytest.mark.parametrize("bits,m,n,k", [(4, 100, 333, 256), (8, 70, 1001, 128), (8, 65, 77, 384)])
def test_short_k_and_odd_n(gpu, oracle, bits, m, n, k):
    # K of one or two 128-code stages (routed to the small-M kernel or the 3-stage ring) and
    # column counts that are not a multiple of the 8-wide output runs.
    w = syn.weights("shortk", f"{bits}-{m}x{n}x{k}", n, k, bits)
    s = syn.row_scales("shortk", f"{bits}-{m}x{n}x{k}", n)
    x = syn.activations("shortk", f"{bits}-{m}x{n}x{k}", m, k)
    print(f"short k bits={bits} m={m} n={n} k={k} kernel={gpu.kernel_for_shape(bits, m, n, k)}",
          flush=True)
    _, acc, codes = oracle.qgemm(bits, w, s, x.astype(np.float32), n, k, m, 0.05, 0.1)
    o8 = out_buf(gpu, (m, n), np.int8)
    gpu.qgemm(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x), o8, k, n, m, 0.05, 0.1)
    assert np.array_equal(o8.download(), codes)
    o32 = out_buf(gpu, (m, n), np.int32)
    gpu.qgemm(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x), o32, k, n, m, 0.05, 0.1)
    assert np.array_equal(o32.download(), acc)
    # the same rows as int8 codes: the tile path reads them in natural order, with no snap pass
    xq = np.clip(np.rint(x.astype(np.float32) / np.float32(0.05)), -128, 127).astype(np.int8)
    o32.fill(0x7B)
    gpu.qgemm(bits, dev(gpu, w), dev(gpu, s), dev(gpu, xq), o32, k, n, m, 0.05, 0.1)
    assert np.array_equal(o32.download(), acc)


@pytest.mark.parametrize("m,n,k", [(512, 6144, 1536), (300, 12291, 512), (384, 8192, 2048)])
def test_wide_tile_kinds_and_ragged_edges(gpu, oracle, m, n, k):
    # The 64 x 192 tile (8 waves, K halves met through LDS, transposed accumulators): every output
    # kind, f16 activations (snapped, interleaved) and int8 codes (natural order), the config-2
    # gate shape and a ragged one (last M tile 44 rows, last N tile 3 columns, N odd so the packed
    # 4-output stores fall back to single ones on misaligned rows).
    assert gpu.kernel_for_shape(4, m, n, k) == "qgemm-4bit-mfma-wide"
    w = syn.int4_weights("wide", f"{m}x{n}x{k}", n, k)
    s = syn.row_scales("wide", f"{m}x{n}x{k}", n)
    x = syn.activations("wide", f"{m}x{n}x{k}", m, k, outlier_frac=0.01)
    want, acc, codes = oracle.qgemm(4, w, s, x.astype(np.float32), n, k, m, syn.IN_SCALE,
                                    syn.OUT_SCALE)
    xq = np.clip(np.rint(x.astype(np.float32) / np.float32(syn.IN_SCALE)), -128, 127).astype(np.int8)
    wb, sb = dev(gpu, w), dev(gpu, s)
    for src_name, src in (("f16", dev(gpu, x)), ("i8", dev(gpu, xq))):
        for name, dt, ref in (("i8", np.int8, codes), ("i32", np.int32, acc), ("f32", np.float32, want)):
            print(f"wide m={m} n={n} k={k} x={src_name} out={name}", flush=True)
            o = out_buf(gpu, (m, n), dt)
            gpu.qgemm(4, wb, sb, src, o, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
            got = o.download()
            if name == "f32":
                assert f32_equal(got, ref)
            else:
                assert np.array_equal(got, ref), f"{int((got != ref).sum())} outputs differ"
    # f32 output without an output snap (outScale 0): y itself
    y0, _, _ = oracle.qgemm(4, w, s, x.astype(np.float32), n, k, m, syn.IN_SCALE, 0.0)
    o = out_buf(gpu, (m, n), np.float32)
    gpu.qgemm(4, wb, sb, dev(gpu, xq), o, k, n, m, syn.IN_SCALE, 0.0)
    assert f32_equal(o.download(), y0)
