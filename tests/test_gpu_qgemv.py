"""GPU parity of the decode GEMV family (qgemv-4bit / -8bit / -m2) against the oracle.

Bar: int32 accumulators, int8 codes and the reference's f32 dst bit-exact on the calibrated path;
the uncalibrated f32 path bit-exact on exact-grid fixtures and within a stated tolerance elsewhere.
"""
import numpy as np
import pytest

import g4synth as syn

pytestmark = pytest.mark.gpu

SRQ_IN_THIRDS, SRQ_IN_CLAMPING, SRQ_OUT = 0.1875, 0.015625, 0.0625


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(g4, shape, dtype):
    b = g4.DeviceBuffer.empty(shape, dtype)
    b.fill(0x7B)  # sentinel: an element the kernel did not write cannot match the oracle
    return b


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.astype(np.float32).view(np.uint32))
    return np.array_equal(a, b)


def grid_case(rows, k, bits, m=1, seed=0):
    g = np.random.default_rng(seed)
    if bits == 4:
        w = g.integers(0, 256, size=(rows, k // 2), dtype=np.uint8)
    else:
        w = g.integers(-127, 128, size=(rows, k)).astype(np.int8).view(np.uint8)
    s = g.uniform(0.005, 0.02, rows).astype(np.float32)
    x = (g.integers(-64, 65, size=(m, k)) / 8.0).astype(np.float32)
    return w, s, x


@pytest.mark.parametrize("name,bits,rows,k", [("qgemv-4bit", 4, 8, 512), ("qgemv-8bit", 8, 10, 256),
                                              ("qgemv-4bit", 4, 1, 256)])
@pytest.mark.parametrize("in_scale,out_scale", [(0.0, 0.0), (SRQ_IN_THIRDS, SRQ_OUT),
                                                (SRQ_IN_CLAMPING, 0.0)])
def test_reference_cases_through_registry(gpu, oracle, name, bits, rows, k, in_scale, out_scale):
    # The reference's own cases (qgemv.ts:1483-1535, :1603-1656) rebuilt from their recipe.
    print(f"case {name} rows={rows} k={k} in={in_scale} out={out_scale}", flush=True)
    w, s, x = grid_case(rows, k, bits, seed=rows + k)
    out = out_buf(gpu, (rows,), np.float32)
    gpu.bind(name, {"wq": dev(gpu, w), "scales": dev(gpu, s), "x": dev(gpu, x[0])}, out,
             {"k": k, "numRows": rows, "inScale": in_scale, "outScale": out_scale})
    want, _, _ = oracle.qgemv(bits, w, s, x[0], rows, k, in_scale, out_scale)
    assert bits_equal(out.download(), want)


@pytest.mark.parametrize("x_kind", ["f16", "f32", "i8"])
def test_config0_bit_exact(gpu, oracle, x_kind):
    # Config 0: K = N = 1536 int4, x f16 N(0,1), static scales fround(0.05) / fround(0.1).
    n = k = 1536
    w = syn.int4_weights("c0", "w", n, k)
    s = syn.row_scales("c0", "w", n)
    x16 = syn.activations("c0", "x", 1, k)[0]
    x32 = x16.astype(np.float32)
    want, acc, codes = oracle.qgemv(4, w, s, x32, n, k, syn.IN_SCALE, syn.OUT_SCALE)
    if x_kind == "f16":
        xb = dev(gpu, x16)
    elif x_kind == "f32":
        xb = dev(gpu, x32)
    else:
        xb = dev(gpu, oracle.srq_codes(x32, syn.IN_SCALE))
    wb, sb = dev(gpu, w), dev(gpu, s)
    print(f"config0 x_kind={x_kind}", flush=True)
    o8 = out_buf(gpu, (n,), np.int8)
    gpu.qgemv(4, wb, sb, xb, o8, k, n, 1, syn.IN_SCALE, syn.OUT_SCALE)
    assert bits_equal(o8.download(), codes)
    o32 = out_buf(gpu, (n,), np.int32)
    gpu.qgemv(4, wb, sb, xb, o32, k, n, 1, syn.IN_SCALE, syn.OUT_SCALE)
    assert bits_equal(o32.download(), acc)
    of = out_buf(gpu, (n,), np.float32)
    gpu.qgemv(4, wb, sb, xb, of, k, n, 1, syn.IN_SCALE, syn.OUT_SCALE)
    assert bits_equal(of.download(), want)
    # How close the snaps came to a tie: the count the reference's 2.5-ulp WGSL divide could flip.
    y = (np.float32(syn.IN_SCALE) * s).astype(np.float32) * acc.astype(np.float32)
    q = (y / np.float32(syn.OUT_SCALE)).astype(np.float32)
    near = int(np.sum(np.abs(np.abs(q - np.trunc(q)) - 0.5) < 4 * np.spacing(np.abs(q))))
    print(f"config0 near-half output quotients: {near} of {n}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,k", [(10, 256), (1000, 1536), (256, 2048), (1536, 6144),
                                    (77, 16384)])
def test_shapes_and_guards(gpu, oracle, bits, rows, k):
    if bits == 8 and k == 16384:
        k = 8192
    print(f"shape bits={bits} rows={rows} k={k}", flush=True)
    g = np.random.default_rng(rows * 7 + k)
    w = syn.weights("shapes", f"{rows}x{k}", rows, k, bits)
    s = syn.row_scales("shapes", f"{rows}x{k}", rows)
    x = (g.standard_normal(k) * 1.5).astype(np.float16)
    want, acc, codes = oracle.qgemv(bits, w, s, x.astype(np.float32), rows, k, 0.05, 0.1)
    o32 = out_buf(gpu, (rows,), np.int32)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x), o32, k, rows, 1, 0.05, 0.1)
    assert bits_equal(o32.download(), acc)
    o8 = out_buf(gpu, (rows,), np.int8)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x), o8, k, rows, 1, 0.05, 0.1)
    assert bits_equal(o8.download(), codes)


@pytest.mark.parametrize("bits", [4, 8])
def test_wide_m2_each_column_matches(gpu, oracle, bits):
    n, k = 2048, 1536
    w = syn.weights("m2", "w", n, k, bits)
    s = syn.row_scales("m2", "w", n)
    x = syn.activations("m2", "x", 2, k)
    print(f"wide m2 bits={bits}", flush=True)
    want, acc, codes = oracle.qgemm(bits, w, s, x.astype(np.float32), n, k, 2, 0.05, 0.1)
    o8 = out_buf(gpu, (2, n), np.int8)
    gpu.bind(f"qgemv-{bits}bit-m2", {"wq": dev(gpu, w), "scales": dev(gpu, s), "x": dev(gpu, x)},
             o8, {"k": k, "numRows": n, "cols": 2, "inScale": 0.05, "outScale": 0.1})
    assert bits_equal(o8.download(), codes)
    of = out_buf(gpu, (2, n), np.float32)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x), of, k, n, 2, 0.05, 0.1)
    assert bits_equal(of.download(), want)


@pytest.mark.parametrize("bits", [4, 8])
def test_uncalibrated_f32_path(gpu, oracle, bits):
    # Grid fixture: every partial is exact, so bit identity is owed.
    w, s, x = grid_case(40, 1024, bits, seed=3)
    want, _, _ = oracle.qgemv(bits, w, s, x[0], 40, 1024, 0.0, 0.0)
    of = out_buf(gpu, (40,), np.float32)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x[0]), of, 1024, 40, 1, 0.0, 0.0)
    assert bits_equal(of.download(), want)
    # Random f32 activations: the reference's own f32 order is adapter dependent (unpinned); the
    # tolerance is f32 rounding over the K-term sum: |err| <= K * 2^-23 * sum|w*x| * |scale|.
    g = np.random.default_rng(4)
    xr = g.standard_normal(1024).astype(np.float32)
    want, _, _ = oracle.qgemv(bits, w, s, xr, 40, 1024, 0.0, 0.0)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, xr), of, 1024, 40, 1, 0.0, 0.0)
    import npref
    mag = (np.abs(npref.codes(bits, w)).astype(np.float64) @ np.abs(xr).astype(np.float64)) * s
    tol = 1024 * 2.0 ** -23 * mag + 1e-30
    assert np.all(np.abs(of.download().astype(np.float64) - want) <= tol)
