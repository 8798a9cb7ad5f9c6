"""Pins of the oracle's linear restatement (CPU): qgemvOracle, qgemmOracle, qmatmul8Oracle, the
split-K band cut and its folds, and the reference's 32-lane reduction structure.

Fixture recipes follow the reference's own (qgemv.ts:1365-1388): integer codes against activations
on the 1/8 grid make every f32 partial exact; SRQ scale 0.1875 cuts the 1/8 grid into thirds so no
quotient sits on a half; 0.015625 drives the activations into the int8 clamp; 0.0625 is the output
scale; 10 rows against 4 per workgroup and 11 columns against a tile of 8 exercise the guards.
"""
import numpy as np
import pytest

import npref

SRQ_IN_THIRDS, SRQ_IN_CLAMPING, SRQ_OUT = 0.1875, 0.015625, 0.0625


def grid_fixture(rows, k, m=1, bits=4, seed=0):
    g = np.random.default_rng(seed)
    nbytes = k // 2 if bits == 4 else k
    if bits == 4:
        packed = g.integers(0, 256, size=(rows, nbytes), dtype=np.uint8)
    else:
        packed = g.integers(-127, 128, size=(rows, nbytes)).astype(np.int8).view(np.uint8)
    scales = g.uniform(0.005, 0.02, size=rows).astype(np.float32)
    x = (g.integers(-64, 65, size=(m, k)) / 8.0).astype(np.float32)  # the 1/8 grid
    return packed, scales, x


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("in_scale,out_scale", [(0.0, 0.0), (SRQ_IN_THIRDS, SRQ_OUT),
                                                (SRQ_IN_CLAMPING, 0.0), (0.0, SRQ_OUT)])
def test_qgemv_grid_fixture_matches_numpy(oracle, bits, in_scale, out_scale):
    packed, scales, x = grid_fixture(10, 512, bits=bits, seed=bits)
    dst, acc, q = oracle.qgemv(bits, packed, scales, x[0], 10, 512, in_scale, out_scale)
    racc, y, rq, rdst = npref.linear(bits, packed, scales, x, in_scale, out_scale)
    assert np.array_equal(dst.view(np.uint32), rdst[0].view(np.uint32))
    if in_scale != 0:
        assert np.array_equal(acc, racc[0])
    if out_scale != 0:
        assert np.array_equal(q, rq[0])


def test_qgemv_clamped_input_really_clamps(oracle):
    packed, scales, x = grid_fixture(8, 512, seed=5)
    xq = oracle.srq_codes(x[0], SRQ_IN_CLAMPING)
    assert np.mean(np.abs(xq.astype(int)) >= 127) > 0.5  # most of the fixture hits the clamp


def test_qgemv_random_config0_integer_path(oracle):
    # Config 0 shape with seeded random data: int32 accumulators equal numpy's integer matmul.
    g = np.random.default_rng(11)
    n, k = 1536, 1536
    packed = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = g.uniform(0.005, 0.02, size=n).astype(np.float32)
    x = g.standard_normal(k).astype(np.float16).astype(np.float32)
    dst, acc, q = oracle.qgemv(4, packed, scales, x, n, k, 0.05, 0.1)
    racc, y, rq, rdst = npref.linear(4, packed, scales, x, np.float32(0.05), np.float32(0.1))
    assert np.array_equal(acc, racc[0])
    assert np.array_equal(q, rq[0])
    assert np.array_equal(dst.view(np.uint32), rdst[0].view(np.uint32))


def test_epilogue_order_is_discriminating(oracle):
    # f32(f32(xs*s)*acc) against the plausible wrong order f32(xs*f32(s*acc)): find inputs where
    # the two differ and check the oracle takes the reference's (qgemv.ts:1168-1172).
    g = np.random.default_rng(12)
    xs = np.float32(0.05)
    s = g.uniform(0.005, 0.02, 20000).astype(np.float32)
    acc = g.integers(-200000, 200000, 20000).astype(np.float32)
    right = (xs * s).astype(np.float32) * acc
    wrong = xs * (s * acc).astype(np.float32)
    assert np.any(right.astype(np.float32) != wrong.astype(np.float32))
    i = int(np.nonzero(right.astype(np.float32) != wrong.astype(np.float32))[0][0])
    # One row of codes summing to acc[i] against xq: build a K=256 row with a single live code.
    k = 256
    target = int(acc[i])
    # Spell `target` as sum(code * xq) with codes 7 (bulk) and 1 (remainder), |xq| <= 127.
    codes = np.zeros(k, np.int8)
    xq = np.zeros(k, np.float32)
    rem, j = target, 0
    while abs(rem) >= 7 * 127:
        step = 127 if rem > 0 else -127
        codes[j], xq[j] = 7, step
        rem -= 7 * step
        j += 1
    q, r = int(rem / 7), rem - 7 * int(rem / 7)
    codes[j], xq[j] = 7, q
    codes[j + 1], xq[j + 1] = 1, r
    rem -= 7 * q + r
    assert rem == 0
    packed = oracle.pack(4, codes)[None, :]
    x = (xq * xs).astype(np.float32)  # snaps back to xq exactly: xq*0.05/0.05 is within an ulp
    dst, a, _ = oracle.qgemv(4, packed, np.array([s[i]], np.float32), x, 1, k, float(xs), 0.0)
    assert int(a[0]) == target
    assert dst[0] == right[i].astype(np.float32)


def test_qgemm_is_gemv_per_column_with_masked_tile(oracle):
    # qgemm.ts:523-530 / the M=11 case: every column equals the one-column GEMV.
    packed, scales, x = grid_fixture(8, 512, m=11, seed=7)
    out, acc, q = oracle.qgemm(4, packed, scales, x, 8, 512, 11, SRQ_IN_THIRDS, SRQ_OUT)
    for c in range(11):
        d, a, qq = oracle.qgemv(4, packed, scales, x[c], 8, 512, SRQ_IN_THIRDS, SRQ_OUT)
        assert np.array_equal(out[c], d) and np.array_equal(acc[c], a) and np.array_equal(q[c], qq)
    racc, y, rq, rdst = npref.linear(4, packed, scales, x, SRQ_IN_THIRDS, SRQ_OUT)
    assert np.array_equal(acc, racc) and np.array_equal(q, rq)


def test_integer_accumulator_is_linear_in_codes(oracle):
    # Size-independent property: acc(x1) + acc(x2) == acc over the summed codes.
    g = np.random.default_rng(13)
    n, k = 64, 1024
    packed = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = np.ones(n, np.float32)
    x1 = g.integers(-60, 60, k).astype(np.float32)
    x2 = g.integers(-60, 60, k).astype(np.float32)
    _, a1, _ = oracle.qgemv(4, packed, scales, x1, n, k, 1.0, 0.0)
    _, a2, _ = oracle.qgemv(4, packed, scales, x2, n, k, 1.0, 0.0)
    _, a12, _ = oracle.qgemv(4, packed, scales, x1 + x2, n, k, 1.0, 0.0)
    assert np.array_equal(a1.astype(np.int64) + a2, a12)


def test_qmatmul8_calibrated_equals_gemm_and_f32_order_brute_force(oracle):
    packed, scales, x = grid_fixture(10, 256, m=3, bits=8, seed=9)
    a = oracle.qmatmul8(packed, scales, x, 10, 256, 3, SRQ_IN_THIRDS, SRQ_OUT)
    b, _, _ = oracle.qgemm(8, packed, scales, x, 10, 256, 3, SRQ_IN_THIRDS, SRQ_OUT)
    assert np.array_equal(a, b)
    # Uncalibrated: the shader's serial vec4 order (pleMatmul.ts:212-222) replayed in numpy f32 on
    # random (non-grid) activations, where the order matters.
    g = np.random.default_rng(10)
    xr = g.standard_normal((2, 256)).astype(np.float32)
    got = oracle.qmatmul8(packed, scales, xr, 10, 256, 2, 0.0, 0.0)
    w = npref.codes_int8(packed).astype(np.float32)
    for c in range(2):
        for r in range(10):
            total = np.float32(0)
            for wd in range(64):
                d = np.float32(0)
                for j in range(4):
                    d = np.float32(d + np.float32(w[r, wd * 4 + j] * xr[c, wd * 4 + j]))
                total = np.float32(total + d)
            want = np.float32(np.float32(scales[r]) * total)
            assert got[c, r] == want


def test_split_bands_partition_k_and_fold(oracle):
    g = np.random.default_rng(14)
    n, k = 24, 1536
    packed = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = g.uniform(0.005, 0.02, n).astype(np.float32)
    x = g.standard_normal(k).astype(np.float16).astype(np.float32)
    _, acc, _ = oracle.qgemv(4, packed, scales, x, n, k, 0.05, 0.0)
    w = npref.codes_int4(packed)
    xq = npref.snap(x, 0.05).astype(np.int64)
    for splits in (2, 4, 8):
        raw = oracle.qgemv_split(4, packed, scales, x, n, k, splits, True, 0.05)
        assert np.array_equal(raw.sum(axis=1).astype(np.int64), acc)  # the bands partition K
        # qgemv.ts:521-548: kWords 192, kIters 6, slots 6 (exact) -> per = ceil(6/splits)
        per = -(-6 // splits)
        for s in range(splits):
            lo, hi = min(s * per, 6) * 256, min(min(s * per, 6) + per, 6) * 256
            assert np.array_equal(raw[:, s], (w[:, lo:hi] @ xq[lo:hi]).astype(np.float32))
        scaled = oracle.qgemv_split(4, packed, scales, x, n, k, splits, False, 0.05)
        per = -(-7 // splits)  # scaled partials count the tail slot: slots = 7
        for s in range(splits):
            lo = min(s * per, 7)
            hi = min(lo + per, 7)
            a, b = lo * 256, min(hi, 6) * 256
            band = (w[:, a:max(a, b)] @ xq[a:max(a, b)]).astype(np.float32)
            want = ((np.float32(0.05) * scales).astype(np.float32) * band).astype(np.float32)
            assert np.array_equal(scaled[:, s], want)
        folded = oracle.qgemv_merge(scaled, 0.1)
        t = np.zeros(n, np.float32)
        for s in range(splits):
            t = (t + scaled[:, s]).astype(np.float32)
        assert np.array_equal(folded, (npref.snap(t, 0.1) * np.float32(0.1)).astype(np.float32))
        exact = oracle.qgemv_exact_merge(raw, scales, 0.05, 0.1)
        _, y, rq, rdst = npref.linear(4, packed, scales, x, np.float32(0.05), np.float32(0.1))
        assert np.array_equal(exact, rdst[0])


def test_reference_lane_reduction_agrees_below_2_24_and_rounds_above(oracle):
    g = np.random.default_rng(15)
    k = 6144
    # Config-1 int8 down projection magnitudes: every lane partial far below 2^24.
    row = g.integers(-127, 128, k).astype(np.int8).view(np.uint8)
    xq = npref.snap(g.standard_normal(k).astype(np.float16).astype(np.float32), 0.05).astype(np.int8)
    exact = int(npref.codes_int8(row) @ xq.astype(np.int64))
    assert oracle.qgemv_ref_lane_sum(8, row, xq, k) == np.float32(exact)
    # Adversarial: every product 127*127 -> total 99M > 2^24; replay the 32-lane butterfly in
    # numpy f32 and check the oracle follows it (and that it differs from fround(exact) here).
    row = np.full(k, 127, np.int8).view(np.uint8)
    xq = np.full(k, 127, np.int8)
    lanes = np.zeros(32, np.float32)
    kw = k // 4
    for l in range(32):
        acc = 0
        for wd in range(l, kw, 32):
            acc += 4 * 127 * 127
        lanes[l] = np.float32(acc)
    for m in (1, 2, 4, 8, 16):
        lanes = (lanes + lanes[np.arange(32) ^ m]).astype(np.float32)
    assert oracle.qgemv_ref_lane_sum(8, row, xq, k) == lanes[0]
    assert abs(int(lanes[0]) - k * 127 * 127) < 64
