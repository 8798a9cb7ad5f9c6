"""Pins of or_qgemv_tile8u, the oracle of qgemv-4bit's tile8u loop (qgemv.ts:870-1015).

- Calibrated: the loop's sum is the exact integer sum(code * xq), so the result must equal the
  classic oracle's (or_qgemv, qgemvOracle qgemv.ts:1131-1176) bit for bit on random data.
- Uncalibrated on the reference's exact-grid fixtures (codes on the integer grid, activations on
  the 1/8 grid with bounded magnitude, qgemv.ts:1365-1388): every order is exact, so the result
  equals or_qgemv bit for bit; a dropped zero point, a wrong row or a lost element fails here.
- Uncalibrated on random data: within a bound of the f64 sum, and equal to a replay of the shader
  text in Python float32 on tiny K (lane l over k = 128 i + 4 l + j, the multiply and the add each
  rounded, then the sgSum32 butterfly 1, 2, 4, 8, 16). The grid check cannot see the lane mapping
  (any permutation of an exact sum is exact); the replay can, because off the grid the order
  shows in the last bits.
"""
import numpy as np
import pytest

import oracle as o


def rand_w(rng, n, k):
    codes = rng.integers(-8, 8, size=(n, k)).astype(np.int8)
    return codes, o.pack_matrix(4, codes)


@pytest.mark.parametrize("n,k", [(13, 256), (40, 1536), (8, 6144)])
def test_calibrated_equals_classic(n, k):
    rng = np.random.default_rng(n * 7 + k)
    _, w = rand_w(rng, n, k)
    s = rng.uniform(0.005, 0.02, n).astype(np.float32)
    x = (rng.standard_normal(k) * 2.5).astype(np.float32)
    for out_scale in (0.0, 0.1):
        got, gc = o.qgemv_tile8u(w, s, x, n, k, 0.05, out_scale)
        want, _, wc = o.qgemv(4, w, s, x, n, k, 0.05, out_scale)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert np.array_equal(gc, wc)


@pytest.mark.parametrize("n,k", [(11, 256), (24, 2048)])
def test_uncalibrated_grid_equals_classic(n, k):
    rng = np.random.default_rng(k + 3)
    codes, w = rand_w(rng, n, k)
    s = rng.uniform(0.5, 2.0, n).astype(np.float32)
    x = (rng.integers(-128, 129, k) / 8.0).astype(np.float32)  # 1/8 grid, |x| <= 16
    got, _ = o.qgemv_tile8u(w, s, x, n, k, 0.0, 0.0)
    want, _, _ = o.qgemv(4, w, s, x, n, k, 0.0, 0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    exact = (codes.astype(np.float64) @ x.astype(np.float64)) * s.astype(np.float64)
    assert np.allclose(got, exact, rtol=1e-6, atol=0)


def replay_row(codes_row, x, k):
    """The shader text for one row in numpy float32 scalars (every operation rounded)."""
    f = np.float32
    lanes = []
    for l in range(32):
        acc, sxf = f(0), f(0)
        for i in range(k // 128):
            for j in range(4):
                kk = 128 * i + 4 * l + j
                u = f(int(codes_row[kk]) + 8)
                sxf = f(sxf + x[kk])
                acc = f(acc + f(u * x[kk]))
        lanes.append(f(acc - f(f(8) * sxf)))
    for m in (1, 2, 4, 8, 16):
        lanes = [f(lanes[l] + lanes[l ^ m]) for l in range(32)]
    return lanes[0]


@pytest.mark.parametrize("k", [256, 512])
def test_uncalibrated_random_order(k):
    n = 6
    rng = np.random.default_rng(k)
    codes, w = rand_w(rng, n, k)
    s = rng.uniform(0.5, 2.0, n).astype(np.float32)
    x = (rng.standard_normal(k) * 3.0).astype(np.float32)
    got, _ = o.qgemv_tile8u(w, s, x, n, k, 0.0, 0.0)
    for r in range(n):
        want = np.float32(s[r] * replay_row(codes[r], x, k))
        assert got[r].view(np.uint32) == want.view(np.uint32), r
    # and close to the f64 sum, within f32 accumulation error
    exact = (codes.astype(np.float64) @ x.astype(np.float64)) * s.astype(np.float64)
    mag = (np.abs(codes.astype(np.float64) + 8) @ np.abs(x.astype(np.float64))) * s
    assert np.all(np.abs(got - exact) <= mag * 2.0 ** -18)


def test_uncalibrated_order_differs_from_classic_somewhere():
    """The check above can tell the two orders apart: off the grid, the tile8u order and the
    classic loop's f64 sum disagree in the last bits on some rows."""
    n, k = 64, 1536
    rng = np.random.default_rng(5)
    _, w = rand_w(rng, n, k)
    s = np.ones(n, np.float32)
    x = (rng.standard_normal(k) * 3.0).astype(np.float32)
    got, _ = o.qgemv_tile8u(w, s, x, n, k, 0.0, 0.0)
    want, _, _ = o.qgemv(4, w, s, x, n, k, 0.0, 0.0)
    assert np.any(got.view(np.uint32) != want.view(np.uint32))


def test_k_not_multiple_of_128_refused():
    with pytest.raises(AssertionError):
        o.qgemv_tile8u(np.zeros(64, np.uint8), np.ones(1, np.float32), np.zeros(128, np.float32),
                       1, 100, 0.05, 0.0)
