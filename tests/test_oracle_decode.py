"""Pins of the decode-step glue oracle (oracle/g4_decode_oracle.c) before the GPU is held to it.

The reference checks each of these WGSL kernels against an f64 CPU oracle within a tolerance it
argues for in the kernel file; the same fixtures and tolerances pin the f32 restatement here:
  rmsNorm.ts:341-350 (8 ULP, exact-sum fixture on the 1/2 grid up to 4),
  mlpEpilogue.ts:305-318 (8 ULP or 4e-6 absolute), blockJoin.ts:229-238 (8 ULP or 4e-6),
  rope.ts:351-361 (1e-6 absolute, inputs under 8), attnPrologue.ts:451-459 (1e-5 absolute),
  attention.ts:1005-1028 (1e-4 absolute and cosine 0.999),
  geluMul.ts:280-291 (2e-5 absolute, gate up to 8 and up to 4), logitSoftcap.ts:189-197 (1e-4),
  argmax.ts:262-277 (first strict maximum, NaN never wins).
The f64 forms below are the textbook formulas those oracles state, not the f32 chain under test.
"""
import math

import numpy as np
import pytest

import decode_oracle as d

EPS = 1e-6


def ulps(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    spacing = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    return np.abs(got - want) / spacing


def within(got, want, tol_ulp, tol_abs):
    """The reference harness's OR of an ULP gate and an absolute gate, per element."""
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    return bool(np.all((ulps(got, want) <= tol_ulp) | (err <= tol_abs)))


def half_grid(rng, shape, top=4.0):
    """The reference norm fixtures: multiples of 1/2 with magnitude at most `top`."""
    return (rng.integers(-int(2 * top), int(2 * top) + 1, size=shape) / 2.0).astype(np.float32)


def rms_f64(x, gain, eps=EPS):
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * inv
    return y if gain is None else y * np.asarray(gain, np.float64)


def gelu_tanh_f64(x):
    x = np.asarray(x, np.float64)
    inner = math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)
    return 0.5 * x * (1.0 + np.tanh(inner))


def gelu_erf_f64(x):
    return np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in np.asarray(x, np.float64)])


def srq_f64(v, s):
    # quant.ts srqCodes: clamp(round-half-even(v / s)); np.rint is half-even.
    return np.clip(np.rint(np.asarray(v, np.float64) / s), -128, 127).astype(np.int8)


def near_half(v, s, margin):
    q = np.asarray(v, np.float64) / s
    return np.abs(q - np.floor(q) - 0.5) < margin


# ---- the math functions -------------------------------------------------------------------------

def test_expf_against_libm():
    rng = np.random.default_rng(1)
    xs = np.concatenate([np.linspace(-87.0, 88.5, 40001), rng.uniform(-30, 30, 20000),
                         rng.uniform(-1, 1, 5000)]).astype(np.float32)
    got = np.array([d.expf(x) for x in xs], np.float64)
    worst = ulps(got, np.exp(xs.astype(np.float64))).max()
    print(f"g4d_expf: max error {worst:.2f} ulp over {xs.size} points")
    assert worst <= 3.0
    assert d.expf(0.0) == 1.0
    assert d.expf(-87.5) == 0.0 and d.expf(-1e30) == 0.0
    assert math.isinf(d.expf(89.0)) and math.isnan(d.expf(float("nan")))
    # softmax weights are exp(s - max) <= 1: monotone on a fine grid of non-positive arguments
    xs = np.linspace(-20, 0, 20001).astype(np.float32)
    ys = np.array([d.expf(x) for x in xs])
    assert np.all(np.diff(ys) >= 0)


def test_tanhf_against_libm():
    xs = np.concatenate([np.linspace(-12, 12, 48001), np.geomspace(1e-6, 2.0, 20001)]).astype(np.float32)
    got = np.array([d.tanhf(x) for x in xs], np.float64)
    want = np.tanh(xs.astype(np.float64))
    worst = ulps(got, want).max()
    print(f"g4d_tanhf: max error {worst:.2f} ulp, {np.abs(got - want).max():.3g} absolute")
    assert worst <= 8.0
    assert np.abs(got - want).max() <= 2.0 ** -22
    for x in (0.3, 1e-3, 5.0, 0.171875, 1e-5):
        assert d.tanhf(-x) == -d.tanhf(x)
    assert d.tanhf(10.0) == 1.0 and d.tanhf(0.0) == 0.0


def test_gelu_tanh_form_within_reference_tolerance():
    # geluMul.ts:280-291: gate up to 8, up up to 4, 2e-5 absolute on the product; the tolerance is
    # twenty times below the gap to the erf form, which must fail it.
    rng = np.random.default_rng(2)
    gate = rng.uniform(-8, 8, 20000).astype(np.float32)
    up = rng.uniform(-4, 4, 20000).astype(np.float32)
    got = np.array([np.float32(d.gelu_tanh(g)) * u for g, u in zip(gate, up)], np.float32)
    want = gelu_tanh_f64(gate) * up.astype(np.float64)
    err = np.abs(got - want).max()
    print(f"gelu*up: max abs error {err:.3g}")
    assert err <= 2e-5
    assert np.abs(gelu_erf_f64(gate) * up - want).max() > 20 * 2e-5
    assert d.gelu_tanh(0.0) == 0.0
    assert d.gelu_tanh(30.0) == 30.0  # clamp at 10: tanh = 1 exactly


# ---- reductions and norms -----------------------------------------------------------------------

def test_sums_exact_on_the_half_grid_and_fixed_order():
    rng = np.random.default_rng(3)
    x = half_grid(rng, 1536)
    assert d.sumsq(x) == float(np.sum(x.astype(np.float64) ** 2))
    ints = rng.integers(-1000, 1000, 5000).astype(np.float32)
    assert d.fsum(ints) == float(ints.sum(dtype=np.int64))
    assert d.fsum(np.zeros(0, np.float32)) == 0.0
    # Outside the exact grid the order is the contract the device follows: 256 lane-strided
    # partials, then the pairwise tree. Stated here with numpy's f32 adds to catch a transposed
    # lane order (strided vs blocked) in the C restatement.
    y = rng.standard_normal(3000).astype(np.float32) * np.float32(1000.0)
    part = np.zeros(256, np.float32)
    for i in range(y.size):
        part[i % 256] = np.float32(part[i % 256] + y[i])
    s = 128
    while s >= 1:
        part[:s] = part[:s] + part[s:2 * s]
        s //= 2
    assert d.fsum(y) == float(part[0])


@pytest.mark.parametrize("width,weighted", [(1536, True), (1536, False), (256, True), (256, False)])
def test_rms_norm_within_8_ulp(width, weighted):
    rng = np.random.default_rng(width + weighted)
    x = half_grid(rng, (6, width))
    gain = rng.uniform(-4, 4, width).astype(np.float32) if weighted else None
    got = d.rms_norm(x, gain, EPS)
    assert within(got, rms_f64(x, gain), 8, 0.0)
    codes = d.rms_norm_codes(x, gain, EPS, 0.05)
    want = srq_f64(rms_f64(x, gain), 0.05)
    ok = (codes == want) | near_half(rms_f64(x, gain), 0.05, 1e-4)
    assert ok.all()


def test_norm_residual_within_reference_gate():
    rng = np.random.default_rng(5)
    src = half_grid(rng, (4, 1536))
    resid = half_grid(rng, (4, 1536))
    gain = half_grid(rng, 1536)
    got = d.norm_residual(src, gain, resid, EPS)
    want = resid.astype(np.float64) + rms_f64(src, gain)
    assert within(got, want, 8, 4e-6)
    # a missing residual or a (1 + w) gain moves the answer by order 1
    assert np.abs(got - rms_f64(src, gain)).max() > 1.0


@pytest.mark.parametrize("alpha", [1.0, 0.5, 0.8125])
def test_norm_residual_norm_join(alpha):
    # blockJoin.ts:229-238's fixture: src +-1 with eps 0 (inv exactly 1), residual on the 1/4 grid
    # under 4, gain on the 1/8 grid under 2.
    rng = np.random.default_rng(6)
    width = 1536
    src = rng.choice([-1.0, 1.0], size=(3, width)).astype(np.float32)
    resid = (rng.integers(-15, 16, (3, width)) / 4.0).astype(np.float32)
    gain = (rng.integers(-15, 16, width) / 8.0).astype(np.float32)
    gain2 = rng.uniform(-2, 2, width).astype(np.float32)
    hidden, codes = d.norm_residual_norm(src, gain, resid, gain2, alpha, 0.0, 0.05)
    want_h = (resid.astype(np.float64) + src * gain.astype(np.float64)) * alpha
    if alpha in (1.0, 0.5):
        assert np.array_equal(hidden, want_h.astype(np.float32))  # exact on the grid
    else:
        assert within(hidden, want_h, 8, 4e-6)
    normed = rms_f64(hidden, gain2, eps=0.0)
    ok = (codes == srq_f64(normed, 0.05)) | near_half(normed, 0.05, 1e-4)
    assert ok.all()


# ---- rope and the attention prologue ------------------------------------------------------------

def rope_tables(positions, head_dim=256, theta=10000.0, partial=1.0):
    """cos/sin rows in the split-half convention (rope.ts:240-258) at f64, rounded to f32."""
    p = head_dim // 2
    rot = int(p * partial)
    inv = np.zeros(p)
    inv[:rot] = 1.0 / theta ** (np.arange(rot) * 2.0 / head_dim)
    ang = np.outer(np.asarray(positions, np.float64), inv)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_f64(x, c, s):
    x = np.asarray(x, np.float64)
    p = x.size // 2
    lo, hi = x[:p], x[p:]
    c, s = c.astype(np.float64), s.astype(np.float64)
    return np.concatenate([lo * c - hi * s, hi * c + lo * s])


def test_rope_row_within_1e6_and_inverse():
    rng = np.random.default_rng(7)
    cos, sin = rope_tables([0, 1, 37, 4095])
    for r in range(4):
        x = rng.uniform(-8, 8, 256).astype(np.float32)
        got = d.rope_row(x, cos[r], sin[r])
        assert np.abs(got - rope_f64(x, cos[r], sin[r])).max() <= 1e-6
        back = rope_f64(got, cos[r], -sin[r])
        assert np.abs(back - x).max() <= 4e-6
    x = rng.uniform(-8, 8, 256).astype(np.float32)
    assert np.array_equal(d.rope_row(x, cos[0], sin[0]), x)  # position 0 is the identity


def test_q_and_kv_prologue_within_1e5():
    rng = np.random.default_rng(8)
    heads, hd = 8, 256
    cos, sin = rope_tables([123], partial=0.25)
    qs, ks, vs = 0.03125, 0.0625, 0.046875
    q_codes = rng.integers(-128, 128, (heads, hd)).astype(np.int8)
    k_codes = rng.integers(-128, 128, hd).astype(np.int8)
    v_codes = rng.integers(-128, 128, hd).astype(np.int8)
    qg = rng.uniform(-4, 4, hd).astype(np.float32)
    kg = rng.uniform(-4, 4, hd).astype(np.float32)
    got = d.q_norm_rope(q_codes, qs, qg, cos[0], sin[0], EPS)
    for h in range(heads):
        want = rope_f64(rms_f64(q_codes[h] * np.float32(qs), qg), cos[0], sin[0])
        assert np.abs(got[h] - want).max() <= 1e-5
    k_row, v_row = d.kv_norm_rope(k_codes, ks, v_codes, vs, kg, cos[0], sin[0], EPS)
    assert np.abs(k_row - rope_f64(rms_f64(k_codes * np.float32(ks), kg), cos[0], sin[0])).max() <= 1e-5
    assert within(v_row, rms_f64(v_codes * np.float32(vs), None), 8, 0.0)


# ---- attention decode ---------------------------------------------------------------------------

def attention_f64(q, k, v, p, window):
    lo = max(0, p - window + 1) if window > 0 else 0
    kk = k[lo:p + 1].astype(np.float64)
    vv = v[lo:p + 1].astype(np.float64)
    s = q.astype(np.float64) @ kk.T
    w = np.exp(s - s.max(axis=1, keepdims=True))
    return (w @ vv) / w.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("p,window", [(0, 0), (1, 0), (255, 0), (256, 0), (700, 0), (1023, 512),
                                      (600, 512), (511, 512)])
def test_attention_decode_within_reference_gates(p, window):
    rng = np.random.default_rng(p * 7 + window)
    heads, hd = 8, 256
    # normed q and k rows (unit rms, like the prologue's output) give scores of order 10
    q = rng.standard_normal((heads, hd)).astype(np.float32) * np.float32(0.2)
    k = rng.standard_normal((p + 1, hd)).astype(np.float32)
    v = rng.standard_normal((p + 1, hd)).astype(np.float32)
    got = d.attention_decode(q, k, v, p, window)
    want = attention_f64(q, k, v, p, window)
    cos = (got * want).sum(axis=1) / np.linalg.norm(got, axis=1) / np.linalg.norm(want, axis=1)
    assert np.abs(got - want).max() <= 1e-4
    assert cos.min() >= 0.999
    if window > 0 and p >= window:
        # positions before the window do not matter
        k2, v2 = k.copy(), v.copy()
        k2[:p - window + 1] = 9.0
        v2[:p - window + 1] = -9.0
        assert np.array_equal(d.attention_decode(q, k2, v2, p, window), got)


def test_attention_single_position_is_v():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((8, 256)).astype(np.float32)
    k = rng.standard_normal((1, 256)).astype(np.float32)
    v = rng.standard_normal((1, 256)).astype(np.float32)
    got = d.attention_decode(q, k, v, 0, 0)
    assert np.array_equal(got, np.broadcast_to(v, got.shape))


# ---- gelu-mul, embedding, per-layer inputs, softcap, argmax -----------------------------------

@pytest.mark.parametrize("ple", [False, True])
def test_gelu_mul_codes_match_f64_srq(ple):
    rng = np.random.default_rng(10 + ple)
    n = 6144
    gs, us, in_scale = 0.0625, 0.03125, 0.05
    g = rng.integers(-128, 128, n).astype(np.int8)
    u = rng.integers(-128, 128, n).astype(np.int8)
    up = rng.uniform(-4, 4, n).astype(np.float32) if ple else None
    codes = d.gelu_mul_codes(g, gs, None if ple else u, us, in_scale, up_f32=up)
    upv = up.astype(np.float64) if ple else u * np.float64(np.float32(us))
    val = gelu_tanh_f64(g * np.float64(np.float32(gs))) * upv
    want = srq_f64(val, np.float32(in_scale))
    # the f32 chain is within 2e-5 of the f64 value, so codes differ only where the quotient lies
    # within 2e-5 / in_scale of a half integer
    ok = (codes == want) | near_half(val, np.float32(in_scale), 2e-5 / in_scale)
    assert ok.all()
    assert np.abs(codes.astype(int) - want.astype(int)).max() <= 1


def test_embed_row_equals_pinned_gather(oracle):
    # embedGather.ts:93-113 folds the embed scale into the row scale once: the f32 product
    # scale * f32(sqrt(1536)), then (code - 8) * that; the pinned f32 gather with that scale.
    rng = np.random.default_rng(11)
    cols = 1536
    table = rng.integers(0, 256, (5, cols // 2)).astype(np.uint8)
    scales = rng.uniform(0.001, 0.05, 5).astype(np.float32)
    es = np.float32(math.sqrt(1536.0))
    assert es == np.float32(float.fromhex("0x1.3988e2p+5"))
    folded = (scales * es).astype(np.float32)
    # the gather oracle applies the PLE output scale 16 (a power of two, so 16 * (folded / 16)
    # is folded exactly)
    want = oracle.embed_gather(table, folded / np.float32(16.0), np.arange(5, dtype=np.int32), cols,
                               cols, out_kind="f32")
    for r in range(5):
        assert np.array_equal(d.embed_row(table[r], scales[r], cols, es), want[r])


def test_ple_combine_within_8_ulp():
    # plan.ts:670-690: rms_norm(proj * alpha) per 256 group, plus the gathered identity, times 2^-0.5
    rng = np.random.default_rng(12)
    groups, group = 35, 256
    codes = rng.integers(-128, 128, groups * group).astype(np.int8)
    gain = rng.uniform(-2, 2, group).astype(np.float32)
    ident = rng.uniform(-3, 3, groups * group).astype(np.float32)
    alpha = np.float32(1536 ** -0.5)
    got = d.ple_combine(codes, 0.0625, alpha, gain, ident, group, EPS)
    proj = (codes * np.float64(np.float32(0.0625)) * alpha).reshape(groups, group)
    want = (rms_f64(proj, gain).reshape(-1) + ident) * 2.0 ** -0.5
    assert within(got, want, 8, 4e-6)


def test_softcap_within_1e4_and_copy():
    rng = np.random.default_rng(13)
    x = rng.uniform(-64, 64, 50000).astype(np.float32)
    got = d.softcap(x, 30.0)
    assert np.abs(got - np.tanh(x.astype(np.float64) / 30.0) * 30.0).max() <= 1e-4
    assert np.array_equal(d.softcap(x, 0.0), x)


def test_argmax_first_strict_maximum():
    x = np.array([1.0, 3.0, np.nan, 3.0, -np.inf, 2.0], np.float32)
    assert d.argmax(x) == 1
    assert d.argmax(np.array([np.nan, 5.0, 5.0], np.float32)) == 1
    assert d.argmax(np.array([-np.inf, -np.inf], np.float32)) == -1
    assert d.argmax(np.array([np.nan, np.nan], np.float32)) == -1
    rng = np.random.default_rng(14)
    for _ in range(20):
        v = rng.integers(-50, 50, 5000).astype(np.float32)  # many ties
        assert d.argmax(v) == int(np.argmax(v))
