"""Pins of the oracle's quant.ts restatement (CPU): rounding, SRQ snap, byte layouts, f16 cast.

Every expected value here comes from a library routine (numpy's IEEE f32 divide, rint, float16
cast), brute force over a small domain, or a literal quoted in the reference's own source.
"""
import math

import numpy as np


def test_round_ties_even_matches_rint_on_every_half(oracle):
    # quant.ts:350-357 against numpy's round-half-to-even.
    halves = np.arange(-300.5, 301.0, 1.0, dtype=np.float32)
    for h in halves:
        got = oracle.round_ties_even(float(h))
        want = float(np.rint(h))
        assert got == want and math.copysign(1, got) == math.copysign(1, want), h


def test_round_ties_even_random_and_signed_zero(oracle):
    g = np.random.default_rng(1)
    xs = np.concatenate([g.standard_normal(3000) * 50, g.uniform(-1, 1, 3000)]).astype(np.float32)
    for v in xs:
        got = oracle.round_ties_even(float(v))
        want = float(np.rint(v))
        assert got == want and math.copysign(1, got) == math.copysign(1, want), v
    # Math.round keeps the sign of a negative value that rounds to zero (quant.ts:333 note).
    assert math.copysign(1, oracle.round_ties_even(-0.3)) == -1
    assert math.copysign(1, oracle.round_ties_even(-0.5)) == -1
    assert oracle.round_ties_even(2.5) == 2 and oracle.round_ties_even(-2.5) == -2
    assert oracle.round_ties_even(3.5) == 4 and oracle.round_ties_even(1.5) == 2


def test_srq_code_in_tree_known_answer(oracle):
    # quant.ts:324-329: layer 0 gate_proj position 112 of interview-300. The f32 quotient is
    # exactly -18.5 and ties to even (-18); the f64 quotient -18.500000144645664 would give -19.
    v, s = -11.435039520263672, 0.6181102395057678
    assert float(np.float32(v) / np.float32(s)) == -18.5
    assert np.rint(v / s) == -19  # the f64 route disagrees, so the pin discriminates
    assert oracle.srq_code_f32(v, s) == -18.0
    assert int(oracle.srq_codes(np.array([v], np.float32), s)[0]) == -18


def test_srq_codes_match_numpy_f32_divide_rint_clip(oracle):
    g = np.random.default_rng(2)
    x = (g.standard_normal(200_000) * 4).astype(np.float32)
    x[:1000] = (np.arange(1000, dtype=np.float32) - 500) * np.float32(0.025)  # many exact ties
    for s in (0.05, 0.1875, 0.015625, 0.6181102395057678, 3.334678888320923):
        s32 = np.float32(s)
        want = np.clip(np.rint(x / s32), -128, 127).astype(np.int8)
        got = oracle.srq_codes(x, s)
        assert np.array_equal(got, want), s


def test_srq_clamp_zero_scale_and_apply(oracle):
    s = np.float32(0.1)
    assert oracle.srq_code_f32(1000.0, s) == 127
    assert oracle.srq_code_f32(-1000.0, s) == -128
    assert oracle.srq_code_f32(float("inf"), s) == 127
    assert oracle.srq_code_f32(1.0, 0.0) == 0  # uncalibrated: no codes
    x = np.array([0.26, -0.31, 12.0, -20.0, 0.05, -0.04], np.float32)
    got = oracle.apply_srq(x, s)
    want = (np.clip(np.rint(x / s), -128, 127) * s).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(oracle.apply_srq(x, 0.0), x)  # quant.ts:281-284 pass-through
    # NaN as an int8 code: WGSL clamp = min(max(NaN, -128), 127) = -128 with maxNum semantics.
    assert int(oracle.srq_codes(np.array([np.nan], np.float32), s)[0]) == -128


def test_unpack_int4_brute_force_all_bytes(oracle):
    b = np.arange(256, dtype=np.uint8)
    got = oracle.unpack(4, b, 512)
    want = np.empty(512, np.int8)
    want[0::2] = (b & 0x0F).astype(np.int8) - 8   # low nibble first (quant.ts:11-13)
    want[1::2] = (b >> 4).astype(np.int8) - 8
    assert np.array_equal(got, want)


def test_unpack_int8_brute_force_all_bytes(oracle):
    b = np.arange(256, dtype=np.uint8)
    assert np.array_equal(oracle.unpack(8, b, 256), b.view(np.int8))


def test_pack_unpack_round_trip(oracle):
    g = np.random.default_rng(3)
    for bits, lo, hi in ((4, -8, 8), (8, -128, 128)):
        codes = g.integers(lo, hi, size=4096).astype(np.int8)
        packed = oracle.pack(bits, codes)
        assert packed.size == (codes.size // 2 if bits == 4 else codes.size)
        assert np.array_equal(oracle.unpack(bits, packed, codes.size), codes)
        raw = g.integers(0, 256, size=2048, dtype=np.uint8)
        width = raw.size * (2 if bits == 4 else 1)
        assert np.array_equal(oracle.pack(bits, oracle.unpack(bits, raw, width)), raw)


def test_f32_to_f16_matches_numpy(oracle):
    g = np.random.default_rng(4)
    vals = np.concatenate([
        g.standard_normal(20000).astype(np.float32),
        (g.standard_normal(5000) * 1e-5).astype(np.float32),     # f16 subnormals
        (g.standard_normal(2000) * 1e5).astype(np.float32),      # overflow to inf
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.9604645e-08,
                  2.9802322e-08, 2.9802326e-08, np.inf, -np.inf], np.float32),
        # exact ties between two f16 neighbours
        (np.float32(1.0) + np.float32(2.0 ** -11) * np.arange(1, 40, 2, dtype=np.float32)),
    ])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)
    nan = oracle.f32_to_f16_bits(float("nan"))
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_f16_to_f32_exact_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    sample = bits[::7]
    for h in sample:
        got = oracle.f16_bits_to_f32(int(h))
        w = float(want[int(h)])
        if math.isnan(w):
            assert math.isnan(got)
        else:
            assert got == w and math.copysign(1, got) == math.copysign(1, w)
