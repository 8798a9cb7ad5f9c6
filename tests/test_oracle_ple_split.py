"""Pins of the oracle's ple-gate-split and foldGate restatement (pleSplit.ts:17-41).

- Layout: the gate split's buffer, read the way the fold's WGSL reads it (one vec4 of four rows
  per split, `gate[i * n + s]`, i.e. numpy [N/4][n][4]), is the plain split's [N][n] partials.
- Exactness: the bands of every row sum to the unsplit exact accumulator.
- The fold of the split partials is the unsplit 8-bit GEMV's f32 output bit for bit (the pinned
  qgemv oracle with outScale = gateOutScale), at every split count: a wrong interleave, a dropped
  split, a swapped scale index or a snap before the epilogue fails this.
- Known answers of the f32 fold order and of the gate snap (ties to even, the clamp, the in-tree
  srqCodes(-11.435039520263672, 0.6181102395057678) = -18 of quant.ts:324-329).
"""
import numpy as np
import pytest

import g4synth as syn

F = np.float32


def gate_operands(n=256, k=1536, seed=3):
    w = syn.int8_weights("plesplit", f"w{n}_{k}", n, k)
    s = syn.row_scales("plesplit", f"s{n}_{k}", n)
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(k) * 1.5).astype(F)
    return w, s, x


@pytest.mark.parametrize("splits", [2, 4, 8])
def test_gate_split_layout_is_the_vec4_read(oracle, splits):
    n, k = 256, 1536
    w, s, x = gate_operands(n, k)
    buf = oracle.ple_gate_split(w, s, x, n, k, splits, syn.IN_SCALE)
    plain = oracle.qgemv_split(8, w, s, x, n, k, splits, True, syn.IN_SCALE)
    as_read = buf.reshape(n // 4, splits, 4).transpose(0, 2, 1).reshape(n, splits)
    assert np.array_equal(as_read.view(np.uint32), plain.view(np.uint32))
    _, acc, _ = oracle.qgemv(8, w, s, x, n, k, syn.IN_SCALE, syn.OUT_SCALE)
    assert np.array_equal(plain.astype(np.int64).sum(axis=1), acc.astype(np.int64))
    assert np.all(np.abs(plain) < 2 ** 24)  # every partial exact in f32


@pytest.mark.parametrize("splits", [2, 4, 8])
@pytest.mark.parametrize("gate_out", [0.0, float(syn.OUT_SCALE), 0.125])
def test_fold_of_split_is_the_unsplit_gate(oracle, splits, gate_out):
    n, k = 256, 1536
    w, s, x = gate_operands(n, k, seed=splits)
    buf = oracle.ple_gate_split(w, s, x, n, k, splits, syn.IN_SCALE)
    folded = oracle.ple_fold_gate(buf, n, splits, s, syn.IN_SCALE, gate_out)
    y, _, _ = oracle.qgemv(8, w, s, x, n, k, syn.IN_SCALE, gate_out)
    assert np.array_equal(folded.view(np.uint32), y.view(np.uint32))


def test_fold_sums_in_split_order_in_f32(oracle):
    """Partials [2^24, 1, 1, -2^24]: the ascending f32 sum from 0 loses both ones (2^24 + 1 rounds
    to 2^24), so the fold is 0 where an exact or f64 sum gives 2."""
    k, splits = 4, 4
    parts = np.zeros(k * splits, F)
    for s_, v in enumerate([2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]):
        parts[s_ * 4 + 0] = v   # element 0 of vec4 0 in split s_
    parts[1 * 4 + 1] = 3.0      # element 1: only split 1 carries a value
    out = oracle.ple_fold_gate(parts, k, splits, np.ones(k, F), 1.0, 0.0)
    assert out[0] == 0.0 and out[1] == 3.0 and out[2] == 0.0 and out[3] == 0.0


def test_fold_epilogue_order_and_gate_snap(oracle):
    """v = f32(f32(in * scale) * total), then the snap: ties to even on exact halves, the clamp at
    -128 / 127, and the in-tree known answer -18."""
    k, splits = 16, 2
    totals = np.array([1, 3, 5, 7, -1, -3, 9, 2000, -2000, 0, 11, 13, 15, 17, 19, 21], F)
    parts = np.zeros(k * splits, F)
    for i, t in enumerate(totals):
        parts[(i // 4) * 4 * splits + 1 * 4 + i % 4] = t  # all in split 1
    # in * scale = 1/16: v = t / 16 exactly; at gate_out 0.125 the quotient is t / 2 (halves)
    out = oracle.ple_fold_gate(parts, k, splits, np.full(k, 0.5, F), 0.125, 0.125)
    want = np.clip(np.rint(totals / 2.0), -128, 127) * 0.125  # rint is ties to even
    assert np.array_equal(out, want.astype(F))
    assert out[0] == 0.0 and out[1] == 0.25 and out[2] == 0.25 and out[3] == 0.5
    assert out[7] == F(127 * 0.125) and out[8] == F(-128 * 0.125)
    # the known answer at the gate snap
    ka = np.zeros(4 * splits, F)
    ka[0] = F(-11.435039520263672)
    got = oracle.ple_fold_gate(ka, 4, splits, np.ones(4, F), 1.0, F(0.6181102395057678))
    assert got[0] == F(-18) * F(0.6181102395057678)
    # a dropped input-scale multiply or the product taken in the other order is visible: in * scale
    # rounds before it meets the total
    a, b, t = F(0.1), F(0.3), F(3.0)
    parts2 = np.zeros(4 * splits, F)
    parts2[0] = t
    got2 = oracle.ple_fold_gate(parts2, 4, splits, np.full(4, b, F), float(a), 0.0)
    assert got2[0] == (a * b) * t
