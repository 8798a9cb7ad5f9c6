"""Adversarial inputs for every SRQ snap site (quant.ts:309-334 srqCodes).

The kernels snap with a reciprocal fast path, rint(v * fl(1/s)), and fall back to the IEEE divide
rint(fl(v / s)) near a half integer. The two differ on inputs whose quotient sits within an ulp of
a half integer; these helpers plant such inputs so a GPU test fails if a site skips the fallback:

  activation snaps   values planted in x at s = fround(0.05): 1.175, -3.6250002, -7.1250005 (and
                     their negatives), whose f32 quotients 23.499998, -72.5, -142.5 round one way
                     and whose reciprocal products 23.5, -72.50001, -142.50002 the other.
  output snaps       row scales tuned so y = f32(f32(inScale * scale) * acc) lands exactly on
                     +-5.95 or +-6.5499997 at s = fround(0.1) (59.499996 vs 59.5, 65.49999 vs 65.5).
  known answer       srqCodes(-11.435039520263672, 0.6181102395057678) = -18 (quant.ts:324-329):
                     the f32 quotient is exactly -18.5 and ties to even; an f64 divide gives -19.
Test helpers only; nothing in the product imports this.
"""
from __future__ import annotations

import numpy as np

F = np.float32
S_IN, S_OUT = F(0.05), F(0.1)
ADV_IN = [F(1.175), F(-3.6250002), F(-7.1250005)]
ADV_OUT = [F(5.95), F(6.5499997)]
KA_SCALE, KA_VALUE = F(0.6181102395057678), F(-11.435039520263672)


def divide_code(v, s):
    return np.clip(np.rint(np.asarray(v, F) / F(s)), -128, 127)


def recip_code(v, s):
    return np.clip(np.rint(np.asarray(v, F) * (F(1) / F(s))), -128, 127)


def plant(x: np.ndarray, values, every: int = 5, offset: int = 0) -> np.ndarray:
    """x (f32, [m, k]) with `values` and their negatives cycled into every `every`-th element."""
    x = np.array(x, dtype=F, copy=True)
    flat = x.reshape(-1)
    vals = np.array([v for v in values] + [-v for v in values], F)
    idx = np.arange(offset, flat.size, every)
    flat[idx] = vals[np.arange(idx.size) % vals.size]
    return x


def solve_factor(a: np.ndarray, targets: np.ndarray, span: int = 256) -> np.ndarray:
    """For each a[i] (f32) an f32 b with fl(a[i] * b) == targets[i], or NaN where the f32
    neighbourhood of targets / a holds none."""
    a = np.asarray(a, F)
    t = np.asarray(targets, F)
    b0 = (t.astype(np.float64) / a.astype(np.float64)).astype(F)
    steps = np.arange(-span, span + 1, dtype=np.int64)
    bits = b0.view(np.int32).astype(np.int64)[:, None] + np.where(b0[:, None] < 0, -steps, steps)
    cand = bits.astype(np.int32).view(F)
    hit = (a[:, None] * cand) == t[:, None]
    out = np.full(a.shape, np.nan, F)
    any_hit = hit.any(axis=1)
    first = hit.argmax(axis=1)
    out[any_hit] = cand[any_hit, first[any_hit]]
    return out


def tune_row_scales(acc: np.ndarray, scales: np.ndarray, in_scale, targets) -> tuple:
    """Row scales (f32 [n]) such that y[m_n, n] = f32(f32(in_scale * scale[n]) * acc[m_n, n]) equals
    one of `targets` (signed to match acc) for column m_n = n % M. acc: [M, n] exact int32 sums
    (independent of the scales). Returns (scales, mask of the rows that were tuned)."""
    acc = np.atleast_2d(acc)
    m, n = acc.shape
    cols = np.arange(n) % m
    a = acc[cols, np.arange(n)].astype(F)
    tv = np.abs(np.array(targets, F))[np.arange(n) % len(targets)]
    tv = np.where(a < 0, -tv, tv)
    ok = a != 0
    # c = f32(in_scale * scale) must satisfy fl(c * a) == t; then scale with fl(in_scale * scale) == c
    c = np.full(n, np.nan, F)
    c[ok] = solve_factor(a[ok], tv[ok])
    s = np.full(n, np.nan, F)
    good = ~np.isnan(c)
    s[good] = solve_factor(np.full(good.sum(), F(in_scale)), c[good])
    tuned = ~np.isnan(s) & (s > 0)
    out = np.array(scales, F, copy=True)
    out[tuned] = s[tuned]
    return out, tuned
