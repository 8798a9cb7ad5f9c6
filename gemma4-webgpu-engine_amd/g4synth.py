"""Seeded synthetic inputs for the BASELINE configurations (no checkpoint exists offline).

Every tensor draws from its own numpy PCG64 stream seeded by (config, tensor name), so a tensor is
the same bytes whichever order a test or the bench asks for it in.

  int4 weights   codes uniform over [-8, 7], stored as code + 8, two per byte, low nibble first
                 (src/quant.ts:11-20): uniform random bytes are exactly that.
  int8 weights   codes uniform over [-127, 127], stored as the signed byte.
  row scales     f32 uniform in [0.005, 0.02).
  activations    f16 N(0, 1) (numpy draws f64, rounded to f16 ties-to-even).
  outliers       config 2: exactly 1% of entries (seeded positions) set to +-8.0 (8 sigma), which
                 saturate after the 0.05 snap (8 / 0.05 = 160 > 127).
  PLE            int4 codes uniform; one f16 scale per (row, 256-wide group) uniform in
                 [0.005, 0.02); ids Zipf(s = 1.1) over the vocabulary by inverse CDF.
"""
from __future__ import annotations

import hashlib

import numpy as np

IN_SCALE = float(np.float32(0.05))    # fround(0.05), the config-0 static input scale
OUT_SCALE = float(np.float32(0.1))    # fround(0.1), the config-0 static output scale

HIDDEN, FFN, HEAD_DIM, Q_HEADS, KV_HEADS = 1536, 6144, 256, 8, 1
# Config 1: one layer's decode projection set (name, N, K).
LAYER_PROJECTIONS = [
    ("q", Q_HEADS * HEAD_DIM, HIDDEN),
    ("k", KV_HEADS * HEAD_DIM, HIDDEN),
    ("v", KV_HEADS * HEAD_DIM, HIDDEN),
    ("o", HIDDEN, Q_HEADS * HEAD_DIM),
    ("gate", FFN, HIDDEN),
    ("up", FFN, HIDDEN),
    ("down", HIDDEN, FFN),
]
PLE_ROWS, PLE_LAYERS, PLE_GROUP = 262144, 35, 256
PLE_COLS = PLE_LAYERS * PLE_GROUP


def rng(config: str, tensor: str) -> np.random.Generator:
    h = hashlib.sha256(f"g4w8a8/{config}/{tensor}".encode()).digest()
    return np.random.Generator(np.random.PCG64(int.from_bytes(h[:8], "little")))


def int4_weights(config: str, name: str, n: int, k: int) -> np.ndarray:
    """[n, k/2] packed bytes."""
    return rng(config, name + ".w").integers(0, 256, size=(n, k // 2), dtype=np.uint8)


def int8_weights(config: str, name: str, n: int, k: int) -> np.ndarray:
    """[n, k] signed bytes viewed as uint8."""
    codes = rng(config, name + ".w").integers(-127, 128, size=(n, k), dtype=np.int16)
    return codes.astype(np.int8).view(np.uint8)


def weights(config: str, name: str, n: int, k: int, bits: int) -> np.ndarray:
    return int4_weights(config, name, n, k) if bits == 4 else int8_weights(config, name, n, k)


def row_scales(config: str, name: str, n: int) -> np.ndarray:
    return rng(config, name + ".s").uniform(0.005, 0.02, size=n).astype(np.float32)


def activations(config: str, name: str, m: int, k: int, outlier_frac: float = 0.0) -> np.ndarray:
    """[m, k] f16 N(0,1), with an exact count of +-8 outliers when outlier_frac > 0."""
    g = rng(config, name + ".x")
    x = g.standard_normal(size=(m, k)).astype(np.float16)
    if outlier_frac > 0:
        count = int(round(outlier_frac * m * k))
        pos = g.choice(m * k, size=count, replace=False)
        sign = np.where(g.integers(0, 2, size=count) == 0, -1.0, 1.0)
        flat = x.reshape(-1)
        flat[pos] = (8.0 * sign).astype(np.float16)
    return x


def ple_codes(config: str, rows: int, cols: int = PLE_COLS) -> np.ndarray:
    """[rows, cols/2] packed int4 table."""
    return rng(config, "ple.codes").integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)


def ple_scales(config: str, rows: int, groups: int = PLE_LAYERS) -> np.ndarray:
    return rng(config, "ple.scales").uniform(0.005, 0.02, size=(rows, groups)).astype(np.float16)


def zipf_ids(config: str, tokens: int, vocab: int = PLE_ROWS, s: float = 1.1) -> np.ndarray:
    """Token ids ~ Zipf(s) over [0, vocab) by inverse CDF on seeded uniforms."""
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    u = rng(config, f"ids.{tokens}").random(tokens)
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.int32)
