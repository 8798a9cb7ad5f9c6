"""Independent numpy routes used to pin the oracle (test helpers, not a restatement of it).

The codes come from numpy bit operations on the stored bytes, the contraction from numpy's integer
or float64 matmul, the rounding from numpy's IEEE f32 divide and rint. A mistake in the oracle's
nibble order, zero point, operand orientation, epilogue order or rounding rule shows up as a
mismatch against these.
"""
import numpy as np


def codes_int4(packed: np.ndarray) -> np.ndarray:
    """[rows, k/2] bytes -> [rows, k] int codes, low nibble first, zero point 8."""
    packed = np.asarray(packed, np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), np.int64)
    out[..., 0::2] = (packed & 0x0F).astype(np.int64) - 8
    out[..., 1::2] = (packed >> 4).astype(np.int64) - 8
    return out


def codes_int8(packed: np.ndarray) -> np.ndarray:
    return np.asarray(packed, np.uint8).view(np.int8).astype(np.int64)


def codes(bits: int, packed: np.ndarray) -> np.ndarray:
    return codes_int4(packed) if bits == 4 else codes_int8(packed)


def snap(x: np.ndarray, s: float) -> np.ndarray:
    x = np.asarray(x, np.float32)
    return np.clip(np.rint(x / np.float32(s)), -128, 127)


def linear(bits, packed, scales, x, in_scale, out_scale):
    """Returns (acc int64 [m, n], y f32 [m, n], q int8 [m, n] or None, dst f32 [m, n])."""
    w = codes(bits, packed)                      # [n, k]
    x = np.atleast_2d(np.asarray(x, np.float32))  # [m, k]
    scales = np.asarray(scales, np.float32)
    if in_scale != 0:
        xq = snap(x, in_scale).astype(np.int64)
        acc = xq @ w.T                            # exact integers
        xs_s = (np.float32(in_scale) * scales).astype(np.float32)
        y = (xs_s[None, :] * acc.astype(np.float32)).astype(np.float32)
    else:
        acc = None
        total = x.astype(np.float64) @ w.T.astype(np.float64)
        y = (scales[None, :] * total.astype(np.float32)).astype(np.float32)
    if out_scale != 0:
        q = snap(y, out_scale)
        dst = (q * np.float32(out_scale)).astype(np.float32)
        return acc, y, q.astype(np.int8), dst
    return acc, y, None, y
