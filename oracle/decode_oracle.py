"""numpy front end of the decode-step glue oracle (oracle/g4_decode_oracle.c).

TEST INFRASTRUCTURE ONLY, like oracle.py: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import it, as the checker. Each wrapper names the reference kernel it restates;
the C file and its header carry the exact arithmetic.
"""
from __future__ import annotations

import ctypes

import numpy as np

import oracle as _o

_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64 = ctypes.c_int64
_f = ctypes.c_float

THREADS = 256
ATTN_CHUNK = 32

_ready = False


def lib():
    global _ready
    L = _o.lib()
    if not _ready:
        sig = {
            "g4d_expf": (_f, [_f]),
            "g4d_tanhf": (_f, [_f]),
            "g4d_gelu_tanh": (_f, [_f]),
            "g4d_sumsq": (_f, [_f32p, _i64]),
            "g4d_sum": (_f, [_f32p, _i64]),
            "g4d_rms_norm": (None, [_f32p, _f32p, _i64, _i64, _f, _f32p]),
            "g4d_norm_residual": (None, [_f32p, _f32p, _f32p, _i64, _i64, _f, _f32p]),
            "g4d_norm_residual_norm": (None, [_f32p, _f32p, _f32p, _f32p, _f, _i64, _i64, _f, _f,
                                              _f32p, _i8p]),
            "g4d_rms_norm_codes": (None, [_f32p, _f32p, _i64, _i64, _f, _f, _i8p]),
            "g4d_rope_row": (None, [_f32p, _f32p, _f32p, _i64, _f32p]),
            "g4d_q_norm_rope": (None, [_i8p, _f, _f32p, _f32p, _f32p, _i64, _i64, _f, _f32p]),
            "g4d_kv_norm_rope": (None, [_i8p, _f, _i8p, _f, _f32p, _f32p, _f32p, _i64, _f, _f32p,
                                        _f32p]),
            "g4d_attention_decode": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _f32p]),
            "g4d_gelu_mul_codes": (None, [_i8p, _f, _i8p, _f, _f32p, _i64, _f, _i8p]),
            "g4d_gelu_mul_f32_codes": (None, [_f32p, _f32p, _i64, _f, _i8p]),
            "g4d_embed_row": (None, [_u8p, _f, _i64, _f, _f32p]),
            "g4d_ple_combine": (None, [_i8p, _f, _f, _f32p, _f32p, _i64, _i64, _f, _f32p]),
            "g4d_softcap": (None, [_f32p, _i64, _f, _f32p]),
            "g4d_argmax": (_i64, [_f32p, _i64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _ready = True
    return L


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a, t):
    return None if a is None else a.ctypes.data_as(t)


def f32(v) -> float:
    return float(np.float32(v))


def expf(x: float) -> float:
    return lib().g4d_expf(f32(x))


def tanhf(x: float) -> float:
    return lib().g4d_tanhf(f32(x))


# geluMul.ts:101-116
def gelu_tanh(x: float) -> float:
    return lib().g4d_gelu_tanh(f32(x))


def sumsq(x) -> float:
    x = _f32(x)
    return lib().g4d_sumsq(_p(x, _f32p), x.size)


def fsum(x) -> float:
    x = _f32(x)
    return lib().g4d_sum(_p(x, _f32p), x.size)


# rmsNorm.ts:131-180
def rms_norm(x, gain, eps: float) -> np.ndarray:
    x = _f32(x)
    rows, width = x.shape
    g = None if gain is None else _f32(gain)
    out = np.empty_like(x)
    lib().g4d_rms_norm(_p(x, _f32p), _p(g, _f32p), rows, width, f32(eps), _p(out, _f32p))
    return out


# mlpEpilogue.ts:196-230
def norm_residual(src, gain, resid, eps: float) -> np.ndarray:
    src, gain, resid = _f32(src), _f32(gain), _f32(resid)
    rows, width = src.shape
    out = np.empty_like(src)
    lib().g4d_norm_residual(_p(src, _f32p), _p(gain, _f32p), _p(resid, _f32p), rows, width,
                            f32(eps), _p(out, _f32p))
    return out


# blockJoin.ts:160-175
def norm_residual_norm(src, gain, resid, gain2, alpha: float, eps: float, in_scale: float):
    src, gain, resid, gain2 = _f32(src), _f32(gain), _f32(resid), _f32(gain2)
    rows, width = src.shape
    hidden = np.empty_like(src)
    codes = np.empty(src.shape, dtype=np.int8)
    lib().g4d_norm_residual_norm(_p(src, _f32p), _p(gain, _f32p), _p(resid, _f32p),
                                 _p(gain2, _f32p), f32(alpha), rows, width, f32(eps),
                                 f32(in_scale), _p(hidden, _f32p), _p(codes, _i8p))
    return hidden, codes


def rms_norm_codes(x, gain, eps: float, in_scale: float) -> np.ndarray:
    x = _f32(x)
    rows, width = x.shape
    g = None if gain is None else _f32(gain)
    codes = np.empty(x.shape, dtype=np.int8)
    lib().g4d_rms_norm_codes(_p(x, _f32p), _p(g, _f32p), rows, width, f32(eps), f32(in_scale),
                             _p(codes, _i8p))
    return codes


# rope.ts:275-303
def rope_row(x, cos_row, sin_row) -> np.ndarray:
    x, c, s = _f32(x), _f32(cos_row), _f32(sin_row)
    out = np.empty_like(x)
    lib().g4d_rope_row(_p(x, _f32p), _p(c, _f32p), _p(s, _f32p), x.size, _p(out, _f32p))
    return out


# attnPrologue.ts:268-280
def q_norm_rope(q_codes, q_scale, gain, cos_row, sin_row, eps) -> np.ndarray:
    q_codes = np.ascontiguousarray(q_codes, dtype=np.int8)
    heads, head_dim = q_codes.shape
    gain, c, s = _f32(gain), _f32(cos_row), _f32(sin_row)
    out = np.empty((heads, head_dim), dtype=np.float32)
    lib().g4d_q_norm_rope(_p(q_codes, _i8p), f32(q_scale), _p(gain, _f32p), _p(c, _f32p),
                          _p(s, _f32p), heads, head_dim, f32(eps), _p(out, _f32p))
    return out


# attnPrologue.ts:316-329
def kv_norm_rope(k_codes, k_scale, v_codes, v_scale, gain, cos_row, sin_row, eps):
    k_codes = np.ascontiguousarray(k_codes, dtype=np.int8)
    v_codes = np.ascontiguousarray(v_codes, dtype=np.int8)
    gain, c, s = _f32(gain), _f32(cos_row), _f32(sin_row)
    hd = k_codes.size
    k_row = np.empty(hd, dtype=np.float32)
    v_row = np.empty(hd, dtype=np.float32)
    lib().g4d_kv_norm_rope(_p(k_codes, _i8p), f32(k_scale), _p(v_codes, _i8p), f32(v_scale),
                           _p(gain, _f32p), _p(c, _f32p), _p(s, _f32p), hd, f32(eps),
                           _p(k_row, _f32p), _p(v_row, _f32p))
    return k_row, v_row


# attention.ts:858-918 (split form)
def attention_decode(q, k, v, p: int, window: int) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    heads, hd = q.shape
    assert k.shape[1] == hd and k.shape[0] > p and v.shape == k.shape
    out = np.empty_like(q)
    lib().g4d_attention_decode(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), heads, hd, p, window,
                               _p(out, _f32p))
    return out


# geluMul.ts:219-233
def gelu_mul_codes(g_codes, g_scale, u_codes, u_scale, in_scale, up_f32=None) -> np.ndarray:
    g_codes = np.ascontiguousarray(g_codes, dtype=np.int8)
    u = None if u_codes is None else np.ascontiguousarray(u_codes, dtype=np.int8)
    up = None if up_f32 is None else _f32(up_f32)
    codes = np.empty(g_codes.shape, dtype=np.int8)
    lib().g4d_gelu_mul_codes(_p(g_codes, _i8p), f32(g_scale), _p(u, _i8p), f32(u_scale),
                             _p(up, _f32p), g_codes.size, f32(in_scale), _p(codes, _i8p))
    return codes


# geluMul.ts:219-233 on f32 operands (the reference's gate and up buffers)
def gelu_mul_f32_codes(g, u, in_scale) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    codes = np.empty(g.shape, dtype=np.int8)
    lib().g4d_gelu_mul_f32_codes(_p(g, _f32p), _p(u, _f32p), g.size, f32(in_scale),
                                 _p(codes, _i8p))
    return codes


# embedGather.ts:93-113
def embed_row(row_codes, row_scale, cols, embed_scale) -> np.ndarray:
    row_codes = np.ascontiguousarray(row_codes, dtype=np.uint8)
    out = np.empty(cols, dtype=np.float32)
    lib().g4d_embed_row(_p(row_codes, _u8p), f32(row_scale), cols, f32(embed_scale),
                        _p(out, _f32p))
    return out


# plan.ts:670-690
def ple_combine(proj_codes, proj_scale, alpha, gain, identity, group, eps) -> np.ndarray:
    proj_codes = np.ascontiguousarray(proj_codes, dtype=np.int8)
    gain, identity = _f32(gain), _f32(identity)
    groups = proj_codes.size // group
    out = np.empty(proj_codes.size, dtype=np.float32)
    lib().g4d_ple_combine(_p(proj_codes, _i8p), f32(proj_scale), f32(alpha), _p(gain, _f32p),
                          _p(identity, _f32p), groups, group, f32(eps), _p(out, _f32p))
    return out


# logitSoftcap.ts:104-124
def softcap(x, cap) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().g4d_softcap(_p(x, _f32p), x.size, f32(cap), _p(out, _f32p))
    return out


# argmax.ts:267-300
def argmax(x) -> int:
    x = _f32(x)
    return int(lib().g4d_argmax(_p(x, _f32p), x.size))
