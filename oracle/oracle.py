"""numpy front end of the C oracle (oracle/g4_oracle.c).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline). The product library never
loads it.

Each wrapper names the reference function it restates; the C file carries the file:line citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libg4oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_vp = ctypes.c_void_p


def build() -> str:
    """Compile the oracle with its Makefile (gcc). Returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_round_ties_even.restype = ctypes.c_float
        L.or_round_ties_even.argtypes = [ctypes.c_float]
        L.or_srq_code_f32.restype = ctypes.c_float
        L.or_srq_code_f32.argtypes = [ctypes.c_float, ctypes.c_float]
        L.or_srq_code.restype = ctypes.c_int8
        L.or_srq_code.argtypes = [ctypes.c_float, ctypes.c_float]
        L.or_apply_srq.argtypes = [_f32p, ctypes.c_int64, ctypes.c_float, _f32p]
        L.or_srq_codes.argtypes = [_f32p, ctypes.c_int64, ctypes.c_float, _i8p]
        L.or_unpack_int4.argtypes = [_u8p, ctypes.c_int64, _i8p]
        L.or_unpack_int8.argtypes = [_u8p, ctypes.c_int64, _i8p]
        L.or_pack_codes.argtypes = [ctypes.c_int, _i8p, ctypes.c_int64, _u8p]
        L.or_f32_to_f16_bits.restype = ctypes.c_uint16
        L.or_f32_to_f16_bits.argtypes = [ctypes.c_float]
        L.or_f16_bits_to_f32.restype = ctypes.c_float
        L.or_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
        L.or_qgemm.restype = ctypes.c_int
        L.or_qgemm.argtypes = [ctypes.c_int, _u8p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                               ctypes.c_int64, ctypes.c_float, ctypes.c_float, _f32p, _i32p, _i8p]
        L.or_qmatmul8.restype = ctypes.c_int
        L.or_qmatmul8.argtypes = [_u8p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.c_float, ctypes.c_float, _f32p]
        L.or_qgemv_split.restype = ctypes.c_int
        L.or_qgemv_split.argtypes = [ctypes.c_int, _u8p, _f32p, _f32p, ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                     _f32p]
        L.or_qgemv_merge.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, _f32p]
        L.or_qgemv_exact_merge.argtypes = [_f32p, _f32p, ctypes.c_int64, ctypes.c_int,
                                           ctypes.c_float, ctypes.c_float, _f32p]
        L.or_ple_gate_split.restype = ctypes.c_int
        L.or_ple_gate_split.argtypes = [_u8p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int, ctypes.c_float, _f32p]
        L.or_ple_fold_gate.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _f32p, ctypes.c_float,
                                       ctypes.c_float, _f32p]
        L.or_qgemv_tile8u.restype = ctypes.c_int
        L.or_qgemv_tile8u.argtypes = [_u8p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_float, ctypes.c_float, _f32p, _i8p]
        L.or_qgemv_ref_lane_sum.restype = ctypes.c_float
        L.or_qgemv_ref_lane_sum.argtypes = [ctypes.c_int, _u8p, _i8p, ctypes.c_int64]
        L.or_embed_gather.restype = ctypes.c_int
        L.or_embed_gather.argtypes = [_u8p, _vp, ctypes.c_int, _i32p, ctypes.c_int64,
                                      ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                      ctypes.c_int64, ctypes.c_int64, _vp, ctypes.c_int]
        L.or_plan_table_split.restype = ctypes.c_int64
        L.or_plan_table_split.argtypes = [ctypes.c_int64] * 5 + [_i64p, _i64p, _i64p, _i64p,
                                                                 ctypes.c_int64]
        L.or_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def num_threads() -> int:
    return lib().or_num_threads()


# quant.ts:350-357
def round_ties_even(x: float) -> float:
    return lib().or_round_ties_even(float(x))


# quant.ts:309-334 (one value, f32 code and int8 code)
def srq_code_f32(v: float, s: float) -> float:
    return lib().or_srq_code_f32(float(v), float(s))


def srq_codes(x: np.ndarray, scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, dtype=np.int8)
    lib().or_srq_codes(_p(x, _f32p), x.size, float(np.float32(scale)), _p(out, _i8p))
    return out


# quant.ts:278-288
def apply_srq(x: np.ndarray, scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty_like(x)
    lib().or_apply_srq(_p(x, _f32p), x.size, float(np.float32(scale)), _p(out, _f32p))
    return out


# quant.ts:87-152
def unpack(bits: int, packed: np.ndarray, width: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(width, dtype=np.int8)
    fn = lib().or_unpack_int4 if bits == 4 else lib().or_unpack_int8
    fn(_p(packed, _u8p), width, _p(out, _i8p))
    return out


def pack(bits: int, codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.int8).ravel()
    n = (codes.size + 1) // 2 if bits == 4 else codes.size
    out = np.empty(n, dtype=np.uint8)
    lib().or_pack_codes(bits, _p(codes, _i8p), codes.size, _p(out, _u8p))
    return out


def pack_matrix(bits: int, codes: np.ndarray) -> np.ndarray:
    """Pack a [rows, k] code matrix row by row (row-major packed rows)."""
    rows, k = codes.shape
    assert bits == 8 or k % 2 == 0, "4-bit rows pack whole bytes"
    return pack(bits, codes.reshape(-1)).reshape(rows, -1)


# f16Cast.ts:120-155
def f32_to_f16_bits(v: float) -> int:
    return lib().or_f32_to_f16_bits(float(v))


def f16_bits_to_f32(h: int) -> float:
    return lib().or_f16_bits_to_f32(int(h))


def qgemm(bits: int, packed: np.ndarray, scales: np.ndarray, x: np.ndarray, num_rows: int, k: int,
          m_cols: int, in_scale: float, out_scale: float):
    """qgemvOracle per column (qgemv.ts:1131-1176, qgemm.ts:532-552).

    Returns (dst_f32 [m, N], acc_i32 [m, N], codes_i8 [m, N])."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size >= m_cols * k
    out = np.empty((m_cols, num_rows), dtype=np.float32)
    acc = np.empty((m_cols, num_rows), dtype=np.int32)
    codes = np.empty((m_cols, num_rows), dtype=np.int8)
    rc = lib().or_qgemm(bits, _p(packed, _u8p), _p(scales, _f32p), _p(x, _f32p), num_rows, k,
                        m_cols, float(np.float32(in_scale)), float(np.float32(out_scale)),
                        _p(out, _f32p), _p(acc, _i32p), _p(codes, _i8p))
    assert rc == 0, "or_qgemm rejected its arguments"
    return out, acc, codes


def qgemv(bits, packed, scales, x, num_rows, k, in_scale, out_scale):
    out, acc, codes = qgemm(bits, packed, scales, x, num_rows, k, 1, in_scale, out_scale)
    return out[0], acc[0], codes[0]


# pleMatmul.ts:176-229
def qmatmul8(packed, scales, x, num_rows, k, m_cols, in_scale, out_scale) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty((m_cols, num_rows), dtype=np.float32)
    rc = lib().or_qmatmul8(_p(packed, _u8p), _p(scales, _f32p), _p(x, _f32p), num_rows, k, m_cols,
                           float(np.float32(in_scale)), float(np.float32(out_scale)),
                           _p(out, _f32p))
    assert rc == 0
    return out


# qgemv.ts:521-548, exactSplit.ts:16
def qgemv_split(bits, packed, scales, x, num_rows, k, splits, exact, in_scale) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty((num_rows, splits), dtype=np.float32)
    rc = lib().or_qgemv_split(bits, _p(packed, _u8p), _p(scales, _f32p), _p(x, _f32p), num_rows,
                              k, splits, 1 if exact else 0, float(np.float32(in_scale)),
                              _p(out, _f32p))
    assert rc == 0
    return out


# pleSplit.ts:17-23: exact 8-bit split partials, row-interleaved; flat [num_rows * splits]
def ple_gate_split(packed, scales, x, num_rows, k, splits, in_scale) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(num_rows * splits, dtype=np.float32)
    rc = lib().or_ple_gate_split(_p(packed, _u8p), _p(scales, _f32p), _p(x, _f32p), num_rows, k,
                                 splits, float(np.float32(in_scale)), _p(out, _f32p))
    assert rc == 0
    return out


# pleSplit.ts:33-41 foldGate over the interleaved partials: the gate's f32 values [k]
def ple_fold_gate(partials, k, splits, gate_scales, gate_in, gate_out) -> np.ndarray:
    partials = np.ascontiguousarray(partials, dtype=np.float32)
    gate_scales = np.ascontiguousarray(gate_scales, dtype=np.float32)
    assert partials.size == k * splits and gate_scales.size >= k
    out = np.empty(k, dtype=np.float32)
    lib().or_ple_fold_gate(_p(partials, _f32p), k, splits, _p(gate_scales, _f32p),
                           float(np.float32(gate_in)), float(np.float32(gate_out)), _p(out, _f32p))
    return out


# qgemv.ts:1027-1072 / attnPrologue.ts:287-296
def qgemv_merge(partials: np.ndarray, out_scale: float) -> np.ndarray:
    partials = np.ascontiguousarray(partials, dtype=np.float32)
    rows, splits = partials.shape
    out = np.empty(rows, dtype=np.float32)
    lib().or_qgemv_merge(_p(partials, _f32p), rows, splits, float(np.float32(out_scale)),
                         _p(out, _f32p))
    return out


# exactSplit.ts:45-57
def qgemv_exact_merge(partials, scales, in_scale, out_scale) -> np.ndarray:
    partials = np.ascontiguousarray(partials, dtype=np.float32)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    rows, splits = partials.shape
    out = np.empty(rows, dtype=np.float32)
    lib().or_qgemv_exact_merge(_p(partials, _f32p), _p(scales, _f32p), rows, splits,
                               float(np.float32(in_scale)), float(np.float32(out_scale)),
                               _p(out, _f32p))
    return out


# qgemv.ts:497-519, 680 + subgroupReduce.ts:49-59
def qgemv_ref_lane_sum(bits: int, row_packed: np.ndarray, xq: np.ndarray, k: int) -> float:
    row_packed = np.ascontiguousarray(row_packed, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    return lib().or_qgemv_ref_lane_sum(bits, _p(row_packed, _u8p), _p(xq, _i8p), k)


# qgemv.ts:870-1015 (the tile8u loop; row-layout weights in, the tile layout being a permutation)
def qgemv_tile8u(packed, scales, x, num_rows, k, in_scale, out_scale):
    """Returns (dst_f32 [N], codes_i8 [N]) as the tile8u geometry of qgemv-4bit computes them."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(num_rows, dtype=np.float32)
    codes = np.empty(num_rows, dtype=np.int8)
    rc = lib().or_qgemv_tile8u(_p(packed, _u8p), _p(scales, _f32p), _p(x, _f32p), num_rows, k,
                               float(np.float32(in_scale)), float(np.float32(out_scale)),
                               _p(out, _f32p), _p(codes, _i8p))
    assert rc == 0, "or_qgemv_tile8u rejected its arguments"
    return out, codes


# embedGather.ts:319-344 (+ sliced guard :188-196)
def embed_gather(codes: np.ndarray, scales: np.ndarray, ids: np.ndarray, cols: int,
                 group_size: int, out_kind: str = "f16", sliced: bool = False,
                 slice_start: int = 0, slice_count: int = 0, out: np.ndarray | None = None):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales)
    assert scales.dtype in (np.float32, np.float16)
    scale_kind = 1 if scales.dtype == np.float16 else 0
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    kinds = {"f32": (0, np.float32), "f16": (1, np.float16), "i8": (2, np.int8)}
    kind, dt = kinds[out_kind]
    if out is None:
        out = np.zeros((ids.size, cols), dtype=dt)
    assert out.dtype == dt and out.flags.c_contiguous
    rc = lib().or_embed_gather(_p(codes, _u8p), scales.ctypes.data, scale_kind, _p(ids, _i32p),
                               ids.size, cols, group_size, cols // group_size, 1 if sliced else 0,
                               slice_start, slice_count, out.ctypes.data, kind)
    assert rc == 0
    return out


# tableSplit.ts:125-215
def plan_table_split(rows: int, row_bytes: int, max_binding: int, max_buffer: int,
                     max_slice_bytes: int = 256 * 1024 * 1024):
    cap = 4096
    starts = np.zeros(cap, dtype=np.int64)
    counts = np.zeros(cap, dtype=np.int64)
    limit = ctypes.c_int64()
    per = ctypes.c_int64()
    n = lib().or_plan_table_split(rows, row_bytes, max_binding, max_buffer, max_slice_bytes,
                                  ctypes.byref(limit), ctypes.byref(per), _p(starts, _i64p),
                                  _p(counts, _i64p), cap)
    return {
        "slices": [(int(starts[i]), int(counts[i])) for i in range(min(n, cap))],
        "limit_bytes": limit.value,
        "rows_per_slice": per.value,
        "feasible": n > 0,
    }
