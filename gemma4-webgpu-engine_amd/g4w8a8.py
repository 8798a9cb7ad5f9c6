"""Python host binding of libg4w8a8 (the C ABI in include/g4w8a8.h), over ctypes.

This is the host side the tests and bench.py drive. It mirrors the reference's operator seam
(src/kernels/registry.ts `Kernel.bind({inputs, output, params})`): `bind(name, inputs, output,
params)` takes the same kernel names, input names and params as the reference and raises
`G4Error` with the reference's message where its `bind` throws. Everything computes in the HIP
library; there is no CPU fallback. Loading fails loudly when lib/libg4w8a8.so is missing.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libg4w8a8.so")

KIND_F32, KIND_F16, KIND_I8, KIND_I32 = 0, 1, 2, 3
_KIND_OF_DTYPE = {np.dtype(np.float32): KIND_F32, np.dtype(np.float16): KIND_F16,
                  np.dtype(np.int8): KIND_I8, np.dtype(np.int32): KIND_I32}
MAX_GROUP = 16

_c_int, _c_float, _vp, _i64 = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_int64


class G4Error(RuntimeError):
    """A refused argument or failed launch, carrying the library's status and message."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class GemvDesc(ctypes.Structure):
    _fields_ = [("wq", _vp), ("scales", _vp), ("x", _vp), ("dst", _vp), ("bits", _c_int),
                ("x_kind", _c_int), ("out_kind", _c_int), ("k", _c_int), ("num_rows", _c_int),
                ("in_scale", _c_float), ("out_scale", _c_float)]


class GeluAct(ctypes.Structure):
    """include/g4w8a8.h g4_gelu_act: the fused gelu prologue's up operand."""
    _fields_ = [("up", _vp), ("up_kind", _c_int), ("gate_scale", _c_float),
                ("up_scale", _c_float), ("up_offset", _i64)]


class TableSplitInput(ctypes.Structure):
    _fields_ = [("rows", _i64), ("row_bytes", _i64), ("max_storage_buffer_binding_size", _i64),
                ("max_buffer_size", _i64), ("max_storage_buffers_per_shader_stage", _i64),
                ("max_slice_bytes", _i64)]


class TableSlice(ctypes.Structure):
    _fields_ = [("index", _i64), ("start_row", _i64), ("row_count", _i64), ("byte_offset", _i64),
                ("byte_length", _i64)]


class TableSplitPlan(ctypes.Structure):
    _fields_ = [("rows", _i64), ("row_bytes", _i64), ("total_bytes", _i64), ("limit_bytes", _i64),
                ("rows_per_slice", _i64), ("num_slices", _i64), ("single", ctypes.c_int32),
                ("feasible", ctypes.c_int32), ("storage_bindings_per_dispatch", _i64),
                ("binding_budget", _i64), ("dispatches_per_gather", _i64)]


class GatherLimits(ctypes.Structure):
    """include/g4w8a8.h g4_gather_limits (tableSplit.ts GatherLimits)."""
    _fields_ = [("max_storage_buffer_binding_size", _i64), ("max_buffer_size", _i64),
                ("max_storage_buffers_per_shader_stage", _i64)]


class GatherSplitPlans(ctypes.Structure):
    """include/g4w8a8.h g4_gather_split_plans (tableSplit.ts GatherSplitPlans, no note)."""
    _fields_ = [("codes", TableSplitPlan), ("scales", TableSplitPlan),
                ("scales_single", ctypes.c_int32)]


class DecodeShape(ctypes.Structure):
    """include/g4decode.h g4_decode_shape."""
    _fields_ = [(n, _c_int) for n in ("layers", "kv_producers", "hidden", "ffn", "q_heads",
                                      "head_dim", "ple_dim", "global_period", "sliding_window",
                                      "kv_capacity", "batch")] + [
        ("vocab", _i64), ("eps", _c_float), ("final_softcap", _c_float), ("in_scale", _c_float),
        ("out_scale", _c_float), ("fold_off", _c_int)]


DECODE_LAYER_FIELDS = ("q", "k", "v", "o", "gate", "up", "down", "ple_gate", "ple_proj",
                       "q_s", "k_s", "v_s", "o_s", "gate_s", "up_s", "down_s", "ple_gate_s",
                       "ple_proj_s", "input_norm", "post_attn_norm", "pre_ffn_norm",
                       "post_ffn_norm", "post_ple_norm", "q_norm", "k_norm")


class DecodeLayer(ctypes.Structure):
    """include/g4decode.h g4_decode_layer (device pointers plus the layer scalar)."""
    _fields_ = [(n, _vp) for n in DECODE_LAYER_FIELDS] + [("layer_scalar", _c_float)]


DECODE_MODEL_FIELDS = ("embed", "embed_s", "ple_table", "ple_table_s", "ple_model_proj",
                       "ple_model_proj_s", "ple_proj_norm", "final_norm", "rope_local_cos",
                       "rope_local_sin", "rope_global_cos", "rope_global_sin")


class DecodeWeights(ctypes.Structure):
    """include/g4decode.h g4_decode_weights."""
    _fields_ = [(n, _vp) for n in DECODE_MODEL_FIELDS] + [
        ("layer", ctypes.POINTER(DecodeLayer)), ("ple_num_slices", _c_int),
        ("ple_slice_codes", ctypes.POINTER(_vp)), ("ple_slice_start", ctypes.POINTER(_i64)),
        ("ple_slice_rows", ctypes.POINTER(_i64))]


class StTensor(ctypes.Structure):
    """include/g4ckpt.h g4_st_tensor."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_char_p), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * 8), ("data_start", ctypes.c_int64),
                ("data_end", ctypes.c_int64), ("file_start", ctypes.c_int64),
                ("file_end", ctypes.c_int64), ("byte_length", ctypes.c_int64),
                ("element_count", ctypes.c_int64)]


_u64 = ctypes.c_uint64
_sz = ctypes.c_size_t
_i32p = ctypes.POINTER(ctypes.c_int32)

# Every symbol include/g4w8a8.h and include/g4decode.h declare, with its ctypes signature
# (restype, argtypes).
SIGNATURES = {
    "g4_abi_version": (_c_int, []),
    "g4_last_error": (ctypes.c_char_p, []),
    "g4_device_count": (_c_int, [ctypes.POINTER(_c_int)]),
    "g4_set_device": (_c_int, [_c_int]),
    "g4_malloc": (_c_int, [ctypes.POINTER(_vp), ctypes.c_size_t]),
    "g4_free": (_c_int, [_vp]),
    "g4_memcpy_h2d": (_c_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "g4_memcpy_d2h": (_c_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "g4_memcpy_d2d": (_c_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "g4_fill_u8": (_c_int, [_vp, ctypes.c_uint8, ctypes.c_size_t, _vp]),
    "g4_stream_create": (_c_int, [ctypes.POINTER(_vp)]),
    "g4_stream_destroy": (_c_int, [_vp]),
    "g4_stream_synchronize": (_c_int, [_vp]),
    "g4_device_synchronize": (_c_int, []),
    "g4_event_create": (_c_int, [ctypes.POINTER(_vp)]),
    "g4_event_destroy": (_c_int, [_vp]),
    "g4_event_record": (_c_int, [_vp, _vp]),
    "g4_event_synchronize": (_c_int, [_vp]),
    "g4_event_elapsed_ms": (_c_int, [ctypes.POINTER(_c_float), _vp, _vp]),
    "g4_graph_begin_capture": (_c_int, [_vp]),
    "g4_graph_end_capture": (_c_int, [_vp, ctypes.POINTER(_vp)]),
    "g4_host_alloc": (_c_int, [ctypes.POINTER(_vp), _sz]),
    "g4_host_free": (_c_int, [_vp]),
    "g4_memcpy_d2h_async": (_c_int, [_vp, _vp, _sz, _vp]),
    "g4_graph_launch": (_c_int, [_vp, _vp]),
    "g4_graph_destroy": (_c_int, [_vp]),
    "g4_qgemv": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                          _c_float, _c_float, _vp]),
    "g4_qgemm": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                          _c_float, _c_float, _vp]),
    "g4_linear": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                           _c_float, _c_float, _vp]),
    "g4_qgemm_noalloc": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int,
                                  _c_int, _c_float, _c_float, _vp]),
    "g4_qgemm_noalloc_max_codes": (ctypes.c_size_t, []),
    "g4_kernel_for_shape": (_c_int, [_c_int, _c_int, _c_int, _c_int, ctypes.c_char_p,
                                     ctypes.c_size_t]),
    "g4_projection_batch": (_c_int, [_c_int, _c_int, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _vp,
                                     _c_int, ctypes.POINTER(_vp), _c_int, ctypes.POINTER(_c_int),
                                     ctypes.POINTER(_c_float), ctypes.POINTER(_c_float), _c_int,
                                     _vp]),
    "g4_qgemv_grouped": (_c_int, [ctypes.POINTER(GemvDesc), _c_int, _vp]),
    "g4_qgemv_plan_create": (_c_int, [ctypes.POINTER(GemvDesc), _c_int, ctypes.POINTER(_vp)]),
    "g4_qgemv_plan_launch": (_c_int, [_vp, _vp]),
    "g4_qgemv_plan_info": (_c_int, [_vp, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)]),
    "g4_qgemv_plan_destroy": (_c_int, [_vp]),
    "g4_qgemv_split": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                                _c_float, _vp]),
    "g4_qgemv_merge": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_float, _vp]),
    "g4_qgemv_exact_merge": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_float, _c_float,
                                      _vp]),
    "g4_qgemv_gelu": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, ctypes.POINTER(GeluAct), _vp, _c_int,
                               _c_int, _c_int, _c_float, _c_float, _vp]),
    "g4_tile8u_repack": (_c_int, [_vp, _vp, _c_int, _c_int, _vp]),
    "g4_qgemv_tile8u": (_c_int, [_vp, _vp, _vp, _c_int, ctypes.POINTER(GeluAct), _vp, _c_int, _c_int,
                                 _c_int, _c_float, _c_float, _vp]),
    "g4_qgemv_gelu_split": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, ctypes.POINTER(GeluAct), _vp,
                                     _c_int, _c_int, _c_int, _c_int, _c_float, _vp]),
    "g4_qgemv_gelu_m2": (_c_int, [_c_int, _vp, _vp, _vp, _c_int, ctypes.POINTER(GeluAct), _vp,
                                  _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _vp]),
    "g4_ple_gate_split": (_c_int, [_vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_float,
                                   _vp]),
    "g4_ple_fold_projection": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_float, _c_float,
                                        ctypes.POINTER(GeluAct), _vp, _c_int, _c_int, _c_int,
                                        _c_float, _c_float, _vp]),
    "g4_qgemv_plan_create_gelu": (_c_int, [ctypes.POINTER(GemvDesc), ctypes.POINTER(GeluAct),
                                           _c_int, ctypes.POINTER(_vp)]),
    "g4_srq_quantize": (_c_int, [_vp, _c_int, _vp, _i64, _c_float, _vp]),
    "g4_ple_gather": (_c_int, [_vp, _vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                               _c_int, _i64, _i64, _vp]),
    "g4_ple_gather_split": (_c_int, [ctypes.POINTER(_vp), ctypes.POINTER(_i64),
                                     ctypes.POINTER(_i64), _c_int, _vp, _c_int, _vp, _vp, _c_int,
                                     _c_int, _c_int, _c_int, _c_int, _vp]),
    "g4_plan_table_split": (_c_int, [ctypes.POINTER(TableSplitInput),
                                     ctypes.POINTER(TableSplitPlan), ctypes.POINTER(TableSlice),
                                     _i64]),
    "g4_slice_for_row": (_i64, [ctypes.POINTER(TableSlice), _i64, _i64]),
    "g4_plan_gather_split": (_c_int, [_i64, _i64, _i64, ctypes.POINTER(GatherLimits),
                                      ctypes.POINTER(GatherSplitPlans), ctypes.POINTER(TableSlice),
                                      _i64, ctypes.POINTER(TableSlice), _i64]),
    # include/g4decode.h
    "g4_rms_join": (_c_int, [_vp, _c_int, _c_float, _vp, _vp, _c_float, _vp, _c_int, _c_int,
                             _c_float, _c_float, _vp, _vp, _vp]),
    "g4_attn_prologue": (_c_int, [_vp, _c_float, _vp, _c_float, _vp, _c_float, _vp, _vp, _vp, _vp,
                                  _c_int, _c_int, _c_int, _c_float, _vp, _vp, _vp, _i64, _c_int,
                                  _vp, _vp]),
    "g4_attention_decode": (_c_int, [_vp, _vp, _vp, _i64, _c_int, _c_int, _c_int, _c_int, _vp,
                                     _c_int, _vp, _sz, _c_float, _vp, _vp, _vp]),
    "g4_attention_workspace_bytes": (_sz, [_c_int, _c_int, _c_int, _c_int]),
    "g4_gelu_mul": (_c_int, [_vp, _c_float, _vp, _c_float, _vp, _i64, _c_int, _c_int, _c_float,
                             _vp, _vp]),
    "g4_gelu_mul_f32": (_c_int, [_vp, _vp, _vp, _i64, _c_float, _vp]),
    "g4_embed_tokens": (_c_int, [_vp, _vp, _vp, _c_int, _i64, _c_int, _c_float, _c_float, _vp,
                                 _vp, _vp]),
    "g4_ple_combine": (_c_int, [_vp, _c_float, _c_float, _vp, _vp, _c_int, _c_int, _c_int,
                                _c_float, _vp, _vp]),
    "g4_softcap_argmax": (_c_int, [_vp, _c_int, _i64, _c_float, _vp, _vp, _sz, _vp, _vp]),
    "g4_argmax_workspace_bytes": (_sz, [_c_int, _i64]),
    "g4_fill_hash_f32": (_c_int, [_vp, _i64, _u64, _c_float, _c_float, _vp]),
    "g4_fill_hash_u8": (_c_int, [_vp, _i64, _u64, _vp]),
    "g4_decode_create": (_c_int, [ctypes.POINTER(DecodeShape), ctypes.POINTER(DecodeWeights),
                                  ctypes.POINTER(_vp)]),
    "g4_decode_destroy": (_c_int, [_vp]),
    "g4_decode_kv": (_c_int, [_vp, _c_int, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                              ctypes.POINTER(_i64)]),
    "g4_decode_position": (_c_int, [_vp, ctypes.POINTER(_vp)]),
    "g4_decode_step": (_c_int, [_vp, _vp, _vp, _vp]),
    "g4_decode_set_position": (_c_int, [_vp, _c_int, _vp]),
    "g4_decode_buffer": (_c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp),
                                  ctypes.POINTER(_sz)]),
    "g4_decode_set_stop": (_c_int, [_vp, _c_int]),
    # include/g4ckpt.h
    "g4_st_parse": (_c_int, [_vp, _sz, _c_int, ctypes.POINTER(_vp)]),
    "g4_st_open": (_c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "g4_st_close": (_c_int, [_vp]),
    "g4_st_info": (_c_int, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                            ctypes.POINTER(_i64)]),
    "g4_st_count": (_i64, [_vp]),
    "g4_st_tensor_at": (_c_int, [_vp, _i64, ctypes.POINTER(StTensor)]),
    "g4_st_find": (_c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(StTensor)]),
    "g4_st_metadata": (ctypes.c_char_p, [_vp, ctypes.c_char_p]),
    "g4_st_coverage_gaps": (_i64, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i64]),
    "g4_st_apply_ties": (_c_int, [_vp]),
    "g4_st_tie_count": (_c_int, []),
    "g4_st_tie": (_c_int, [_c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                           ctypes.POINTER(_i64)]),
    "g4_st_read": (_c_int, [_vp, ctypes.c_char_p, _i64, _vp, _sz]),
    "g4_st_upload": (_c_int, [_vp, ctypes.c_char_p, _vp, _sz, _vp]),
    "g4_st_upload_f32": (_c_int, [_vp, ctypes.c_char_p, _vp, _i64, _vp]),
    "g4_st_upload_split": (_c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(TableSlice), _c_int,
                                    ctypes.POINTER(_vp), _vp]),
    "g4_st_plan_ple_split": (_c_int, [_vp, ctypes.c_char_p, _i64, ctypes.POINTER(GatherLimits),
                                      ctypes.POINTER(GatherSplitPlans), ctypes.POINTER(TableSlice),
                                      _i64]),
    "g4_tie_guard": (_c_int, [_vp, _sz, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "g4_sha256_hex": (None, [_vp, _sz, ctypes.c_char_p]),
    "g4_quant_bits": (_c_int, [ctypes.c_char_p]),
    "g4_module_path_for_tensor": (_c_int, [ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "g4_text_tensor_names": (_i64, [_c_int, _c_int, _c_int, ctypes.c_char_p, _sz,
                                    ctypes.POINTER(_sz)]),
}

_lib = None


def lib():
    """The loaded library. Raises FileNotFoundError when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `make -C gemma4-webgpu-engine_amd` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(status: int):
    if status != 0:
        msg = lib().g4_last_error().decode("utf-8", "replace")
        raise G4Error(status, msg)


def device_count() -> int:
    n = ctypes.c_int(0)
    st = lib().g4_device_count(ctypes.byref(n))
    return n.value if st == 0 else 0


# ---- device memory ------------------------------------------------------------------------------

class DeviceBuffer:
    """A device allocation owned by this object (freed on close / garbage collection)."""

    def __init__(self, nbytes: int, dtype=np.uint8, shape=None):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = _vp()
        _check(lib().g4_malloc(ctypes.byref(p), max(1, self.nbytes)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes, a.dtype, a.shape)
        buf.upload(a, stream)
        return buf

    @classmethod
    def empty(cls, shape, dtype) -> "DeviceBuffer":
        dt = np.dtype(dtype)
        return cls(int(np.prod(shape)) * dt.itemsize, dt, shape)

    def upload(self, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(lib().g4_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, stream))

    def download(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _check(lib().g4_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, stream))
        return out

    def fill(self, value: int, stream=None):
        _check(lib().g4_fill_u8(self.ptr, value & 0xFF, self.nbytes, stream))

    def close(self):
        if getattr(self, "ptr", None):
            lib().g4_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def kind(self) -> int:
        return _KIND_OF_DTYPE[self.dtype]


def _ptr(b):
    """A device address: a DeviceBuffer, anything with a .ptr, or a plain integer address."""
    if b is None:
        return None
    return int(b.ptr) if hasattr(b, "ptr") else int(b)


class Stream:
    def __init__(self):
        p = _vp()
        _check(lib().g4_stream_create(ctypes.byref(p)))
        self.handle = p.value

    def synchronize(self):
        _check(lib().g4_stream_synchronize(self.handle))

    def close(self):
        if self.handle:
            lib().g4_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        p = _vp()
        _check(lib().g4_event_create(ctypes.byref(p)))
        self.handle = p.value

    def record(self, stream=None):
        _check(lib().g4_event_record(self.handle, stream))

    def synchronize(self):
        _check(lib().g4_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(lib().g4_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return ms.value

    def close(self):
        if self.handle:
            lib().g4_event_destroy(self.handle)
            self.handle = None


class Graph:
    """A captured sequence of enqueues, replayed with one launch (hipGraphExec)."""

    def __init__(self, stream: "Stream", record):
        _check(lib().g4_graph_begin_capture(stream.handle))
        try:
            record()
        finally:
            p = _vp()
            _check(lib().g4_graph_end_capture(stream.handle, ctypes.byref(p)))
        self.handle = p.value
        self.stream = stream

    def launch(self):
        _check(lib().g4_graph_launch(self.handle, self.stream.handle))

    def close(self):
        if self.handle:
            lib().g4_graph_destroy(self.handle)
            self.handle = None


def synchronize():
    _check(lib().g4_device_synchronize())


# ---- the entry points ---------------------------------------------------------------------------

def qgemv(bits, wq, scales, x, dst, k, num_rows, cols=1, in_scale=0.0, out_scale=0.0,
          x_kind=None, out_kind=None, stream=None):
    _check(lib().g4_qgemv(bits, _ptr(wq), _ptr(scales), _ptr(x),
                          x.kind if x_kind is None else x_kind, _ptr(dst),
                          dst.kind if out_kind is None else out_kind, k, num_rows, cols,
                          float(in_scale), float(out_scale), stream))


def qgemm(bits, wq, scales, x, dst, k, num_rows, m_cols, in_scale=0.0, out_scale=0.0,
          x_kind=None, out_kind=None, stream=None):
    _check(lib().g4_qgemm(bits, _ptr(wq), _ptr(scales), _ptr(x),
                          x.kind if x_kind is None else x_kind, _ptr(dst),
                          dst.kind if out_kind is None else out_kind, k, num_rows, m_cols,
                          float(in_scale), float(out_scale), stream))


def qgemm_noalloc(bits, wq, scales, x, dst, k, num_rows, m_cols, in_scale=0.0, out_scale=0.0,
                  x_kind=None, out_kind=None, stream=None):
    """g4_qgemm without any device allocation (a static scratch array; see include/g4w8a8.h)."""
    _check(lib().g4_qgemm_noalloc(bits, _ptr(wq), _ptr(scales), _ptr(x),
                                  x.kind if x_kind is None else x_kind, _ptr(dst),
                                  dst.kind if out_kind is None else out_kind, k, num_rows, m_cols,
                                  float(in_scale), float(out_scale), stream))


def linear(bits, wq, scales, x, dst, k, num_rows, m_cols, in_scale=0.0, out_scale=0.0,
           x_kind=None, out_kind=None, stream=None):
    _check(lib().g4_linear(bits, _ptr(wq), _ptr(scales), _ptr(x),
                           x.kind if x_kind is None else x_kind, _ptr(dst),
                           dst.kind if out_kind is None else out_kind, k, num_rows, m_cols,
                           float(in_scale), float(out_scale), stream))


def kernel_for_shape(bits, m_cols, num_rows, k) -> str:
    buf = ctypes.create_string_buffer(64)
    _check(lib().g4_kernel_for_shape(bits, m_cols, num_rows, k, buf, 64))
    return buf.value.decode()


def projection_batch(bits, ws, scales, x, outs, rows, in_scales, out_scales, k, out_kind=None,
                     stream=None):
    n = len(ws)
    W = (_vp * n)(*[_ptr(w) for w in ws])
    S = (_vp * n)(*[_ptr(s) for s in scales])
    O = (_vp * n)(*[_ptr(o) for o in outs])
    R = (_c_int * n)(*rows)
    I = (_c_float * n)(*[float(v) for v in in_scales])
    U = (_c_float * n)(*[float(v) for v in out_scales])
    _check(lib().g4_projection_batch(bits, n, W, S, _ptr(x), x.kind, O,
                                     outs[0].kind if out_kind is None else out_kind, R, I, U, k,
                                     stream))


@dataclass
class Gemv:
    """One projection of a grouped launch."""
    wq: DeviceBuffer
    scales: DeviceBuffer
    x: DeviceBuffer
    dst: DeviceBuffer
    bits: int
    k: int
    num_rows: int
    in_scale: float
    out_scale: float


def make_group(items) -> ctypes.Array:
    arr = (GemvDesc * len(items))()
    for i, g in enumerate(items):
        arr[i] = GemvDesc(_ptr(g.wq), _ptr(g.scales), _ptr(g.x), _ptr(g.dst), g.bits, g.x.kind,
                          g.dst.kind, g.k, g.num_rows, float(g.in_scale), float(g.out_scale))
    return arr


def qgemv_grouped(items_or_array, stream=None):
    arr = items_or_array if isinstance(items_or_array, ctypes.Array) else make_group(items_or_array)
    _check(lib().g4_qgemv_grouped(arr, len(arr), stream))


def gelu_act(up, up_kind=None, gate_scale=0.0, up_scale=0.0, up_offset=0) -> GeluAct:
    """The fused gelu prologue's up operand (g4_gelu_act); up_kind defaults to the buffer's."""
    kind = up.kind if up_kind is None else up_kind
    return GeluAct(_ptr(up), kind, float(gate_scale), float(up_scale), int(up_offset))


class GemvPlan:
    """A device-resident grouped GEMV over any number of projections (g4_qgemv_plan_*). acts: an
    optional list (one per item, None for no prologue) of gelu_act(...) prologues."""

    def __init__(self, items, acts=None):
        self._arr = make_group(items)
        self._items = list(items)  # keeps the buffers the plan points at alive
        h = _vp()
        if acts is None:
            _check(lib().g4_qgemv_plan_create(self._arr, len(self._arr), ctypes.byref(h)))
        else:
            self._acts = (GeluAct * len(items))(*[a if a is not None else GeluAct() for a in acts])
            _check(lib().g4_qgemv_plan_create_gelu(self._arr, self._acts, len(self._arr),
                                                   ctypes.byref(h)))
        self.handle = h.value

    def launch(self, stream=None):
        _check(lib().g4_qgemv_plan_launch(self.handle, stream))

    def info(self):
        tiles, grid = _c_int(), _c_int()
        _check(lib().g4_qgemv_plan_info(self.handle, ctypes.byref(tiles), ctypes.byref(grid)))
        return tiles.value, grid.value

    def close(self):
        if self.handle:
            lib().g4_qgemv_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def qgemv_gelu(bits, wq, scales, gate, act: GeluAct, dst, k, num_rows, in_scale, out_scale,
               gate_kind=None, out_kind=None, stream=None):
    """qgemv-4bit-gelu / qgemv-8bit-gelu: gelu(gate) * up read in place of x."""
    _check(lib().g4_qgemv_gelu(bits, _ptr(wq), _ptr(scales), _ptr(gate),
                               gate.kind if gate_kind is None else gate_kind, ctypes.byref(act),
                               _ptr(dst), dst.kind if out_kind is None else out_kind, k, num_rows,
                               float(in_scale), float(out_scale), stream))


def qgemv_gelu_m2(bits, wq, scales, gate, act: GeluAct, dst, k, num_rows, cols, in_scale,
                  out_scale, gate_kind=None, out_kind=None, stream=None):
    """qgemv-4bit-gelu-m2 / qgemv-8bit-gelu-m2: the prologue over cols (1..2) token columns, gate
    and up [cols][K], dst [cols][num_rows]."""
    _check(lib().g4_qgemv_gelu_m2(bits, _ptr(wq), _ptr(scales), _ptr(gate),
                                  gate.kind if gate_kind is None else gate_kind, ctypes.byref(act),
                                  _ptr(dst), dst.kind if out_kind is None else out_kind, k,
                                  num_rows, cols, float(in_scale), float(out_scale), stream))


def ple_gate_split(wq, scales, x, partials, k, num_rows, k_splits, in_scale, stream=None):
    """ple-gate-split: exact 8-bit split partials, row-interleaved for the fold (pleSplit.ts:17-23)."""
    _check(lib().g4_ple_gate_split(_ptr(wq), _ptr(scales), _ptr(x), x.kind, _ptr(partials), k,
                                   num_rows, k_splits, float(in_scale), stream))


def ple_fold_projection(wq, scales, gate_parts, gate_scales, k_splits, gate_in_scale,
                        gate_out_scale, act: GeluAct, dst, k, num_rows, in_scale, out_scale,
                        out_kind=None, stream=None):
    """ple-fold-projection: qgemv-8bit-gelu over the fold of ple-gate-split's partials
    (pleSplit.ts:24-41)."""
    _check(lib().g4_ple_fold_projection(_ptr(wq), _ptr(scales), _ptr(gate_parts),
                                        _ptr(gate_scales), k_splits, float(gate_in_scale),
                                        float(gate_out_scale), ctypes.byref(act), _ptr(dst),
                                        dst.kind if out_kind is None else out_kind, k, num_rows,
                                        float(in_scale), float(out_scale), stream))


def qgemv_gelu_split(bits, wq, scales, gate, act: GeluAct, partials, k, num_rows, k_splits, exact,
                     in_scale, gate_kind=None, stream=None):
    """qgemv-4bit-gelu-exact-split (exact) or the scaled split over the gelu prologue's codes."""
    _check(lib().g4_qgemv_gelu_split(bits, _ptr(wq), _ptr(scales), _ptr(gate),
                                     gate.kind if gate_kind is None else gate_kind,
                                     ctypes.byref(act), _ptr(partials), k, num_rows, k_splits,
                                     1 if exact else 0, float(in_scale), stream))


def gelu_mul(gate, up, dst, count, srq_scale=0.0, stream=None):
    """gelu-mul on f32 buffers (geluMul.ts:101-116): dst = gelu_tanh(gate) * up, snapped on
    srq_scale when it is non-zero."""
    _check(lib().g4_gelu_mul_f32(_ptr(gate), _ptr(up), _ptr(dst), int(count), float(srq_scale),
                                 stream))


def tile8u_bytes(k, num_rows) -> int:
    """Bytes of a 4-bit matrix in the tile8u layout: ceil(N / 8) tiles of K u32 words."""
    return (num_rows + 7) // 8 * k * 4


def tile8u_repack(wq, tile_wq, k, num_rows, stream=None):
    """The eight-row tile layout of a row-layout 4-bit matrix (qgemv.ts:871-876)."""
    _check(lib().g4_tile8u_repack(_ptr(wq), _ptr(tile_wq), k, num_rows, stream))


def qgemv_tile8u(tile_wq, scales, x, dst, k, num_rows, in_scale=0.0, out_scale=0.0,
                 act: "GeluAct | None" = None, x_kind=None, out_kind=None, stream=None):
    """qgemv-4bit (or qgemv-4bit-gelu with act) on the tile8u geometry (qgemv.ts:870-1015)."""
    _check(lib().g4_qgemv_tile8u(_ptr(tile_wq), _ptr(scales), _ptr(x),
                                 x.kind if x_kind is None else x_kind,
                                 ctypes.byref(act) if act is not None else None, _ptr(dst),
                                 dst.kind if out_kind is None else out_kind, k, num_rows,
                                 float(in_scale), float(out_scale), stream))


def qgemv_split(bits, wq, scales, x, partials, k, num_rows, k_splits, exact, in_scale,
                stream=None):
    _check(lib().g4_qgemv_split(bits, _ptr(wq), _ptr(scales), _ptr(x), x.kind, _ptr(partials), k,
                                num_rows, k_splits, 1 if exact else 0, float(in_scale), stream))


def qgemv_merge(partials, dst, num_rows, k_splits, out_scale, stream=None):
    _check(lib().g4_qgemv_merge(_ptr(partials), _ptr(dst), dst.kind, num_rows, k_splits,
                                float(out_scale), stream))


def qgemv_exact_merge(partials, scales, dst, num_rows, k_splits, in_scale, out_scale, stream=None):
    _check(lib().g4_qgemv_exact_merge(_ptr(partials), _ptr(scales), _ptr(dst), dst.kind, num_rows,
                                      k_splits, float(in_scale), float(out_scale), stream))


def srq_quantize(x, codes, n, scale, stream=None):
    _check(lib().g4_srq_quantize(_ptr(x), x.kind, _ptr(codes), n, float(scale), stream))


def ple_gather(codes, scales, ids, dst, slots, cols, group_size, sliced=False, slice_start=0,
               slice_count=0, stream=None):
    _check(lib().g4_ple_gather(_ptr(codes), _ptr(scales), scales.kind, _ptr(ids), _ptr(dst),
                               dst.kind, slots, cols, group_size, cols // group_size,
                               1 if sliced else 0, slice_start, slice_count, stream))


def ple_gather_split(slice_codes, starts, counts, scales, ids, dst, slots, cols, group_size,
                     stream=None):
    n = len(slice_codes)
    C = (_vp * n)(*[_ptr(c) for c in slice_codes])
    S = (_i64 * n)(*starts)
    N = (_i64 * n)(*counts)
    _check(lib().g4_ple_gather_split(C, S, N, n, _ptr(scales), scales.kind, _ptr(ids), _ptr(dst),
                                     dst.kind, slots, cols, group_size, cols // group_size,
                                     stream))


def plan_table_split(rows, row_bytes, max_binding, max_buffer, max_buffers_per_stage=10,
                     max_slice_bytes=0):
    inp = TableSplitInput(rows, row_bytes, max_binding, max_buffer, max_buffers_per_stage,
                          max_slice_bytes)
    plan = TableSplitPlan()
    cap = 4096
    slices = (TableSlice * cap)()
    _check(lib().g4_plan_table_split(ctypes.byref(inp), ctypes.byref(plan), slices, cap))
    return plan, [slices[i] for i in range(min(plan.num_slices, cap))]


def plan_gather_split(rows, code_row_bytes, scales_per_row, max_binding, max_buffer,
                      max_buffers_per_stage=10):
    """planGatherSplit (tableSplit.ts:257-287): (plans, code slices, scale slices)."""
    lim = GatherLimits(max_binding, max_buffer, max_buffers_per_stage)
    plans = GatherSplitPlans()
    cap = 4096
    cs, ss = (TableSlice * cap)(), (TableSlice * cap)()
    _check(lib().g4_plan_gather_split(rows, code_row_bytes, scales_per_row, ctypes.byref(lim),
                                      ctypes.byref(plans), cs, cap, ss, cap))
    return (plans, [cs[i] for i in range(min(plans.codes.num_slices, cap))],
            [ss[i] for i in range(min(plans.scales.num_slices, cap))])


def slice_for_row(slices, row) -> int:
    arr = (TableSlice * len(slices))(*slices)
    return lib().g4_slice_for_row(arr, len(slices), row)


# ---- the registry seam (src/kernels/registry.ts:108-119) ----------------------------------------
#
# bind(name, inputs, output, params) runs the named reference kernel through the library with the
# reference's input names and params. Inputs and output are DeviceBuffers; params are numbers.

def _p(params, key, default=None):
    v = params.get(key, default)
    return default if v is None else v


def _need(inputs, names, who):
    missing = [n for n in names if inputs.get(n) is None]
    if missing:
        raise G4Error(1, f"{who} needs inputs named {', '.join(names)}")


# GemvGeometry.inner per bit width (qgemv.ts:146, 239-241; the device profile's setGemvGeometry):
# 'tile8u' makes the 4-bit pipeline the tile loop (qgemv.ts:440), which reads wq in the eight-row
# tile layout (tile8u_repack). The 8-bit family has no tile loop, so there it runs the classic one.
_gemv_inner = {4: "classic", 8: "classic"}


def set_gemv_inner(bits: int, inner: str):
    if bits not in _gemv_inner:
        raise G4Error(1, f"gemv geometry: bits must be 4 or 8, got {bits}")
    if inner not in ("classic", "tile8u"):
        raise G4Error(1, f"gemv geometry: inner must be classic or tile8u on this build, got {inner}")
    _gemv_inner[bits] = inner


def gemv_inner(bits: int) -> str:
    return _gemv_inner[bits]


def _tile8u(bits) -> bool:
    return bits == 4 and _gemv_inner[4] == "tile8u"


def _bind_gemv(bits, wide):
    def run(inputs, output, params, stream=None):
        _need(inputs, ["wq", "scales", "x"], f"qgemv-{bits}bit")
        if not wide and _tile8u(bits):
            qgemv_tile8u(inputs["wq"], inputs["scales"], inputs["x"], output, int(_p(params, "k", 0)),
                         int(_p(params, "numRows", 0)), _p(params, "inScale", 0.0),
                         _p(params, "outScale", 0.0), stream=stream)
            return
        cols = int(_p(params, "cols", 1)) if wide else 1
        qgemv(bits, inputs["wq"], inputs["scales"], inputs["x"], output, int(_p(params, "k", 0)),
              int(_p(params, "numRows", 0)), cols, _p(params, "inScale", 0.0),
              _p(params, "outScale", 0.0), stream=stream)
    return run


def _bind_gemm(bits):
    def run(inputs, output, params, stream=None):
        _need(inputs, ["wq", "scales", "x"], "qgemm-4bit" if bits == 4 else "qmatmul-8bit")
        qgemm(bits, inputs["wq"], inputs["scales"], inputs["x"], output, int(_p(params, "k", 0)),
              int(_p(params, "numRows", 0)), int(_p(params, "mCols", 1)),
              _p(params, "inScale", 0.0), _p(params, "outScale", 0.0), stream=stream)
    return run


def _bind_batch(count):
    def run(inputs, output, params, stream=None):
        out_index = int(_p(params, "outputIndex", count - 1))
        if out_index < 0 or out_index >= count:
            raise G4Error(1, "invalid batch output index")
        ws = [inputs.get(f"w{i}") for i in range(count)]
        ss = [inputs.get(f"s{i}") for i in range(count)]
        outs = [output if i == out_index else inputs.get(f"out{i}") for i in range(count)]
        if any(v is None for v in ws + ss + outs) or inputs.get("x") is None:
            raise G4Error(1, "batched projection is missing an input buffer")
        projection_batch(4, ws, ss, inputs["x"], outs,
                         [int(_p(params, f"rows{i}", 0)) for i in range(count)],
                         [_p(params, f"inScale{i}", 0.0) for i in range(count)],
                         [_p(params, f"outScale{i}", 0.0) for i in range(count)],
                         int(_p(params, "k", 0)), out_kind=output.kind, stream=stream)
    return run


def _bind_split(bits):
    def run(inputs, output, params, stream=None):
        _need(inputs, ["wq", "scales", "x"], f"qgemv-{bits}bit-split")
        if _tile8u(bits):
            raise G4Error(1, "qgemv-4bit tile8u has no K split yet")
        qgemv_split(bits, inputs["wq"], inputs["scales"], inputs["x"], output,
                    int(_p(params, "k", 0)), int(_p(params, "numRows", 0)),
                    int(_p(params, "kSplits", 1)), bool(_p(params, "exact", 0)),
                    _p(params, "inScale", 0.0), stream=stream)
    return run


def _bind_merge(inputs, output, params, stream=None):
    if inputs.get("part") is None:
        raise G4Error(1, "qgemv-merge needs an input named part")
    qgemv_merge(inputs["part"], output, int(_p(params, "numRows", 0)),
                int(_p(params, "kSplits", 0)), _p(params, "outScale", 0.0), stream=stream)


def _bind_exact_merge(inputs, output, params, stream=None):
    _need(inputs, ["part", "scales"], "qgemv-exact-merge")
    qgemv_exact_merge(inputs["part"], inputs["scales"], output, int(_p(params, "numRows", 0)),
                      int(_p(params, "kSplits", 0)), _p(params, "inScale", 0.0),
                      _p(params, "outScale", 0.0), stream=stream)


def _up_offset(params) -> int:
    """params.upOffset counts vec4s (qgemv.ts:398, execute.ts:886 layer * dim / 4); the C ABI
    takes elements."""
    return 4 * int(_p(params, "upOffset", 0))


def _bind_gelu(bits, split, wide=False):
    """qgemv-4bit-gelu / qgemv-8bit-gelu, their -m2 forms and the gelu exact split: gate and up in
    place of x (qgemv.ts:359-400, 1668-1696; qgemvWide.ts:660-709; exactSplit.ts:19-31). gate/up
    are f32 buffers (the reference's) or int8 codes with params gateScale / upScale."""
    who = (f"qgemv-{bits}bit-gelu-exact-split" if split else
           f"qgemv-{bits}bit-gelu-m2" if wide else f"qgemv-{bits}bit-gelu")

    def run(inputs, output, params, stream=None):
        _need(inputs, ["wq", "scales", "gate", "up"], who)
        act = gelu_act(inputs["up"], gate_scale=_p(params, "gateScale", 0.0),
                       up_scale=_p(params, "upScale", 0.0), up_offset=_up_offset(params))
        if split:
            qgemv_gelu_split(bits, inputs["wq"], inputs["scales"], inputs["gate"], act, output,
                             int(_p(params, "k", 0)), int(_p(params, "numRows", 0)),
                             int(_p(params, "kSplits", 1)), True, _p(params, "inScale", 0.0),
                             stream=stream)
        elif not wide and _tile8u(bits):
            qgemv_tile8u(inputs["wq"], inputs["scales"], inputs["gate"], output,
                         int(_p(params, "k", 0)), int(_p(params, "numRows", 0)),
                         _p(params, "inScale", 0.0), _p(params, "outScale", 0.0), act=act,
                         stream=stream)
        elif wide:
            qgemv_gelu_m2(bits, inputs["wq"], inputs["scales"], inputs["gate"], act, output,
                          int(_p(params, "k", 0)), int(_p(params, "numRows", 0)),
                          int(_p(params, "cols", 0)), _p(params, "inScale", 0.0),
                          _p(params, "outScale", 0.0), stream=stream)
        else:
            qgemv_gelu(bits, inputs["wq"], inputs["scales"], inputs["gate"], act, output,
                       int(_p(params, "k", 0)), int(_p(params, "numRows", 0)),
                       _p(params, "inScale", 0.0), _p(params, "outScale", 0.0), stream=stream)
    return run


_ple_gate_splits = 1


def set_ple_gate_splits(value: int):
    """setPleGateSplits (pleSplit.ts:11-15): the split count both PLE split kernels run."""
    global _ple_gate_splits
    if value not in (1, 2, 4, 8):
        raise G4Error(1, "PLE splits must be 1, 2, 4 or 8")
    _ple_gate_splits = int(value)


def ple_gate_splits() -> int:
    return _ple_gate_splits


def _bind_ple_gate_split(inputs, output, params, stream=None):
    """ple-gate-split (pleSplit.ts:50-63): x in, exact partials out."""
    _need(inputs, ["wq", "scales", "x"], "ple-gate-split")
    ple_gate_split(inputs["wq"], inputs["scales"], inputs["x"], output, int(_p(params, "k", 0)),
                   int(_p(params, "numRows", 0)), _ple_gate_splits, _p(params, "inScale", 0.0),
                   stream=stream)


def _bind_ple_fold(inputs, output, params, stream=None):
    """ple-fold-projection (pleSplit.ts:64-84): gate (the partials), up, gateScales."""
    _need(inputs, ["wq", "scales", "gate", "up", "gateScales"], "ple-fold-projection")
    act = gelu_act(inputs["up"], up_scale=_p(params, "upScale", 0.0), up_offset=_up_offset(params))
    ple_fold_projection(inputs["wq"], inputs["scales"], inputs["gate"], inputs["gateScales"],
                        _ple_gate_splits, _p(params, "gateInScale", 0.0),
                        _p(params, "gateOutScale", 0.0), act, output, int(_p(params, "k", 0)),
                        int(_p(params, "numRows", 0)), _p(params, "inScale", 0.0),
                        _p(params, "outScale", 0.0), stream=stream)


def _bind_gelu_mul(inputs, output, params, stream=None):
    """gelu-mul (geluMul.ts:250-278): gate and up, params count and srqScale."""
    _need(inputs, ["gate", "up"], "gelu-mul")
    gelu_mul(inputs["gate"], inputs["up"], output, int(_p(params, "count", 0)),
             _p(params, "srqScale", 0.0), stream=stream)


PLE_COLS, PLE_GROUP_SIZE = 8960, 256  # PLE_ROW_VALUES and PLE_GROUP_SIZE (quant.ts:35-37)


def _bind_gather(sliced):
    def run(inputs, output, params, stream=None):
        who = "ple-gather-4bit-sliced" if sliced else "ple-gather-4bit"
        _need(inputs, ["codes", "scales", "ids"], who)
        cols = int(_p(params, "cols", PLE_COLS))
        group = int(_p(params, "groupSize", PLE_GROUP_SIZE))
        slots = int(_p(params, "slots", 0)) or 1
        if sliced:
            start, count = params.get("sliceStartRow"), params.get("sliceRowCount")
            if start is None or count is None or not count > 0:
                raise G4Error(1, f"{who} needs params sliceStartRow and sliceRowCount naming a non "
                                 "empty vocabulary range")
        else:
            start, count = 0, inputs["codes"].nbytes // (cols // 2)
        ple_gather(inputs["codes"], inputs["scales"], inputs["ids"], output, slots, cols, group,
                   sliced, int(start), int(count), stream=stream)
    return run


KERNELS = {
    "qgemv-4bit": _bind_gemv(4, False),
    "qgemv-8bit": _bind_gemv(8, False),
    "qgemv-4bit-m2": _bind_gemv(4, True),
    "qgemv-8bit-m2": _bind_gemv(8, True),
    "qgemm-4bit": _bind_gemm(4),
    "qgemm-4bit-single": _bind_gemm(4),
    "qgemm-4bit-prefill4": _bind_gemm(4),
    "qmatmul-8bit": _bind_gemm(8),
    "qkv-batch-4bit": _bind_batch(3),
    "gate-up-batch-4bit": _bind_batch(2),
    "qgemv-4bit-gelu": _bind_gelu(4, False),
    "qgemv-8bit-gelu": _bind_gelu(8, False),
    "qgemv-4bit-gelu-m2": _bind_gelu(4, False, True),
    "qgemv-8bit-gelu-m2": _bind_gelu(8, False, True),
    "qgemv-4bit-gelu-exact-split": _bind_gelu(4, True),
    "gelu-mul": _bind_gelu_mul,
    "ple-gate-split": _bind_ple_gate_split,
    "ple-fold-projection": _bind_ple_fold,
    "qgemv-4bit-split": _bind_split(4),
    "qgemv-8bit-split": _bind_split(8),
    "qgemv-merge": _bind_merge,
    "qgemv-exact-merge": _bind_exact_merge,
    "ple-gather-4bit": _bind_gather(False),
    "ple-gather-4bit-sliced": _bind_gather(True),
}


def kernel_names():
    return list(KERNELS)


def bind(name, inputs, output, params, stream=None):
    """Run registry kernel `name` (the reference's Kernel.bind + dispatch, registry.ts:108-119).
    Unknown names are refused by name, as runtime.ts:440-444 does."""
    fn = KERNELS.get(name)
    if fn is None:
        raise G4Error(2, f"gemma4 engine: no registered kernel named {name}")
    fn(inputs, output, params, stream)
