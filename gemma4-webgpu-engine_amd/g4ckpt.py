"""Python front end of the checkpoint layer (include/g4ckpt.h): a safetensors directory read by the
native library, the lm_head tie and its guard, QUANT_RULES resolution and the text allow list.

Mirrors src/safetensors.ts (parseHeader, coverageGaps, applyTies, checkTieGuard, sha256Hex,
textTensorNames) and src/quant.ts (resolveQuantBits, modulePathForTensor) of the reference.
Errors raise g4w8a8.G4Error whose message starts "safetensors <code>:" with the reference's
SafetensorsErrorCode.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

import g4w8a8 as g4

_vp = ctypes.c_void_p

NUMPY_DTYPE = {"BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "U16": np.uint16,
               "I16": np.int16, "F16": np.float16, "U32": np.uint32, "I32": np.int32,
               "F32": np.float32, "U64": np.uint64, "I64": np.int64, "F64": np.float64}


@dataclass(frozen=True)
class Tensor:
    """TensorEntry (safetensors.ts:85-105)."""
    name: str
    dtype: str
    shape: tuple
    data_start: int
    data_end: int
    file_start: int
    file_end: int
    byte_length: int
    element_count: int


def _tensor(t: g4.StTensor) -> Tensor:
    return Tensor(t.name.decode(), t.dtype.decode(), tuple(t.shape[:t.ndim]), t.data_start,
                  t.data_end, t.file_start, t.file_end, t.byte_length, t.element_count)


class Directory:
    """A parsed safetensors header (from bytes) or an opened file (payload reads allowed)."""

    def __init__(self, handle):
        self.handle = handle

    @classmethod
    def parse(cls, data: bytes, reject_overlaps: bool = True) -> "Directory":
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        h = _vp()
        g4._check(g4.lib().g4_st_parse(buf, len(data), 1 if reject_overlaps else 0, ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def open(cls, path: str) -> "Directory":
        h = _vp()
        g4._check(g4.lib().g4_st_open(str(path).encode(), ctypes.byref(h)))
        return cls(h.value)

    def close(self):
        if getattr(self, "handle", None):
            g4.lib().g4_st_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        v = [ctypes.c_int64() for _ in range(4)]
        g4._check(g4.lib().g4_st_info(self.handle, *[ctypes.byref(x) for x in v]))
        return dict(zip(("header_length", "payload_start", "payload_length", "file_length"),
                        (x.value for x in v)))

    def tensors(self) -> list[Tensor]:
        out = []
        for i in range(g4.lib().g4_st_count(self.handle)):
            t = g4.StTensor()
            g4._check(g4.lib().g4_st_tensor_at(self.handle, i, ctypes.byref(t)))
            out.append(_tensor(t))
        return out

    def find(self, name: str) -> Tensor:
        t = g4.StTensor()
        g4._check(g4.lib().g4_st_find(self.handle, name.encode(), ctypes.byref(t)))
        return _tensor(t)

    def __contains__(self, name: str) -> bool:
        t = g4.StTensor()
        return g4.lib().g4_st_find(self.handle, name.encode(), ctypes.byref(t)) == 0

    def metadata(self, key: str):
        v = g4.lib().g4_st_metadata(self.handle, key.encode())
        return None if v is None else v.decode()

    def coverage_gaps(self) -> list[tuple[int, int]]:
        n = g4.lib().g4_st_coverage_gaps(self.handle, None, None, 0)
        s = (ctypes.c_int64 * max(1, n))()
        e = (ctypes.c_int64 * max(1, n))()
        g4.lib().g4_st_coverage_gaps(self.handle, s, e, n)
        return [(s[i], e[i]) for i in range(n)]

    def apply_ties(self):
        g4._check(g4.lib().g4_st_apply_ties(self.handle))

    def read_bytes(self, name: str, offset: int = 0, size: int | None = None) -> bytes:
        t = self.find(name)
        size = t.byte_length - offset if size is None else size
        buf = ctypes.create_string_buffer(max(1, size))
        g4._check(g4.lib().g4_st_read(self.handle, name.encode(), offset, buf, size))
        return buf.raw[:size]

    def read(self, name: str) -> np.ndarray:
        """A tensor as a numpy array in its stored dtype (BF16 as its uint16 bits)."""
        t = self.find(name)
        dt = np.uint16 if t.dtype == "BF16" else NUMPY_DTYPE[t.dtype]
        return np.frombuffer(self.read_bytes(name), dtype=dt).reshape(t.shape)

    def upload(self, name: str, dst=None, stream=None) -> "g4.DeviceBuffer":
        """The tensor's bytes into device memory (a new buffer unless dst is given)."""
        t = self.find(name)
        if dst is None:
            dt = np.uint16 if t.dtype == "BF16" else NUMPY_DTYPE.get(t.dtype, np.uint8)
            dst = g4.DeviceBuffer(t.byte_length, dt, t.shape or (1,))
        g4._check(g4.lib().g4_st_upload(self.handle, name.encode(), g4._ptr(dst), dst.nbytes, stream))
        return dst

    def plan_ple_split(self, codes_name: str, groups_per_row: int, max_binding: int,
                       max_buffer: int, max_buffers_per_stage: int = 10):
        """declarePleSplit's planning (engine.ts:308-345): (GatherSplitPlans, code slices). The
        slices are empty when the table fits one buffer (plans.codes.single)."""
        lim = g4.GatherLimits(max_binding, max_buffer, max_buffers_per_stage)
        plans = g4.GatherSplitPlans()
        cap = 4096
        sl = (g4.TableSlice * cap)()
        g4._check(g4.lib().g4_st_plan_ple_split(self.handle, codes_name.encode(), groups_per_row,
                                                ctypes.byref(lim), ctypes.byref(plans), sl, cap))
        n = 0 if plans.codes.single else min(plans.codes.num_slices, cap)
        return plans, [sl[i] for i in range(n)]

    def upload_split(self, name: str, slices, dsts=None, stream=None) -> list:
        """declareSplit + uploadWeight (buffers.ts:291-423): the tensor's bytes routed into one
        device buffer per slice (new buffers unless dsts is given)."""
        if dsts is None:
            dsts = [g4.DeviceBuffer(sl.byte_length) for sl in slices]
        arr = (g4.TableSlice * max(1, len(slices)))(*slices)
        ptrs = (_vp * max(1, len(dsts)))(*[g4._ptr(b) for b in dsts])
        g4._check(g4.lib().g4_st_upload_split(self.handle, name.encode(), arr, len(slices), ptrs,
                                              stream))
        return dsts

    def upload_f32(self, name: str, stream=None) -> "g4.DeviceBuffer":
        """A BF16 / F16 / F32 tensor widened exactly to f32 in device memory."""
        t = self.find(name)
        dst = g4.DeviceBuffer(4 * max(1, t.element_count), np.float32, t.shape or (1,))
        g4._check(g4.lib().g4_st_upload_f32(self.handle, name.encode(), dst.ptr, t.element_count,
                                            stream))
        return dst


def ties() -> list[tuple[str, str, int]]:
    """TIED_TENSORS (safetensors.ts:623-637): (alias, source, byte length)."""
    out = []
    for i in range(g4.lib().g4_st_tie_count()):
        a, s, n = ctypes.c_char_p(), ctypes.c_char_p(), ctypes.c_int64()
        g4._check(g4.lib().g4_st_tie(i, ctypes.byref(a), ctypes.byref(s), ctypes.byref(n)))
        out.append((a.value.decode(), s.value.decode(), n.value))
    return out


def sha256_hex(data: bytes) -> str:
    buf = ctypes.create_string_buffer(65)
    src = ctypes.create_string_buffer(bytes(data), max(1, len(data)))
    g4.lib().g4_sha256_hex(src, len(data), buf)
    return buf.value.decode()


def tie_guard(sample: bytes, revision: str) -> dict:
    """checkTieGuard (safetensors.ts:762-800)."""
    digest = ctypes.create_string_buffer(65)
    reason = ctypes.create_string_buffer(512)
    src = ctypes.create_string_buffer(bytes(sample), max(1, len(sample)))
    tied = g4.lib().g4_tie_guard(src, len(sample), revision.encode(), digest, reason, 512)
    return {"tied": bool(tied), "digest": digest.value.decode(), "reason": reason.value.decode()}


def quant_bits(module_path: str):
    """resolveQuantBits (quant.ts:494-513): 2, 4 or 8, or None when stored unquantized."""
    b = g4.lib().g4_quant_bits(module_path.encode())
    return None if b == 0 else b


def module_path_for_tensor(tensor_name: str) -> str:
    buf = ctypes.create_string_buffer(len(tensor_name) + 1)
    g4._check(g4.lib().g4_module_path_for_tensor(tensor_name.encode(), buf, len(buf)))
    return buf.value.decode()


def text_tensor_names(layers: int, kv_shared: int, fetch_tied_pair: bool = False) -> list[str]:
    """textTensorNames (safetensors.ts:930-985)."""
    need = ctypes.c_size_t()
    g4.lib().g4_text_tensor_names(layers, kv_shared, int(fetch_tied_pair), None, 0,
                                  ctypes.byref(need))
    buf = ctypes.create_string_buffer(need.value)
    g4.lib().g4_text_tensor_names(layers, kv_shared, int(fetch_tied_pair), buf, need.value, None)
    text = buf.value.decode()
    return text.split("\n") if text else []
