"""Host side of the decode step (include/g4decode.h): the E2B-shape model description, a synthetic
model filled on the device from per-tensor seeds, and the native step runner.

The reference builds its decode step from src/plan.ts (planEmbed, planLayer, planHead; the arch
constants GEMMA4_E2B at plan.ts:62-82) and walks it in src/execute.ts. Here the walk is native
(csrc/decode_step.hip); this module only describes the model, owns the device tensors and drives
`g4_decode_step`. Everything computes in the HIP library.
"""
from __future__ import annotations

import ctypes
import math
import zlib
from dataclasses import dataclass, fields

import numpy as np

import g4w8a8 as g4

_vp = ctypes.c_void_p


@dataclass
class Shape:
    """g4_decode_shape; defaults are the E2B-shape config."""
    layers: int = 35
    kv_producers: int = 15
    hidden: int = 1536
    ffn: int = 6144
    q_heads: int = 8
    head_dim: int = 256
    ple_dim: int = 256
    global_period: int = 5
    sliding_window: int = 512
    kv_capacity: int = 4096
    batch: int = 1
    vocab: int = 262144
    eps: float = 1e-6
    final_softcap: float = 30.0
    in_scale: float = float(np.float32(0.05))
    out_scale: float = float(np.float32(0.1))
    # batch 1: launch folds left out even where they fit (bit 0 o_proj in the merge, bit 1 the
    # FFN block, bit 2 the per-layer-input block); a test switch, results are identical
    fold_off: int = 0

    def c(self) -> g4.DecodeShape:
        return g4.DecodeShape(**{f.name: getattr(self, f.name) for f in fields(self)})

    def is_global(self, layer: int) -> bool:
        return layer % self.global_period == self.global_period - 1

    def kv_source(self, layer: int) -> int:
        """kv.ts:76-93: own cache on a producer, else the last producer of the same kind."""
        if layer < self.kv_producers:
            return layer
        same = [p for p in range(self.kv_producers) if self.is_global(p) == self.is_global(layer)]
        return same[-1]

    def window(self, layer: int) -> int:
        return 0 if self.is_global(layer) else self.sliding_window


def rope_tables(positions: int, head_dim: int, theta: float, partial: float):
    """rope.ts:146-180: inverse frequencies theta^(-2i/head_dim) (the denominator is head_dim, not
    the rotary width) for the head_dim * partial / 2 pairs that rotate, 0 for the rest; cos and sin
    in f64, rounded to f32. [positions][head_dim / 2]."""
    pairs = head_dim // 2
    rot = int(head_dim * partial) // 2
    inv = np.zeros(pairs)
    inv[:rot] = np.power(theta, -2.0 * np.arange(rot) / head_dim)
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def tensor_seed(seed: int, name: str) -> int:
    return (seed * 0x9E3779B1 + zlib.crc32(name.encode())) & 0xFFFFFFFFFFFFFFFF


def splitmix64(x: np.ndarray) -> np.ndarray:
    """The device fill's hash (g4_fill_hash_*), vectorised over uint64."""
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def hash_f32(n: int, seed: int, lo: float, hi: float, start: int = 0) -> np.ndarray:
    """numpy restatement of g4_fill_hash_f32 for elements start .. start + n."""
    h = splitmix64(np.uint64(seed) + np.arange(start, start + n, dtype=np.uint64))
    u = (h >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    span = np.float32(np.float32(hi) - np.float32(lo))
    return (np.float32(lo) + u * span).astype(np.float32)


def hash_u8(n: int, seed: int, start: int = 0) -> np.ndarray:
    h = splitmix64(np.uint64(seed) + np.arange(start, start + n, dtype=np.uint64))
    return (h >> np.uint64(56)).astype(np.uint8)


def _scale_range(k: int, bits: int):
    """Row scales that keep a projection's outputs around 1.5 for inputs of unit RMS: the int32
    sum of K products of a weight code of RMS w (int4 4.6, int8 73.6) and an input code of RMS
    1/in_scale is brought back by in_scale * scale, so y ~ scale * sqrt(K) * w."""
    w_rms = 4.6 if bits == 4 else 73.6
    center = 1.5 / (math.sqrt(k) * w_rms)
    return 0.5 * center, 1.5 * center


def model_spec(s: Shape):
    """Every tensor of the synthetic model: (name, kind, shape, lo, hi); kind "u8" (packed int4
    pairs or int8 codes, uniform bytes) or "f32" (uniform in [lo, hi)). Projections are int4
    except the per-layer gate and projection (int8, plan.ts:116-117); one f32 scale per row."""
    H, F, QW, P = s.hidden, s.ffn, s.q_heads * s.head_dim, s.ple_dim
    PL = s.layers * P
    spec = []

    def codes(name, n, k, bits):
        spec.append((name, "u8", (n, k // 2 if bits == 4 else k), 0.0, 0.0))
        lo, hi = _scale_range(k, bits)
        spec.append((name + "_s", "f32", (n,), lo, hi))

    def vec(name, n, lo=0.5, hi=1.5):
        spec.append((name, "f32", (n,), lo, hi))

    spec.append(("embed", "u8", (s.vocab, H // 2), 0.0, 0.0))
    # a row scale of about 0.01 times sqrt(hidden) gives embeddings of RMS about 1.8
    vec("embed_s", s.vocab, 0.005, 0.02)
    spec.append(("ple_table", "u8", (s.vocab, PL // 2), 0.0, 0.0))
    spec.append(("ple_table_s", "f32", (s.vocab, s.layers), 0.005, 0.02))
    codes("ple_model_proj", PL, H, 4)
    vec("ple_proj_norm", P)
    vec("final_norm", H)
    for l in range(s.layers):
        pre = f"l{l}."
        prod = l < s.kv_producers
        codes(pre + "q", QW, H, 4)
        if prod:
            codes(pre + "k", s.head_dim, H, 4)
            codes(pre + "v", s.head_dim, H, 4)
        codes(pre + "o", H, QW, 4)
        codes(pre + "gate", F, H, 4)
        codes(pre + "up", F, H, 4)
        codes(pre + "down", H, F, 4)
        codes(pre + "ple_gate", P, H, 8)
        codes(pre + "ple_proj", H, P, 8)
        for n in ("input_norm", "post_attn_norm", "pre_ffn_norm", "post_ffn_norm",
                  "post_ple_norm"):
            vec(pre + n, H)
        # small q/k gains keep the scale-1.0 attention scores of order 1 (unit-RMS q and k)
        vec(pre + "q_norm", s.head_dim, 0.15, 0.35)
        if prod:
            vec(pre + "k_norm", s.head_dim, 0.15, 0.35)
    return spec


def _rope_all(s: Shape):
    out = {}
    for kind, theta, partial in (("local", 1e4, 1.0), ("global", 1e6, 0.25)):
        cos, sin = rope_tables(s.kv_capacity, s.head_dim, theta, partial)
        out[f"rope_{kind}_cos"], out[f"rope_{kind}_sin"] = cos, sin
    return out


def layer_scalars(s: Shape, seed: int) -> np.ndarray:
    return hash_f32(s.layers, tensor_seed(seed, "layer_scalar"), 0.2, 0.9)


KV_SEED, KV_AMPLITUDE = 99, 1.7


def kv_history(shape: Shape, producer: int, seed: int = KV_SEED,
               amplitude: float = KV_AMPLITUDE) -> np.ndarray:
    """Host restatement of Decoder.fill_kv_history for one producer: [batch][2][capacity][hd]."""
    n = shape.batch * 2 * shape.kv_capacity * shape.head_dim
    a = hash_f32(n, tensor_seed(seed, f"kv{producer}"), -amplitude, amplitude)
    return a.reshape(shape.batch, 2, shape.kv_capacity, shape.head_dim)


class HostReplica:
    """The same synthetic model generated on the host by the numpy restatement of the device fill
    (for small shapes: the CPU step composition without a device, or without downloads)."""

    def __init__(self, shape: Shape, seed: int = 4):
        self.shape = shape
        self.seed = seed
        self.spec = {t[0]: t for t in model_spec(shape)}
        self.rope = _rope_all(shape)
        self.layer_scalar = layer_scalars(shape, seed)
        self.cache = {}

    def host(self, name) -> np.ndarray:
        if name in self.rope:
            return self.rope[name]
        if name not in self.cache:
            _, kind, shp, lo, hi = self.spec[name]
            n = int(np.prod(shp))
            sd = tensor_seed(self.seed, name)
            a = hash_u8(n, sd) if kind == "u8" else hash_f32(n, sd, lo, hi)
            self.cache[name] = a.reshape(shp)
        return self.cache[name]

    def host_rows(self, name, rows) -> np.ndarray:
        _, kind, shp, lo, hi = self.spec[name]
        w = shp[1]
        sd = tensor_seed(self.seed, name)
        return np.stack([hash_u8(w, sd, int(r) * w) if kind == "u8" else
                         hash_f32(w, sd, lo, hi, int(r) * w) for r in rows])


class SyntheticModel:
    """Random-init weights of the E2B architecture (int4 projections and tied table, int8 per-layer
    linears), filled on the device from per-tensor seeds; host copies are fetched on demand."""

    def __init__(self, shape: Shape, seed: int = 4, stream=None):
        self.shape = s = shape
        self.seed = seed
        self.buffers: dict[str, g4.DeviceBuffer] = {}
        for name, kind, shp, lo, hi in model_spec(s):
            n = int(np.prod(shp))
            if kind == "u8":
                b = g4.DeviceBuffer(n, np.uint8, shp)
                g4._check(g4.lib().g4_fill_hash_u8(b.ptr, n, tensor_seed(seed, name), stream))
            else:
                b = g4.DeviceBuffer(n * 4, np.float32, shp)
                g4._check(g4.lib().g4_fill_hash_f32(b.ptr, n, tensor_seed(seed, name), lo, hi,
                                                    stream))
            self.buffers[name] = b
        for name, a in _rope_all(s).items():
            self.buffers[name] = g4.DeviceBuffer.from_array(a)
        self.layer_scalar = layer_scalars(s, seed)
        self._keep = None
        self.ple_split = None  # [(device buffer, start row, rows)] when the PLE table is split

    def split_ple(self, slices, drop_whole: bool = False):
        """Carry the PLE table as one device buffer per slice (g4_table_slice rows), copied from the
        whole table, the way a split checkpoint upload leaves it (buffers.ts sliceName)."""
        whole = self.buffers["ple_table"]
        row_bytes = whole.shape[1]
        parts = []
        for sl in slices:
            b = g4.DeviceBuffer(sl.row_count * row_bytes)
            g4._check(g4.lib().g4_memcpy_d2d(b.ptr, whole.ptr + sl.start_row * row_bytes,
                                              sl.row_count * row_bytes, None))
            parts.append((b, sl.start_row, sl.row_count))
        g4.synchronize()
        self.ple_split = parts
        if drop_whole:
            self.buffers.pop("ple_table").close()

    def ptr(self, name):
        b = self.buffers.get(name)
        return None if b is None else b.ptr

    def host(self, name) -> np.ndarray:
        return self.buffers[name].download()

    def host_rows(self, name, rows) -> np.ndarray:
        """Selected rows of a 2-D device tensor (the PLE table is 1.2 GB; tests read a few rows).
        A split PLE table is read from the slice that carries each row."""
        split = getattr(self, "ple_split", None)
        if name == "ple_table" and split and "ple_table" not in self.buffers:
            width = self.shape.layers * self.shape.ple_dim // 2
            out = np.empty((len(rows), width), dtype=np.uint8)
            for i, r in enumerate(rows):
                b, start, n = next(p for p in split if p[1] <= int(r) < p[1] + p[2])
                g4._check(g4.lib().g4_memcpy_d2h(out[i].ctypes.data, b.ptr + (int(r) - start) * width,
                                                  width, None))
            return out
        b = self.buffers[name]
        width = b.shape[1]
        out = np.empty((len(rows), width), dtype=b.dtype)
        for i, r in enumerate(rows):
            g4._check(g4.lib().g4_memcpy_d2h(out[i].ctypes.data, b.ptr + int(r) * width * b.dtype.itemsize,
                                              width * b.dtype.itemsize, None))
        return out

    def weights(self) -> g4.DecodeWeights:
        s = self.shape
        layers = (g4.DecodeLayer * s.layers)()
        for l in range(s.layers):
            L = layers[l]
            for f in g4.DECODE_LAYER_FIELDS:
                setattr(L, f, self.ptr(f"l{l}.{f}"))
            L.layer_scalar = float(self.layer_scalar[l])
        w = g4.DecodeWeights(**{f: self.ptr(f) for f in g4.DECODE_MODEL_FIELDS})
        w.layer = ctypes.cast(layers, ctypes.POINTER(g4.DecodeLayer))
        keep = [layers]
        split = getattr(self, "ple_split", None)
        if split:
            n = len(split)
            codes = (ctypes.c_void_p * n)(*[b.ptr for b, _, _ in split])
            starts = (ctypes.c_int64 * n)(*[st for _, st, _ in split])
            rows = (ctypes.c_int64 * n)(*[r for _, _, r in split])
            w.ple_num_slices = n
            w.ple_slice_codes = ctypes.cast(codes, ctypes.POINTER(ctypes.c_void_p))
            w.ple_slice_start = ctypes.cast(starts, ctypes.POINTER(ctypes.c_int64))
            w.ple_slice_rows = ctypes.cast(rows, ctypes.POINTER(ctypes.c_int64))
            keep += [codes, starts, rows]
        self._keep = keep
        return w

    def nbytes(self) -> int:
        return sum(b.nbytes for b in self.buffers.values())


# The checkpoint's tensor names for each device tensor of the step (textTensorNames,
# src/safetensors.ts:930-985; the families of src/quant.ts:546-647).
CKPT_MODEL = {
    "embed": "model.language_model.embed_tokens.embedding_quantized",
    "embed_s": "model.language_model.embed_tokens.embedding_scale",
    "ple_table": "model.language_model.embed_tokens_per_layer.embedding_quantized",
    "ple_table_s": "model.language_model.embed_tokens_per_layer.embedding_scale",
    "ple_model_proj": "model.language_model.per_layer_model_projection.weight",
    "ple_model_proj_s": "model.language_model.per_layer_model_projection.weight_scale",
    "ple_proj_norm": "model.language_model.per_layer_projection_norm.weight",
    "final_norm": "model.language_model.norm.weight",
}
CKPT_LINEARS = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
                "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
                "down": "mlp.down_proj", "ple_gate": "per_layer_input_gate",
                "ple_proj": "per_layer_projection"}
CKPT_NORMS = {"input_norm": "input_layernorm", "post_attn_norm": "post_attention_layernorm",
              "pre_ffn_norm": "pre_feedforward_layernorm",
              "post_ffn_norm": "post_feedforward_layernorm",
              "post_ple_norm": "post_per_layer_input_norm", "q_norm": "self_attn.q_norm",
              "k_norm": "self_attn.k_norm"}


def ckpt_layer(l: int, part: str) -> str:
    return f"model.language_model.layers.{l}.{part}"


class CheckpointModel:
    """The step's device tensors read from a local safetensors file in the checkpoint's naming
    (include/g4ckpt.h), the same interface as SyntheticModel. The lm_head pair resolves to the
    embed pair through the tie. A linear's family is read from its stored shape: int4 U8 [N, K/2]
    and int8 I8 [N, K] are served; the 2-bit families and the bf16 dense per-layer projection are
    not, and neither are activation scales that differ from the shape's one static pair."""

    def __init__(self, shape: Shape, path: str, stream=None, limits=None):
        """limits: (maxStorageBufferBindingSize, maxBufferSize) of the device profile; when the
        PLE table does not fit them it is planned and uploaded split (engine.ts:308-345)."""
        import g4ckpt as ck
        self.shape = s = shape
        self.buffers: dict[str, g4.DeviceBuffer] = {}
        self.families: dict[str, tuple] = {}
        d = ck.Directory.open(path)
        self.directory = d
        d.apply_ties()
        H, F, QW, P = s.hidden, s.ffn, s.q_heads * s.head_dim, s.ple_dim
        PL = s.layers * P

        def scalar(name):
            t = d.find(name)
            a = d.read(name).reshape(-1)
            if t.dtype == "BF16":
                return float((a.astype(np.uint32) << 16).view(np.float32)[0])
            return float(a.astype(np.float32)[0])

        def linear(key, base, n, k):
            w = d.find(base + ".weight")
            bits = {(w.dtype, (n, k // 2)): 4, (w.dtype, (n, k)): 8}.get((w.dtype, tuple(w.shape)))
            if w.dtype == "U8" and tuple(w.shape) == (n, k // 4):
                raise ValueError(f"{base}: the 2-bit family is not served by this build")
            if (w.dtype, bits) not in (("U8", 4), ("I8", 8)):
                raise ValueError(f"{base}.weight is {w.dtype} {list(w.shape)}; expected U8 "
                                 f"[{n}, {k // 2}] (int4) or I8 [{n}, {k}] (int8)")
            self.families[key] = (bits, ck.quant_bits(base))
            self.buffers[key] = d.upload(base + ".weight", stream=stream)
            sc = d.find(base + ".weight_scale")
            if sc.dtype != "F32" or sc.element_count != n:
                raise ValueError(f"{base}.weight_scale must be F32 with {n} values")
            self.buffers[key + "_s"] = d.upload(base + ".weight_scale", stream=stream)
            for which, want in (("input", s.in_scale), ("output", s.out_scale)):
                name = f"{base}.{which}_activation_scale"
                if name in d and np.float32(scalar(name)) != np.float32(want):
                    raise ValueError(f"{name} = {scalar(name)}; the step serves one static "
                                     f"{which} scale, {want}")
            return bits

        self.ple_split = None
        if limits is not None:
            plans, slices = d.plan_ple_split(CKPT_MODEL["ple_table"], s.layers, *limits)
            if slices:
                parts = d.upload_split(CKPT_MODEL["ple_table"], slices, stream=stream)
                self.ple_split = [(b, sl.start_row, sl.row_count) for b, sl in zip(parts, slices)]
        for key, name in CKPT_MODEL.items():
            if key.endswith("_s") or key in ("ple_model_proj",):
                continue
            if key == "ple_table" and self.ple_split:
                continue
            if key.endswith("norm"):
                self.buffers[key] = d.upload_f32(name, stream=stream)
            else:
                self.buffers[key] = d.upload(name, stream=stream)
        if d.find(CKPT_MODEL["ple_model_proj"]).dtype == "BF16":
            raise ValueError("per_layer_model_projection is the bf16 dense matmul, which this build "
                             "serves only as an int4 projection")
        linear("ple_model_proj", "model.language_model.per_layer_model_projection", PL, H)
        for key in ("embed_s", "ple_table_s"):
            self.buffers[key] = d.upload(CKPT_MODEL[key], stream=stream)
        if "lm_head.input_activation_scale" in d and \
                np.float32(scalar("lm_head.input_activation_scale")) != np.float32(s.in_scale):
            raise ValueError("lm_head.input_activation_scale differs from the static input scale")
        for name, a in _rope_all(s).items():
            self.buffers[name] = g4.DeviceBuffer.from_array(a)
        self.layer_scalar = np.zeros(s.layers, np.float32)
        for l in range(s.layers):
            prod = l < s.kv_producers
            dims = {"q": (QW, H), "k": (s.head_dim, H), "v": (s.head_dim, H), "o": (H, QW),
                    "gate": (F, H), "up": (F, H), "down": (H, F), "ple_gate": (P, H),
                    "ple_proj": (H, P)}
            for key, part in CKPT_LINEARS.items():
                if key in ("k", "v") and not prod:
                    continue
                bits = linear(f"l{l}.{key}", ckpt_layer(l, part), *dims[key])
                if (key in ("ple_gate", "ple_proj")) != (bits == 8):
                    raise ValueError(f"{ckpt_layer(l, part)}: int{bits} where the step runs "
                                     f"{'int8' if key in ('ple_gate', 'ple_proj') else 'int4'}")
            for key, part in CKPT_NORMS.items():
                if key == "k_norm" and not prod:
                    continue
                self.buffers[f"l{l}.{key}"] = d.upload_f32(ckpt_layer(l, part + ".weight"),
                                                           stream=stream)
            self.layer_scalar[l] = scalar(ckpt_layer(l, "layer_scalar"))
        self._keep = None

    ptr = SyntheticModel.ptr
    host = SyntheticModel.host
    host_rows = SyntheticModel.host_rows
    weights = SyntheticModel.weights
    nbytes = SyntheticModel.nbytes


class Decoder:
    """The native runner (g4_decode_create / g4_decode_step) over one model."""

    def __init__(self, shape: Shape, model: SyntheticModel):
        self.shape = shape
        self.model = model
        h = _vp()
        w = model.weights()
        sc = shape.c()
        g4._check(g4.lib().g4_decode_create(ctypes.byref(sc), ctypes.byref(w), ctypes.byref(h)))
        self.handle = h.value
        p = _vp()
        g4._check(g4.lib().g4_decode_position(self.handle, ctypes.byref(p)))
        self.pos_ptr = p.value

    def set_position(self, pos: int, stream=None):
        if not 0 <= pos < self.shape.kv_capacity:
            raise ValueError(f"position {pos} outside the KV capacity {self.shape.kv_capacity}")
        a = np.array([pos], dtype=np.int32)
        g4._check(g4.lib().g4_memcpy_h2d(self.pos_ptr, a.ctypes.data, 4, stream))
        if stream is None:
            g4.synchronize()
        self._last_pos = a  # keep the host word alive until the copy has run

    def set_position_async(self, pos: int, stream=None):
        """The position word written in stream order (g4_decode_set_position): no host wait."""
        g4._check(g4.lib().g4_decode_set_position(self.handle, pos, stream))

    def step(self, tokens, next_tokens, stream=None):
        g4._check(g4.lib().g4_decode_step(self.handle, g4._ptr(tokens), g4._ptr(next_tokens), stream))

    def set_stop(self, last_layer: int):
        g4._check(g4.lib().g4_decode_set_stop(self.handle, last_layer))

    def kv(self, layer: int):
        k, v, stride = _vp(), _vp(), ctypes.c_int64()
        g4._check(g4.lib().g4_decode_kv(self.handle, layer, ctypes.byref(k), ctypes.byref(v),
                                        ctypes.byref(stride)))
        return k.value, v.value, stride.value

    def fill_kv_history(self, seed: int = KV_SEED, amplitude: float = KV_AMPLITUDE, stream=None):
        """Every producer cache filled with seeded values in [-amplitude, amplitude): the stand-in
        for a 4096-position prompt (BASELINE config 4 decodes against a seeded KV)."""
        s = self.shape
        n = s.batch * 2 * s.kv_capacity * s.head_dim
        for p in range(s.kv_producers):
            k, _, _ = self.kv(p)
            g4._check(g4.lib().g4_fill_hash_f32(k, n, tensor_seed(seed, f"kv{p}"), -amplitude,
                                                amplitude, stream))

    def buffer(self, name: str):
        p, n = _vp(), ctypes.c_size_t()
        g4._check(g4.lib().g4_decode_buffer(self.handle, name.encode(), ctypes.byref(p),
                                            ctypes.byref(n)))
        return p.value, n.value

    def download(self, name: str, dtype) -> np.ndarray:
        p, n = self.buffer(name)
        out = np.empty(n // np.dtype(dtype).itemsize, dtype=dtype)
        g4._check(g4.lib().g4_memcpy_d2h(out.ctypes.data, p, n, None))
        return out.reshape(self.shape.batch, -1)

    def download_kv(self, layer: int) -> tuple[np.ndarray, np.ndarray]:
        """K and V of a producer: [batch][kv_capacity][head_dim] each."""
        s = self.shape
        k, _, _ = self.kv(layer)
        out = np.empty((s.batch, 2, s.kv_capacity, s.head_dim), dtype=np.float32)
        g4._check(g4.lib().g4_memcpy_d2h(out.ctypes.data, k, out.nbytes, None))
        return out[:, 0], out[:, 1]

    def close(self):
        if getattr(self, "handle", None):
            g4.lib().g4_decode_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
