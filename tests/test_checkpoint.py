"""The checkpoint layer (include/g4ckpt.h) on the CPU: the safetensors directory against the
`safetensors` package's own files and every rejection the reference's parseHeader raises
(src/safetensors.ts:122-295), the tie table and guard (:616-800), SHA-256 against hashlib, the
QUANT_RULES resolution (src/quant.ts:430-513) and the text allow list (:930-985), with the
reference's own known answers where it states them."""
import hashlib
import json
import re
import struct

import numpy as np
import pytest

import g4ckpt as ck
import g4w8a8 as g4


def header_bytes(obj, pad_payload=0, raw_json=None):
    js = (raw_json if raw_json is not None else json.dumps(obj)).encode()
    return struct.pack("<Q", len(js)) + js + b"\0" * pad_payload


def expect(code, fragment, data, **kw):
    with pytest.raises(g4.G4Error) as e:
        ck.Directory.parse(data, **kw)
    assert f"safetensors {code}:" in str(e.value), str(e.value)
    assert fragment in str(e.value), str(e.value)


def test_directory_matches_the_safetensors_package(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(1)
    tensors = {
        "a.weight": rng.integers(0, 256, (16, 48)).astype(np.uint8),
        "a.weight_scale": rng.random((16, 1)).astype(np.float32),
        "b.norm.weight": rng.standard_normal(64).astype(np.float16),
        "scalar": np.array(3.5, np.float32),
        "codes": rng.integers(-128, 128, (8, 32)).astype(np.int8),
        "empty": np.zeros((0, 4), np.float32),
    }
    path = tmp_path / "m.safetensors"
    save_file(tensors, str(path), metadata={"format": "pt", "note": "x"})
    raw = path.read_bytes()
    hlen = struct.unpack("<Q", raw[:8])[0]
    head = json.loads(raw[8:8 + hlen])
    with ck.Directory.open(str(path)) as d:
        info = d.info()
        assert info["header_length"] == hlen and info["payload_start"] == 8 + hlen
        assert info["file_length"] == len(raw)
        got = {t.name: t for t in d.tensors()}
        assert set(got) == set(tensors)
        starts = [t.data_start for t in d.tensors()]
        assert starts == sorted(starts)
        for name, arr in tensors.items():
            t = got[name]
            assert list(t.shape) == head[name]["shape"]
            assert [t.data_start, t.data_end] == head[name]["data_offsets"]
            assert t.file_start == 8 + hlen + t.data_start
            assert t.byte_length == arr.nbytes and t.element_count == arr.size
            assert np.array_equal(d.read(name), arr)
        assert d.metadata("note") == "x" and d.metadata("absent") is None
        assert d.coverage_gaps() == []
        assert d.read_bytes("a.weight", 5, 7) == tensors["a.weight"].tobytes()[5:12]
        with pytest.raises(g4.G4Error, match="short-range"):
            d.read_bytes("a.weight", 760, 10)
        with pytest.raises(g4.G4Error, match="bad-entry: tensor nope is not in this checkpoint"):
            d.find("nope")


def test_parse_header_rejections():
    # readHeaderLength (safetensors.ts:130-147)
    expect("short-prefix", "need 8 bytes to read the header length, got 3", b"\1\2\3")
    expect("bad-header-length", "exceeds the 67108864 byte ceiling", struct.pack("<Q", 1 << 40))
    expect("bad-header-length", "header length 0 is not a positive integer", struct.pack("<Q", 0))
    expect("truncated-header", "header claims 100 JSON bytes so 108 are needed, got 20",
           struct.pack("<Q", 100) + b"{" * 12)
    expect("bad-json", "header JSON did not parse", header_bytes(None, raw_json='{"a": '))
    expect("bad-json", "header JSON is not an object", header_bytes([1, 2]))
    ok = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    expect("bad-entry", "__metadata__ is present but is not an object",
           header_bytes({"__metadata__": [1], "t": ok}))
    expect("bad-entry", "tensor t is not an object", header_bytes({"t": 5}))
    expect("bad-dtype", "tensor t has dtype Q8", header_bytes({"t": dict(ok, dtype="Q8")}))
    expect("bad-dtype", "tensor t has dtype undefined",
           header_bytes({"t": {"shape": [2], "data_offsets": [0, 8]}}))
    for shape in ([2, -1], [1.5], "2", [2**60], [2**30, 2**30]):
        frag = "element count that overflows" if shape == [2**30, 2**30] else "not a list of counts"
        expect("bad-shape", frag, header_bytes({"t": dict(ok, shape=shape)}))
    expect("bad-offsets", "data_offsets that are not a pair of counts",
           header_bytes({"t": dict(ok, data_offsets=[0])}))
    expect("bad-offsets", "tensor t ends at 0 before it starts at 8",
           header_bytes({"t": dict(ok, data_offsets=[8, 0])}))
    expect("size-mismatch", "tensor t spans 12 bytes but F32 [2] needs 8",
           header_bytes({"t": dict(ok, data_offsets=[0, 12])}))
    two = {"a": ok, "b": {"dtype": "U8", "shape": [4], "data_offsets": [4, 8]}}
    expect("overlap", "tensor b starts at 4 inside a which ends at 8", header_bytes(two))
    # overlaps are allowed when not rejected; a gap is reported, not thrown
    d = ck.Directory.parse(header_bytes(two), reject_overlaps=False)
    assert [t.name for t in d.tensors()] == ["a", "b"]
    gap = {"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]},
           "b": {"dtype": "U8", "shape": [4], "data_offsets": [10, 14]}}
    assert ck.Directory.parse(header_bytes(gap)).coverage_gaps() == [(4, 10)]
    # JSON details: escapes, numbers in exponent form, a repeated key keeps its last value
    esc = '{"t\\u00e9\\n": {"dtype": "U8", "shape": [2e0], "data_offsets": [0, 2]},' \
          ' "r": {"dtype": "U8", "shape": [1], "data_offsets": [9, 9]},' \
          ' "r": {"dtype": "U8", "shape": [1], "data_offsets": [2, 3]}}'
    names = {t.name: t for t in ck.Directory.parse(header_bytes(None, raw_json=esc)).tensors()}
    assert "té\n" in names and names["r"].data_start == 2


def test_open_refuses_a_short_file(tmp_path):
    p = tmp_path / "short.safetensors"
    p.write_bytes(header_bytes({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}},
                               pad_payload=8))
    with pytest.raises(g4.G4Error, match="short-range: payload ends at"):
        ck.Directory.open(str(p))


def test_ties_and_their_byte_count():
    t = ck.ties()
    assert [a for a, _, _ in t] == ["lm_head.weight", "lm_head.weight_scale"]
    # TIED_PAIR_BYTES (safetensors.ts:637): the bytes the tie keeps off the wire
    assert sum(n for _, _, n in t) == 101_711_872
    src_w, src_s = t[0][1], t[1][1]
    hdr = {src_w: {"dtype": "U8", "shape": [4, 2], "data_offsets": [0, 8]},
           src_s: {"dtype": "F32", "shape": [4, 1], "data_offsets": [8, 24]}}
    d = ck.Directory.parse(header_bytes(hdr))
    assert "lm_head.weight" not in d
    d.apply_ties()
    w = d.find("lm_head.weight")
    assert w.name == "lm_head.weight" and w.data_start == 0 and w.dtype == "U8"
    assert d.find("lm_head.weight_scale").data_start == 8
    # a table whose source the file lacks is refused (applyTies, safetensors.ts:680-690)
    d2 = ck.Directory.parse(header_bytes({src_w: hdr[src_w]}))
    with pytest.raises(g4.G4Error, match="bad-entry: tie lm_head.weight_scale points at"):
        d2.apply_ties()


def test_sha256_against_hashlib():
    rng = np.random.default_rng(3)
    for n in (0, 1, 3, 55, 56, 57, 63, 64, 65, 119, 120, 1000, 262144):
        data = rng.integers(0, 256, n).astype(np.uint8).tobytes()
        assert ck.sha256_hex(data) == hashlib.sha256(data).hexdigest(), n
    assert ck.sha256_hex(b"abc") == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"  # FIPS 180-2 B.1


def test_tie_guard_refuses_what_it_cannot_vouch_for():
    rev = "dd693ff40353f057ca5f07e945ad867f4afbf2ec"
    r = ck.tie_guard(b"\0" * 262144, "main")
    assert not r["tied"] and "is not the pinned" in r["reason"] and r["digest"] == ""
    r = ck.tie_guard(b"\0" * 100, rev)
    assert not r["tied"] and "sample is 100 bytes, expected 262144" in r["reason"]
    sample = np.random.default_rng(4).integers(0, 256, 262144).astype(np.uint8).tobytes()
    r = ck.tie_guard(sample, rev)
    assert not r["tied"] and r["digest"] == hashlib.sha256(sample).hexdigest()
    assert "The checkpoint is not the one the tie was verified on" in r["reason"]


# The checkpoint's module_quant_configs (quant.ts:449-461), restated with Python's regex engine to
# cross-check the native leftmost-match resolution on many paths.
PY_RULES = [("^lm_head$", 2), (r"audio_tower(?!.*lconv1d\.linear_start)", 2),
            (r"audio_tower\.layers\.\d+\.lconv1d\.linear_start\.", 4),
            (r"language_model\.embed_tokens$", 2), (r"language_model\.embed_tokens_per_layer$", 4),
            (r"language_model\.layers\.(\d|1[0-4])\.mlp\.", 4),
            (r"language_model\.layers\.\d+\.mlp\.", 2),
            (r"language_model\.layers\.\d+\.per_layer_input_gate$", 8),
            (r"language_model\.layers\.\d+\.per_layer_projection$", 8),
            (r"language_model\.layers\.\d+\.self_attn\.", 4), ("vision_tower", 8)]


def py_bits(path):
    best, bits = None, 4
    for pat, b in PY_RULES:
        m = re.search(pat, path)
        if m and (best is None or m.start() < best):
            best, bits = m.start(), b
    return bits


def test_quant_bits_known_answers():
    L = "model.language_model"
    # TEXT_STORAGE_FAMILIES (quant.ts:546-647) and the producer / consumer split (quant.ts:432-436)
    assert ck.quant_bits(f"{L}.layers.0.self_attn.q_proj") == 4
    assert ck.quant_bits(f"{L}.layers.14.mlp.down_proj") == 4
    assert ck.quant_bits(f"{L}.layers.15.mlp.gate_proj") == 2
    assert ck.quant_bits(f"{L}.layers.0.per_layer_input_gate") == 8
    assert ck.quant_bits(f"{L}.layers.34.per_layer_projection") == 8
    assert ck.quant_bits(f"{L}.embed_tokens") == 2
    assert ck.quant_bits(f"{L}.embed_tokens_per_layer") == 4
    assert ck.quant_bits("lm_head") == 2
    for stored in (f"{L}.layers.3.input_layernorm", f"{L}.norm", f"{L}.layers.3.self_attn.q_norm",
                   f"{L}.per_layer_model_projection", f"{L}.layers.3.layer_scalar",
                   f"{L}.layers.3.self_attn.k_cache_scale", "model.embed_vision.x"):
        assert ck.quant_bits(stored) is None, stored
    paths = [f"{L}.layers.{i}.{m}" for i in range(36) for m in
             ("mlp.gate_proj", "mlp.up_proj", "self_attn.o_proj", "per_layer_input_gate",
              "per_layer_projection", "something")]
    paths += ["model.audio_tower.layers.3.lconv1d.linear_start.x", "model.audio_tower.layers.3.ffw",
              "model.vision_tower.encoder.attn", "model.language_model.embed_tokens.x", "foo.bar"]
    for p in paths:
        assert ck.quant_bits(p) == py_bits(p), p


def test_module_path_for_tensor():
    for name, want in (("a.b.weight_scale", "a.b"), ("a.b.input_activation_scale", "a.b"),
                       ("a.b.output_activation_scale", "a.b"), ("x.embedding_quantized", "x"),
                       ("x.embedding_scale", "x"), ("a.b.weight", "a.b"), ("a.layer_scalar", "a.layer_scalar")):
        assert ck.module_path_for_tensor(name) == want


def test_text_allow_list_counts():
    # safetensors.ts:345-349: "the 1,439 text tensors of the mobile checkpoint with the lm_head tie
    # taken" and "1,441 tensors ... before the tie"
    names = ck.text_tensor_names(35, 20)
    assert len(names) == 1439 and len(set(names)) == 1439
    assert len(ck.text_tensor_names(35, 20, fetch_tied_pair=True)) == 1441
    assert "model.language_model.layers.14.self_attn.k_proj.weight" in names
    assert "model.language_model.layers.15.self_attn.k_proj.weight" not in names
    assert "lm_head.weight" not in names and "lm_head.input_activation_scale" in names


def test_split_upload_and_plan_refusals(g4, tmp_path):
    """declareSplit's refusals (buffers.ts:291-327) and declarePleSplit's (engine.ts:308-345),
    checked before any device work, so they run without a GPU."""
    import g4ckpt as ck
    from safetensors.numpy import save_file
    name = "model.language_model.embed_tokens_per_layer.embedding_quantized"
    codes = np.zeros((4096, 4480), np.uint8)
    save_file({name: codes, name.replace("quantized", "scale"): np.zeros((4096, 35), np.float32)},
              str(tmp_path / "p.safetensors"))
    with ck.Directory.open(str(tmp_path / "p.safetensors")) as d:
        # a 4 GiB device: one buffer, no slices
        plans, slices = d.plan_ple_split(name, 35, 4_294_967_292, 4_294_967_292)
        assert plans.codes.single and slices == []
        # 4 MiB bindings: 5 code slices of 928 rows (16-row aligned), scales 573,440 B whole
        plans, slices = d.plan_ple_split(name, 35, 4 << 20, 4 << 20)
        assert plans.scales_single and [s.row_count for s in slices] == [928] * 4 + [384]
        # 256 KiB bindings: the scales split too, which the sliced gather cannot address
        with pytest.raises(g4.G4Error, match="scales do NOT fit in one binding"):
            d.plan_ple_split(name, 35, 256 << 10, 256 << 10)
        with pytest.raises(g4.G4Error, match="storage bindings against a budget of 3"):
            d.plan_ple_split(name, 35, 4 << 20, 4 << 20, 3)

        def sl(i, off, n):
            return g4.TableSlice(i, 0, 0, off, n)
        total = codes.nbytes
        fake = [16, 16]
        with pytest.raises(g4.G4Error, match="needs at least one range"):
            d.upload_split(name, [], [])
        with pytest.raises(g4.G4Error, match="slice 1 starts at 100, not at 64; the ranges have to "
                                             "partition the tensor in offset order"):
            d.upload_split(name, [sl(0, 0, 64), sl(1, 100, total - 100)], fake)
        with pytest.raises(g4.G4Error, match="slice 1 starts at 66, which is not four byte aligned"):
            d.upload_split(name, [sl(0, 0, 66), sl(1, 66, total - 66)], fake)
        with pytest.raises(g4.G4Error, match="outside every declared slice"):
            d.upload_split(name, [sl(0, 0, 64), sl(1, 64, 64)], fake)
