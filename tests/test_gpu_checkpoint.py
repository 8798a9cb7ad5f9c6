"""The checkpoint layer on the device: payload uploads (chunked, and BF16 / F16 widened exactly to
f32), and a decode step run from a safetensors file in the checkpoint's naming (src/safetensors.ts
textTensorNames) equal bit for bit to the same model filled on the device."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def save(path, tensors, metadata=None):
    from safetensors.numpy import save_file
    save_file(tensors, str(path), metadata=metadata)


def retype(src, dst, name, dtype):
    """Copy a safetensors file with one tensor's dtype string changed (same byte size)."""
    import json
    import struct
    body = src.read_bytes()
    hl = struct.unpack("<Q", body[:8])[0]
    head = json.loads(body[8:8 + hl])
    head[name]["dtype"] = dtype
    js = json.dumps(head).encode()
    dst.write_bytes(struct.pack("<Q", len(js)) + js + body[8 + hl:])


def test_uploads_and_exact_widening(gpu, tmp_path):
    import g4ckpt as ck
    rng = np.random.default_rng(2)
    f32 = rng.standard_normal(3000).astype(np.float32)
    bf16_bits = (f32.view(np.uint32) >> 16).astype(np.uint16)  # truncated: any bit pattern is a bf16
    f16 = rng.standard_normal(3000).astype(np.float16)
    f16[:4] = [0.0, -0.0, 6e-8, -65504.0]                      # zero, sign, subnormal, max
    big = rng.integers(0, 256, (70 << 20,), dtype=np.uint8)     # past the 64 MiB bounce buffer
    save(tmp_path / "u.safetensors", {"f32": f32, "f16": f16, "big": big,
                                      "bf16": bf16_bits.view(np.float16)})
    # numpy has no bfloat16: stored as F16 bits, then the header's dtype is rewritten
    retype(tmp_path / "u.safetensors", tmp_path / "b.safetensors", "bf16", "BF16")
    with ck.Directory.open(str(tmp_path / "b.safetensors")) as d:
        assert d.find("bf16").dtype == "BF16"
        got = d.upload_f32("bf16").download()
        assert np.array_equal(got.view(np.uint32), bf16_bits.astype(np.uint32) << 16)
        assert np.array_equal(d.upload_f32("f16").download().view(np.uint32),
                              f16.astype(np.float32).view(np.uint32))
        assert np.array_equal(d.upload_f32("f32").download().view(np.uint32), f32.view(np.uint32))
        assert np.array_equal(d.upload("big").download(), big)
        with pytest.raises(gpu.G4Error, match="not BF16, F16 or F32"):
            d.upload_f32("big")


def write_checkpoint(path, shape, replica, norm_dtype=np.float32, extra=None):
    """A model in the checkpoint's naming from the host replica of the device fill."""
    import g4decode as gd
    s = shape
    t = {}
    sc = np.float32(s.in_scale), np.float32(s.out_scale)

    def linear(base, key):
        w = replica.host(key)
        bits8 = key.endswith("ple_gate") or key.endswith("ple_proj")
        t[base + ".weight"] = w.view(np.int8) if bits8 else w
        t[base + ".weight_scale"] = replica.host(key + "_s").reshape(-1, 1)
        t[base + ".input_activation_scale"] = np.array(sc[0], np.float32)
        t[base + ".output_activation_scale"] = np.array(sc[1], np.float32)

    M = gd.CKPT_MODEL
    t[M["embed"]] = replica.host("embed")
    t[M["embed_s"]] = replica.host("embed_s").reshape(-1, 1)
    t[M["ple_table"]] = replica.host("ple_table")
    t[M["ple_table_s"]] = replica.host("ple_table_s")
    linear("model.language_model.per_layer_model_projection", "ple_model_proj")
    t[M["ple_proj_norm"]] = replica.host("ple_proj_norm").astype(norm_dtype)
    t[M["final_norm"]] = replica.host("final_norm").astype(norm_dtype)
    t["lm_head.input_activation_scale"] = np.array(sc[0], np.float32)
    t["lm_head.output_activation_scale"] = np.array(0.0, np.float32)
    for l in range(s.layers):
        for key, part in gd.CKPT_LINEARS.items():
            if key in ("k", "v") and l >= s.kv_producers:
                continue
            linear(gd.ckpt_layer(l, part), f"l{l}.{key}")
        for key, part in gd.CKPT_NORMS.items():
            if key == "k_norm" and l >= s.kv_producers:
                continue
            t[gd.ckpt_layer(l, part + ".weight")] = replica.host(f"l{l}.{key}").astype(norm_dtype)
        t[gd.ckpt_layer(l, "layer_scalar")] = np.array(replica.layer_scalar[l], np.float32)
    t.update(extra or {})
    save(path, t, metadata={"format": "pt"})
    return t


def tiny():
    import g4decode as gd
    return gd.Shape(layers=5, kv_producers=3, hidden=512, ffn=1024, q_heads=8, global_period=3,
                    sliding_window=512, kv_capacity=640, batch=1, vocab=2000)


def run(gpu, shape, model):
    import g4decode as gd
    dec = gd.Decoder(shape, model)
    dec.fill_kv_history()
    dec.set_position(600)
    nxt = gpu.DeviceBuffer.empty((shape.batch,), np.int32)
    dec.step(gpu.DeviceBuffer.from_array(np.array([7] * shape.batch, np.int32)), nxt)
    gpu.synchronize()
    out = (nxt.download(), dec.download("logits", np.float32), dec.download("hidden", np.float32))
    dec.close()
    return out


def test_decode_from_a_checkpoint_file(gpu, tmp_path):
    import g4decode as gd
    shape = tiny()
    write_checkpoint(tmp_path / "m.safetensors", shape, gd.HostReplica(shape, seed=4))
    from_file = gd.CheckpointModel(shape, str(tmp_path / "m.safetensors"))
    # the weights' families as stored, beside QUANT_RULES's answer (layers below 15: 4-bit MLPs)
    assert from_file.families["l0.gate"] == (4, 4) and from_file.families["l4.gate"] == (4, 4)
    assert from_file.families["l0.ple_gate"] == (8, 8)
    a = run(gpu, shape, from_file)
    b = run(gpu, shape, gd.SyntheticModel(shape, seed=4))
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    assert np.array_equal(a[2].view(np.uint32), b[2].view(np.uint32))


def test_checkpoint_refusals(gpu, tmp_path):
    import g4decode as gd
    shape = tiny()
    rep = gd.HostReplica(shape, seed=4)
    base = gd.ckpt_layer(4, "mlp.gate_proj")
    cases = [
        ({base + ".weight": np.zeros((shape.ffn, shape.hidden // 4), np.uint8)}, "2-bit family"),
        ({base + ".input_activation_scale": np.array(0.07, np.float32)}, "one static input scale"),
        ({"model.language_model.per_layer_model_projection.weight":
          np.zeros((shape.layers * 256, shape.hidden), np.float16)}, "bf16 dense matmul"),
    ]
    for i, (extra, fragment) in enumerate(cases):
        p = tmp_path / f"r{i}.safetensors"
        write_checkpoint(p, shape, rep, extra=extra)
        name = next(iter(extra))
        if "per_layer_model_projection" in name:
            retype(p, p, name, "BF16")  # the checkpoint stores it as bf16
        with pytest.raises(ValueError, match=fragment):
            gd.CheckpointModel(shape, str(p))


def test_ple_table_split_upload_and_gather(gpu, oracle, tmp_path):
    """BASELINE config 3 through the loader: the 1,174,405,120-byte PLE tensor of a safetensors
    file, planned for a device with 1 GiB bindings (engine.ts:308-345 declarePleSplit:
    planGatherSplit under the default 256 MiB slice cap gives 5 slices, scales whole), uploaded
    piece by piece into one device buffer per slice (buffers.ts:291-423), then gathered over the
    split plan for 2048 Zipf ids, bit for bit against the oracle on the host table."""
    import g4ckpt as ck
    import g4synth as syn
    rows, cols, groups = syn.PLE_ROWS, syn.PLE_COLS, syn.PLE_LAYERS
    print("writing the 1.17 GB PLE tensor", flush=True)
    table = syn.ple_codes("ckpt-split", rows, cols)
    scales = syn.ple_scales("ckpt-split", rows, groups).astype(np.float32)
    name = "model.language_model.embed_tokens_per_layer.embedding_quantized"
    save(tmp_path / "ple.safetensors", {name: table, name.replace("quantized", "scale"): scales})
    with ck.Directory.open(str(tmp_path / "ple.safetensors")) as d:
        plans, slices = d.plan_ple_split(name, groups, 1 << 30, 1 << 30)
        assert plans.scales_single == 1 and len(slices) == 5
        assert [(s.start_row, s.row_count) for s in slices] == [
            (0, 59904), (59904, 59904), (119808, 59904), (179712, 59904), (239616, 22528)]
        print("uploading into 5 slices", flush=True)
        parts = d.upload_split(name, slices)
        s_dev = d.upload(name.replace("quantized", "scale"))
    ids = syn.zipf_ids("ckpt-split", 2048, rows)
    ids[:3] = [0, 59904 - 1, rows - 1]  # first row, a slice's last row, the table's last row
    # every slice holds exactly its rows of the file
    for p, sl in zip(parts, slices):
        head = np.empty(4480 * 2, np.uint8)
        gpu._check(gpu.lib().g4_memcpy_d2h(head.ctypes.data, p.ptr, head.size, None))
        assert np.array_equal(head.reshape(2, -1), table[sl.start_row:sl.start_row + 2])
    dids = gpu.DeviceBuffer.from_array(ids)
    for kind, dt in (("f32", np.float32), ("f16", np.float16)):
        dst = gpu.DeviceBuffer.empty((ids.size, cols), dt)
        dst.fill(0x7B)
        gpu.ple_gather_split(parts, [s.start_row for s in slices], [s.row_count for s in slices],
                             s_dev, dids, dst, ids.size, cols, syn.PLE_GROUP)
        want = oracle.embed_gather(table[ids], scales[ids], np.arange(ids.size, dtype=np.int32),
                                   cols, syn.PLE_GROUP, out_kind=kind)
        got = dst.download()
        assert np.array_equal(got.view(np.uint32 if kind == "f32" else np.uint16),
                              want.view(np.uint32 if kind == "f32" else np.uint16)), kind


def test_decode_from_a_split_checkpoint(gpu, tmp_path):
    """A checkpoint loaded for a device whose bindings cannot hold the PLE table: the table goes
    into slices and the step's gather runs over them; every output equals the unsplit model's."""
    import g4decode as gd
    shape = tiny()
    write_checkpoint(tmp_path / "m.safetensors", shape, gd.HostReplica(shape, seed=4))
    row_bytes = shape.layers * shape.ple_dim // 2
    lim = 600 * row_bytes  # 2000 rows -> slices of 592 rows (16-row aligned): 4 slices
    split = gd.CheckpointModel(shape, str(tmp_path / "m.safetensors"), limits=(lim, lim))
    assert split.ple_split and len(split.ple_split) == 4 and "ple_table" not in split.buffers
    a = run(gpu, shape, split)
    b = run(gpu, shape, gd.SyntheticModel(shape, seed=4))
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    assert np.array_equal(a[2].view(np.uint32), b[2].view(np.uint32))
