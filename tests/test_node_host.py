"""The Node host (gemma4-webgpu-engine_amd/host/index.js over the N-API addon): CPU checks of its
registry, refusals, routing mirror and split planner, and GPU parity of kernels bound through it."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import g4synth as syn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "gemma4-webgpu-engine_amd", "host", "g4w8a8.node")
needs_node = pytest.mark.skipif(NODE is None or not os.path.exists(ADDON),
                                reason="node or the N-API addon is absent")


@needs_node
def test_node_host_cpu_checks():
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "cpu_checks.js")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "cpu checks ok" in r.stdout


@needs_node
@pytest.mark.gpu
def test_node_host_gpu_parity(tmp_path, oracle):
    cases, want = [], {}

    def put(name, arr):
        np.ascontiguousarray(arr).tofile(tmp_path / name)
        return name

    # config 0 through qgemv-4bit
    n, k = 1536, 1536
    w = syn.int4_weights("node", "c0", n, k)
    s = syn.row_scales("node", "c0", n)
    x = syn.activations("node", "c0", 1, k)[0]
    want["c0"] = oracle.qgemv(4, w, s, x.astype(np.float32), n, k, syn.IN_SCALE, syn.OUT_SCALE)[2]
    cases.append({"name": "c0", "kernel": "qgemv-4bit",
                  "inputs": {"wq": {"file": put("c0.w", w), "kind": "i8"},
                             "scales": {"file": put("c0.s", s), "kind": "f32"},
                             "x": {"file": put("c0.x", x), "kind": "f16"}},
                  "output": {"bytes": n, "kind": "i8"},
                  "params": {"k": k, "numRows": n, "inScale": syn.IN_SCALE, "outScale": syn.OUT_SCALE}})
    # a prefill chunk through qgemm-4bit (M = 96, the MFMA tile path)
    m, n2 = 96, 512
    w2 = syn.int4_weights("node", "g", n2, k)
    s2 = syn.row_scales("node", "g", n2)
    x2 = syn.activations("node", "g", m, k, outlier_frac=0.01)
    want["g"] = oracle.qgemm(4, w2, s2, x2.astype(np.float32), n2, k, m, syn.IN_SCALE,
                             syn.OUT_SCALE)[2].reshape(-1)
    cases.append({"name": "g", "kernel": "qgemm-4bit",
                  "inputs": {"wq": {"file": put("g.w", w2), "kind": "i8"},
                             "scales": {"file": put("g.s", s2), "kind": "f32"},
                             "x": {"file": put("g.x", x2), "kind": "f16"}},
                  "output": {"bytes": m * n2, "kind": "i8"},
                  "params": {"k": k, "numRows": n2, "mCols": m, "inScale": syn.IN_SCALE,
                             "outScale": syn.OUT_SCALE}})
    # one vocabulary slice of a PLE table through ple-gather-4bit-sliced, f32 out
    rows, cols, slots = 64, 8960, 6
    codes = syn.ple_codes("node", rows, cols)
    scales = syn.ple_scales("node", rows).astype(np.float32)
    ids = np.array([3, 40, 17, 63, 0, 3], np.int32)
    start, count = 16, 32  # slice rows [16, 48): ids 40 and 17 inside, the rest outside
    sliced = np.frombuffer(np.full(slots * cols * 4, 0x7B, np.uint8).tobytes(), np.float32).copy()
    sliced = sliced.reshape(slots, cols)
    oracle.embed_gather(codes[start:start + count], scales, ids, cols, 256, out_kind="f32",
                        sliced=True, slice_start=start, slice_count=count, out=sliced)
    want["ple"] = sliced.reshape(-1)
    cases.append({"name": "ple", "kernel": "ple-gather-4bit-sliced",
                  "inputs": {"codes": {"file": put("ple.c", codes[start:start + count]), "kind": "i8"},
                             "scales": {"file": put("ple.s", scales), "kind": "f32"},
                             "ids": {"file": put("ple.i", ids), "kind": "i32"}},
                  "output": {"bytes": slots * cols * 4, "kind": "f32"},
                  "params": {"slots": slots, "sliceStartRow": start, "sliceRowCount": count}})
    # the down_proj of a decode MLP through qgemv-4bit-gelu: the reference's f32 gate and up, the
    # up row at an offset (upOffset), against gelu-mul codes fed to the GEMV oracle
    import decode_oracle as d
    n3, k3, off = 1536, 6144, 256
    rng = np.random.default_rng(5)
    gate = (rng.standard_normal(k3) * 2.0).astype(np.float32)
    up = (rng.standard_normal(k3 + off) * 1.5).astype(np.float32)
    w3 = syn.int4_weights("node", "down", n3, k3)
    s3 = syn.row_scales("node", "down", n3)
    act = d.gelu_mul_f32_codes(gate, up[off:], syn.IN_SCALE)
    want["gelu"] = oracle.qgemv(4, w3, s3, act.astype(np.float32) * np.float32(syn.IN_SCALE), n3,
                                k3, syn.IN_SCALE, syn.OUT_SCALE)[2]
    cases.append({"name": "gelu", "kernel": "qgemv-4bit-gelu",
                  "inputs": {"wq": {"file": put("gelu.w", w3), "kind": "i8"},
                             "scales": {"file": put("gelu.s", s3), "kind": "f32"},
                             "gate": {"file": put("gelu.g", gate), "kind": "f32"},
                             "up": {"file": put("gelu.u", up), "kind": "f32"}},
                  "output": {"bytes": n3, "kind": "i8"},
                  "params": {"k": k3, "numRows": n3, "inScale": syn.IN_SCALE,
                             "outScale": syn.OUT_SCALE, "upOffset": off // 4}})  # vec4s
    (tmp_path / "manifest.json").write_text(json.dumps({"cases": cases}))
    print("node gpu parity: running node", flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "gpu_parity.js"), str(tmp_path)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    got_c0 = np.fromfile(tmp_path / "c0.out", np.int8)
    assert np.array_equal(got_c0, want["c0"])
    got_g = np.fromfile(tmp_path / "g.out", np.int8)
    assert np.array_equal(got_g, want["g"])
    assert np.array_equal(np.fromfile(tmp_path / "gelu.out", np.int8), want["gelu"])
    got_ple = np.fromfile(tmp_path / "ple.out", np.float32)
    assert np.array_equal(got_ple.view(np.uint32), want["ple"].view(np.uint32))


_NP = {"Float32Array": np.float32, "Int8Array": np.int8, "Uint8Array": np.uint8,
       "Int32Array": np.int32}


def _load(tmp_path, spec):
    return np.fromfile(tmp_path / spec["file"], _NP[spec["type"]])


def _gelu_mul_f32(g, u):
    """geluMul.ts:101-116 without a snap: f32(gelu_tanh(g)) * u in f32, the oracle's gelu."""
    import decode_oracle as d
    gv = np.array([d.gelu_tanh(float(v)) for v in np.asarray(g, np.float32)], np.float32)
    return gv * np.asarray(u, np.float32)


@needs_node
def test_node_registry_cases_match_the_oracle(tmp_path, oracle):
    """The known answers the Node registry carries (registry.ts:72-119 `cases`), computed in JS on
    the reference's exact-grid recipe, against the C oracle's restatement of each kernel."""
    import decode_oracle as d
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "dump_cases.js"), str(tmp_path)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    cases = json.loads((tmp_path / "cases.json").read_text())
    seen = set()
    for c in cases:
        name, p = c["kernel"], c["params"]
        I = {k: _load(tmp_path, v) for k, v in c["inputs"].items()}
        want = _load(tmp_path, c["expected"])
        bits = 8 if ("8bit" in name or name.startswith("ple-gate-split")
                     or name == "ple-fold-projection") else 4
        if name.startswith(("qgemv-4bit", "qgemv-8bit", "qgemm", "qmatmul")) and "gelu" not in name \
                and "split" not in name:
            m = p.get("cols", p.get("mCols", 1))
            k, n = p["k"], p["numRows"]
            x = I["x"].reshape(m, k)
            if name == "qmatmul-8bit":
                got = oracle.qmatmul8(I["wq"], I["scales"], x, n, k, m, p["inScale"], p["outScale"])
                got = got.reshape(-1)
                if want.dtype == np.int8:
                    got = oracle.qgemm(8, I["wq"], I["scales"], x, n, k, m, p["inScale"],
                                       p["outScale"])[2].reshape(-1)
            else:
                y, _, q = oracle.qgemm(bits, I["wq"], I["scales"], x, n, k, m, p["inScale"],
                                       p["outScale"])
                got = (q if want.dtype == np.int8 else y).reshape(-1)
        elif name in ("qkv-batch-4bit", "gate-up-batch-4bit"):
            i = p["outputIndex"]
            got = oracle.qgemv(4, I[f"w{i}"], I[f"s{i}"], I["x"], p[f"rows{i}"], p["k"],
                               p[f"inScale{i}"], p[f"outScale{i}"])[0]
        elif name.endswith("-split") and "gelu" not in name and not name.startswith("ple-"):
            got = oracle.qgemv_split(bits, I["wq"], I["scales"], I["x"], p["numRows"], p["k"],
                                     p["kSplits"], p["exact"], p["inScale"]).reshape(-1)
        elif name == "qgemv-merge":
            got = oracle.qgemv_merge(I["part"].reshape(p["numRows"], -1), p["outScale"])
        elif name == "qgemv-exact-merge":
            got = oracle.qgemv_exact_merge(I["part"].reshape(p["numRows"], -1), I["scales"],
                                           p["inScale"], p["outScale"])
        elif name == "gelu-mul":
            got = oracle.apply_srq(_gelu_mul_f32(I["gate"], I["up"]), p.get("srqScale", 0.0))
        elif name == "ple-gate-split":
            n, k = p["numRows"], p["k"]
            got = oracle.ple_gate_split(I["wq"], I["scales"], I["x"], n, k, want.size // n,
                                        p["inScale"])
        elif "gelu" in name or name == "ple-fold-projection":
            k, n, m = p["k"], p["numRows"], p.get("cols", 1)
            off = 4 * p.get("upOffset", 0)  # vec4s (qgemv.ts:398)
            up = I["up"][off:off + m * k].reshape(m, k)
            if name == "ple-fold-projection":
                splits = I["gate"].size // k
                gate = oracle.ple_fold_gate(I["gate"], k, splits, I["gateScales"],
                                            p["gateInScale"], p["gateOutScale"]).reshape(1, k)
            else:
                gate = I["gate"].reshape(m, k)
            ins = p.get("inScale", 0.0)
            if ins:
                x = np.stack([d.gelu_mul_f32_codes(gate[c], up[c], ins) for c in range(m)])
                x = x.astype(np.float32) * np.float32(ins)
            else:
                x = np.stack([_gelu_mul_f32(gate[c], up[c]) for c in range(m)])
            if name.endswith("exact-split"):
                got = oracle.qgemv_split(bits, I["wq"], I["scales"], x[0], n, k, p["kSplits"],
                                         True, ins).reshape(-1)
            else:
                y, _, q = oracle.qgemm(bits, I["wq"], I["scales"], x, n, k, m, ins,
                                       p.get("outScale", 0.0))
                got = (q if want.dtype == np.int8 else y).reshape(-1)
        elif name.startswith("ple-gather"):
            sliced = name.endswith("sliced")
            out = np.zeros((p["slots"], p["cols"]), np.float32)
            oracle.embed_gather(I["codes"], I["scales"], I["ids"], p["cols"], p["groupSize"],
                                out_kind="f32", sliced=sliced,
                                slice_start=p.get("sliceStartRow", 0),
                                slice_count=p.get("sliceRowCount", 0), out=out)
            got = out.reshape(-1)
        else:
            raise AssertionError(f"no oracle for {name}")
        assert got.dtype == want.dtype or want.dtype == np.float32, (name, c["case"])
        assert np.array_equal(np.asarray(got, want.dtype).view(np.uint8), want.view(np.uint8)), \
            (name, c["case"])
        seen.add(name)
    assert len(seen) == 24


@needs_node
@pytest.mark.gpu
def test_node_registry_cases_on_gpu_and_async_readback():
    """Every registry entry's known-answer cases through the Node host on the device, and the
    asynchronous boundary: downloadAsync / synchronizeAsync settle Promises from a worker thread
    (the reference's mapAsync readback, runtime.ts:866-878) and a failing copy rejects."""
    print("node registry cases", flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "gpu_cases.js")],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["cases"] >= 40 and res["failed"] == [] and res["asyncOk"] and res["rejected"]


@needs_node
@pytest.mark.gpu
def test_node_two_decode_steps_in_flight(gpu, tmp_path):
    """Two decode steps enqueued back to back from Node (the reference keeps steps in flight,
    plan.ts:942-973): the second step reads the first's next tokens on the device, positions are
    set in stream order, and the host waits only on async downloads. Both steps are checked
    against the CPU composition of the oracle on the same seeded model and KV history."""
    import decode_ref as ref
    import g4decode as gd
    shape = gd.Shape(layers=5, kv_producers=3, hidden=512, ffn=1024, q_heads=8, global_period=3,
                     sliding_window=512, kv_capacity=640, batch=3, vocab=3000)
    seed, pos, toks = 4, 600, [11, 2999, 1234]
    spec = {"shape": {f: getattr(shape, f) for f in shape.__dataclass_fields__},
            "model_fields": list(gpu.DECODE_MODEL_FIELDS),
            "layer_fields": [f for f in gpu.DECODE_LAYER_FIELDS],
            "layer_scalar": [float(v) for v in gd.layer_scalars(shape, seed)],
            "tokens": toks, "pos": pos, "tensors": [],
            "kv_elems": shape.batch * 2 * shape.kv_capacity * shape.head_dim,
            "kv_seeds": [str(gd.tensor_seed(gd.KV_SEED, f"kv{p}")) for p in range(shape.kv_producers)],
            "kv_amplitude": gd.KV_AMPLITUDE}
    for name, kind, shp, lo, hi in gd.model_spec(shape):
        spec["tensors"].append({"name": name, "kind": kind, "shape": list(shp),
                                "seed": str(gd.tensor_seed(seed, name)), "lo": lo, "hi": hi})
    for name, a in gd._rope_all(shape).items():
        np.ascontiguousarray(a, np.float32).tofile(tmp_path / f"{name}.bin")
        spec["tensors"].append({"name": name, "kind": "host", "file": f"{name}.bin",
                                "shape": list(a.shape)})
    (tmp_path / "spec.json").write_text(json.dumps(spec))
    print("node decode in flight", flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "decode_inflight.js"),
                        str(tmp_path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    next0 = np.fromfile(tmp_path / "next0.out", np.int32)
    next1 = np.fromfile(tmp_path / "next1.out", np.int32)
    # the same model and history on the Python side, composed on the CPU
    model = gd.SyntheticModel(shape, seed=seed)
    dec = gd.Decoder(shape, model)
    dec.fill_kv_history()
    gpu.synchronize()
    kv = {p: tuple(a.copy() for a in dec.download_kv(p)) for p in range(shape.kv_producers)}
    dec.close()
    W = ref.Weights(model)
    want0 = ref.step(shape, W, kv, toks, pos)
    want1 = ref.step(shape, W, kv, [int(t) for t in want0["next"]], pos + 1)
    assert np.array_equal(next0, want0["next"]) and np.array_equal(next1, want1["next"])
    logits0 = np.fromfile(tmp_path / "logits0.out", np.float32).reshape(shape.batch, -1)
    assert np.array_equal(logits0.view(np.uint32),
                          np.asarray(want0["logits"], np.float32).view(np.uint32))
    logits = np.fromfile(tmp_path / "logits1.out", np.float32).reshape(shape.batch, -1)
    hidden = np.fromfile(tmp_path / "hidden1.out", np.float32).reshape(shape.batch, -1)
    assert np.array_equal(logits.view(np.uint32), np.asarray(want1["logits"], np.float32).view(np.uint32))
    assert np.array_equal(hidden.view(np.uint32), np.asarray(want1["hidden"], np.float32).view(np.uint32))
