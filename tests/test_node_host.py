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
                             "outScale": syn.OUT_SCALE, "upOffset": off}})
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
