"""The C ABI library loads and exports every symbol include/*.h declares, and refuses bad
arguments with the reference's messages before touching a device (no compute calls here)."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = "".join(open(os.path.join(ROOT, "include", h)).read()
                   for h in sorted(os.listdir(os.path.join(ROOT, "include"))) if h.endswith(".h"))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g4_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(g4):
    syms = header_symbols()
    assert len(syms) >= 30
    for name in syms:
        assert hasattr(g4.lib(), name), name
    assert set(syms) == set(g4.SIGNATURES), set(syms) ^ set(g4.SIGNATURES)
    assert g4.lib().g4_abi_version() == 1


def expect(g4, fn, status, fragment):
    with pytest.raises(g4.G4Error) as e:
        fn()
    assert e.value.status == status, str(e.value)
    assert fragment in str(e.value), str(e.value)


def test_gemv_refusals(g4):
    L = g4.lib()
    def call(bits=4, k=1536, n=16, cols=1, xk=g4.KIND_F16, ok=g4.KIND_I8, ins=0.05, outs=0.1,
             w=0x1000, s=0x1000, x=0x1000, d=0x1000):
        g4._check(L.g4_qgemv(bits, w, s, x, xk, d, ok, k, n, cols, ins, outs, None))
    expect(g4, lambda: call(k=100), 1, "qgemv-4bit needs K a multiple of 256, got 100")
    expect(g4, lambda: call(bits=8, k=1000), 1, "qgemv-8bit needs K a multiple of 128")
    expect(g4, lambda: call(cols=3), 1, "needs params.cols in 1..2, got 3")
    expect(g4, lambda: call(n=0), 1, "qgemv needs params.k and params.numRows")
    expect(g4, lambda: call(outs=0.0), 1, "int8 output codes need a calibrated outScale")
    expect(g4, lambda: call(w=0), 1, "needs inputs named wq, scales and x")
    expect(g4, lambda: call(w=0x1008), 1, "16-byte aligned")
    expect(g4, lambda: call(bits=2), 1, "bits must be 4 or 8")


def test_gemm_batch_merge_gather_refusals(g4):
    L = g4.lib()
    expect(g4, lambda: g4._check(L.g4_qgemm(4, 0x1000, 0x1000, 0x1000, 1, 0x1000, 2, 300, 8, 11,
                                            0.1, 0.1, None)), 1, "qgemm-4bit needs K a multiple of 256")
    expect(g4, lambda: g4._check(L.g4_qgemm(8, 0x1000, 0x1000, 0x1000, 1, 0x1000, 2, 130, 8, 11,
                                            0.1, 0.1, None)), 1, "qmatmul-8bit needs K a multiple of 4")
    expect(g4, lambda: g4.projection_batch(4, [0x1000] * 2, [0x1000] * 2, _Fake(), [_Fake()] * 2,
                                           [16, 32], [0.1, 0.1], [0.1, 0.1], 256), 1,
           "gate/up batch requires equal row counts")
    expect(g4, lambda: g4._check(L.g4_qgemv_merge(0x1000, 0x1000, 0, 8, 1, 0.1, None)), 1,
           "qgemv-merge only exists on a split dispatch, got kSplits 1")
    expect(g4, lambda: g4._check(L.g4_qgemv_split(4, 0x1000, 0x1000, 0x1000, 1, 0x1000, 256, 8, 3,
                                                  0, 0.1, None)), 1, "kSplits must be 1, 2, 4 or 8")
    expect(g4, lambda: g4._check(L.g4_qgemv_split(4, 0x1000, 0x1000, 0x1000, 1, 0x1000, 256, 8, 2,
                                                  1, 0.0, None)), 1,
           "exact split needs calibrated int8 input")
    expect(g4, lambda: g4._check(L.g4_ple_gather(0x1000, 0x1000, 1, 0x1000, 0x1000, 1, 4, 8960, 256,
                                                 35, 1, 0, 0, None)), 1,
           "needs params sliceStartRow and sliceRowCount naming a non empty vocabulary range")
    expect(g4, lambda: g4._check(L.g4_ple_gather(0x1000, 0x1000, 1, 0x1000, 0x1000, 1, 4, 8960, 250,
                                                 35, 0, 0, 100, None)), 1, "does not divide")


def test_ple_split_wide_gelu_and_gelu_mul_refusals(g4):
    """pleSplit.ts:11-15, 58-59; qgemvWide.ts:522-526; geluMul.ts:253-255: refused before any
    device call, with the reference's wording."""
    import ctypes
    L = g4.lib()
    act = g4.GeluAct(0x1000, g4.KIND_F32, 0.0, 0.0, 0)
    gate_split = lambda **kw: g4._check(L.g4_ple_gate_split(
        0x1000, 0x1000, 0x1000, g4.KIND_F32, 0x1000, kw.get("k", 1536), kw.get("n", 256),
        kw.get("splits", 2), kw.get("ins", 0.05), None))
    expect(g4, lambda: gate_split(n=250), 1, "PLE split row count must be divisible by four")
    expect(g4, lambda: gate_split(ins=0.0), 1, "PLE split needs calibrated input")
    expect(g4, lambda: gate_split(splits=3), 1, "PLE splits must be 1, 2, 4 or 8")
    expect(g4, lambda: gate_split(k=1000), 1, "qgemv-8bit needs K a multiple of 128")
    fold = lambda **kw: g4._check(L.g4_ple_fold_projection(
        0x1000, 0x1000, kw.get("parts", 0x1000), kw.get("gs", 0x1000), kw.get("splits", 2), 0.05,
        0.1, ctypes.byref(kw.get("act", act)), 0x1000, g4.KIND_I8, 256, 1536, 0.05, 0.1, None))
    expect(g4, lambda: fold(splits=5), 1, "PLE splits must be 1, 2, 4 or 8")
    expect(g4, lambda: fold(gs=0), 1, "needs inputs named gate, up and gateScales")
    expect(g4, lambda: fold(parts=0x1004), 1, "16-byte aligned")
    expect(g4, lambda: fold(act=g4.GeluAct(None, g4.KIND_F32, 0.0, 0.0, 0)), 1,
           "needs inputs named gate and up")
    m2 = lambda cols: g4._check(L.g4_qgemv_gelu_m2(
        8, 0x1000, 0x1000, 0x1000, g4.KIND_F32, ctypes.byref(act), 0x1000, g4.KIND_I8, 256, 8, cols,
        0.05, 0.1, None))
    expect(g4, lambda: m2(3), 1, "qgemv-8bit-gelu-m2 needs params.cols in 1..2, got 3")
    expect(g4, lambda: g4._check(L.g4_gelu_mul_f32(0x1000, 0x1000, 0x1000, 6, 0.0, None)), 1,
           "gelu-mul needs params.count a positive multiple of 4, got 6")
    expect(g4, lambda: g4.bind("ple-fold-projection", {"wq": 1, "scales": 1, "gate": 1, "up": 1},
                               None, {}), 1, "needs inputs named wq, scales, gate, up, gateScales")
    expect(g4, lambda: g4.set_ple_gate_splits(3), 1, "PLE splits must be 1, 2, 4 or 8")
    for n in ("ple-gate-split", "ple-fold-projection", "qgemv-4bit-gelu-m2", "qgemv-8bit-gelu-m2",
              "gelu-mul"):
        assert n in g4.kernel_names(), n


def test_registry_refuses_unknown_names_and_missing_inputs(g4):
    expect(g4, lambda: g4.bind("qgemv-3bit", {}, None, {}), 2, "no registered kernel named qgemv-3bit")
    expect(g4, lambda: g4.bind("qgemv-4bit", {"wq": 1}, None, {}), 1,
           "needs inputs named wq, scales, x")
    expect(g4, lambda: g4.bind("ple-gather-4bit-sliced", {"codes": 1, "scales": 1, "ids": 1}, None,
                               {"slots": 4}), 1, "naming a non empty vocabulary range")
    expect(g4, lambda: g4.bind("gate-up-batch-4bit", {"x": 1}, None, {"outputIndex": 5}), 1,
           "invalid batch output index")
    assert "qgemv-4bit" in g4.kernel_names() and "ple-gather-4bit-sliced" in g4.kernel_names()


def test_kernel_choice_per_shape(g4):
    assert g4.kernel_for_shape(4, 1, 1536, 1536) == "qgemv-4bit-stream"
    assert g4.kernel_for_shape(8, 1, 1536, 6144) == "qgemv-8bit-stream"
    assert g4.kernel_for_shape(4, 1, 16, 1280) == "qgemv-4bit"  # 40 chunks: no streaming class
    assert g4.kernel_for_shape(4, 2, 6144, 1536) == "qgemv-4bit"
    assert g4.kernel_for_shape(4, 8, 6144, 1536) == "qgemm-4bit-mfma-small16"
    assert g4.kernel_for_shape(4, 512, 6144, 1536) == "qgemm-4bit-mfma-wide"
    assert g4.kernel_for_shape(4, 128, 6144, 1536) == "qgemm-4bit-mfma-tile"
    assert g4.kernel_for_shape(8, 512, 6144, 1536) == "qmatmul-8bit-mfma-tile"
    assert g4.kernel_for_shape(8, 4, 1536, 6144) == "qmatmul-8bit-mfma-small16"
    assert g4.kernel_for_shape(4, 32, 1536, 6144) == "qgemm-4bit-mfma-small32"
    # the tied head at a decode batch: the small kernel would re-snap x in each of 16384 blocks
    assert g4.kernel_for_shape(4, 32, 262144, 1536) == "qgemm-4bit-mfma-tile"
    assert g4.kernel_for_shape(4, 3, 262144, 1536) == "qgemm-4bit-mfma-tile"


class _Fake:
    ptr = 0x1000
    kind = 2


def test_struct_layouts_match_the_headers(g4, tmp_path):
    """ctypes mirrors of the C structs: sizes and every field offset, as gcc lays them out."""
    import ctypes
    import subprocess
    structs = {"g4_decode_shape": g4.DecodeShape, "g4_decode_layer": g4.DecodeLayer,
               "g4_decode_weights": g4.DecodeWeights, "g4_gemv_desc": g4.GemvDesc,
               "g4_table_split_input": g4.TableSplitInput, "g4_table_slice": g4.TableSlice,
               "g4_table_split_plan": g4.TableSplitPlan, "g4_gelu_act": g4.GeluAct,
               "g4_st_tensor": g4.StTensor}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "g4decode.h"', '#include "g4ckpt.h"',
             'int main(void){']
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l}
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert got[(cname, f)] == getattr(py, f).offset, (cname, f)
