"""g4_qgemm_noalloc (the entry point for callers that cannot allocate) against g4_qgemm: the same
outputs bit for bit, on two calls in a row that share the static scratch array, the second with a
smaller input; the oversized refusal; and the paths that need no scratch at all."""
import numpy as np
import pytest

import g4synth as syn

pytestmark = pytest.mark.gpu


def run_both(g4, bits, m, n, k, x_dtype, seed):
    w = syn.weights("noalloc", f"w{bits}_{n}_{k}", n, k, bits)
    s = syn.row_scales("noalloc", f"s{n}", n)
    x = syn.activations("noalloc", f"x{seed}", m, k, outlier_frac=0.01).astype(x_dtype)
    dw, ds, dx = (g4.DeviceBuffer.from_array(a) for a in (w, s, x))
    outs = []
    for which in ("noalloc", "qgemm"):
        dst = g4.DeviceBuffer.empty((m, n), np.int8)
        dst.fill(0x7B)
        if which == "noalloc":
            g4.qgemm_noalloc(bits, dw, ds, dx, dst, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
        else:
            g4.qgemm(bits, dw, ds, dx, dst, k, n, m, syn.IN_SCALE, syn.OUT_SCALE)
        g4.synchronize()
        outs.append(dst.download())
    return w, s, x, outs


@pytest.mark.parametrize("bits", [4, 8])
def test_noalloc_matches_qgemm_two_calls(gpu, oracle, bits):
    # first call: the tile path with f16 activations snapped into the scratch array
    print(f"noalloc bits={bits} call 1: M=512 N=1536 K=1536 f16", flush=True)
    w, s, x, (a, b) = run_both(gpu, bits, 512, 1536, 1536, np.float16, 1)
    assert np.array_equal(a, b)
    _, _, want = oracle.qgemm(bits, w, s, x.astype(np.float32), 1536, 1536, 512, syn.IN_SCALE,
                              syn.OUT_SCALE)
    assert np.array_equal(a, want)
    # second call, smaller: the scratch array still holds the first call's codes
    print(f"noalloc bits={bits} call 2: M=40 N=512 K=1024 f32", flush=True)
    w, s, x, (a, b) = run_both(gpu, bits, 40, 512, 1024, np.float32, 2)
    assert np.array_equal(a, b)
    _, _, want = oracle.qgemm(bits, w, s, x, 512, 1024, 40, syn.IN_SCALE, syn.OUT_SCALE)
    assert np.array_equal(a, want)


def test_noalloc_paths_without_scratch(gpu):
    # small M (fused snap) and int8 codes in: no scratch; the same outputs as g4_qgemm
    print("noalloc small-M and int8-in paths", flush=True)
    for m, dt in ((8, np.float16), (96, np.int8)):
        if dt == np.int8:
            w = syn.int4_weights("noalloc", "w_i8", 768, 1536)
            s = syn.row_scales("noalloc", "s_i8", 768)
            x = np.random.default_rng(3).integers(-128, 128, (m, 1536)).astype(np.int8)
            dw, ds, dx = (gpu.DeviceBuffer.from_array(a) for a in (w, s, x))
            outs = []
            for which in ("noalloc", "qgemm"):
                dst = gpu.DeviceBuffer.empty((m, 768), np.int8)
                if which == "noalloc":
                    gpu.qgemm_noalloc(4, dw, ds, dx, dst, 1536, 768, m, syn.IN_SCALE, syn.OUT_SCALE)
                else:
                    gpu.qgemm(4, dw, ds, dx, dst, 1536, 768, m, syn.IN_SCALE, syn.OUT_SCALE)
                gpu.synchronize()
                outs.append(dst.download())
            assert np.array_equal(outs[0], outs[1])
        else:
            _, _, _, (a, b) = run_both(gpu, 4, m, 768, 1536, dt, 3)
            assert np.array_equal(a, b)


def test_noalloc_refuses_oversized(gpu):
    cap = gpu.lib().g4_qgemm_noalloc_max_codes()
    m, k, n = 4096, 4096, 256
    assert m * k > cap
    rc = gpu.lib().g4_qgemm_noalloc(4, 16, 16, 16, gpu.KIND_F16, 16, gpu.KIND_I8, k, n, m,
                                    syn.IN_SCALE, syn.OUT_SCALE, None)
    assert rc == 1
    msg = gpu.lib().g4_last_error().decode()
    assert "g4_qgemm_noalloc" in msg and "scratch" in msg and str(cap) in msg
    # an invalid call gets the reference's refusal, not the size message (checked first)
    rc = gpu.lib().g4_qgemm_noalloc(4, 16, 16, 16, gpu.KIND_F16, 16, gpu.KIND_I8, 300, n, m,
                                    syn.IN_SCALE, syn.OUT_SCALE, None)
    assert rc == 1 and "K a multiple of 256" in gpu.lib().g4_last_error().decode()


@pytest.mark.parametrize("bits,k,ins", [(8, 4096, 0.0), (4, 4096, 0.0), (8, 4112, syn.IN_SCALE)])
def test_noalloc_large_calls_that_need_no_scratch(gpu, bits, k, ins):
    """M * K above the scratch size on paths that snap nothing into it: the uncalibrated serial
    qmatmul-8bit and f32 code dot (inScale 0), and 8-bit K % 128 != 0 (K 4112, the per-column
    GEMV). They run, and give g4_qgemm's outputs."""
    m, n = 4096 if k == 4096 else 2100, 64
    assert m * k > gpu.lib().g4_qgemm_noalloc_max_codes()
    print(f"noalloc large bits={bits} m={m} k={k} in={ins}", flush=True)
    w = syn.weights("noalloc", f"big{bits}_{k}", n, k, bits)
    s = syn.row_scales("noalloc", f"bigs{k}", n)
    x = syn.activations("noalloc", f"bigx{k}", m, k).astype(np.float32)
    dw, ds, dx = (gpu.DeviceBuffer.from_array(a) for a in (w, s, x))
    dt, outs_scale = (np.float32, 0.0) if ins == 0.0 else (np.int8, syn.OUT_SCALE)
    outs = []
    for which in ("noalloc", "qgemm"):
        dst = gpu.DeviceBuffer.empty((m, n), dt)
        dst.fill(0x7B)
        fn = gpu.qgemm_noalloc if which == "noalloc" else gpu.qgemm
        fn(bits, dw, ds, dx, dst, k, n, m, ins, outs_scale)
        gpu.synchronize()
        outs.append(dst.download())
    assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8))
