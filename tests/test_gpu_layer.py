"""GPU parity of the config-1 projection set: the grouped layer GEMV, the reference's projection
batches, the split-K build and its folds, and the standalone SRQ quantizer."""
import numpy as np
import pytest

import g4synth as syn

pytestmark = pytest.mark.gpu


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(g4, shape, dtype):
    b = g4.DeviceBuffer.empty(shape, dtype)
    b.fill(0x7B)
    return b


def f32_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("down_bits", [4, 8])
def test_config1_layer_grouped(gpu, oracle, down_bits):
    print(f"config1 grouped down_bits={down_bits}", flush=True)
    items, wants = [], []
    for name, n, k in syn.LAYER_PROJECTIONS:
        bits = down_bits if name == "down" else 4
        w = syn.weights("c1", name, n, k, bits)
        s = syn.row_scales("c1", name, n)
        x = syn.activations("c1", name, 1, k)[0]
        _, acc, codes = oracle.qgemv(bits, w, s, x.astype(np.float32), n, k, syn.IN_SCALE,
                                     syn.OUT_SCALE)
        wants.append(codes)
        items.append(gpu.Gemv(dev(gpu, w), dev(gpu, s), dev(gpu, x), out_buf(gpu, (n,), np.int8),
                              bits, k, n, syn.IN_SCALE, syn.OUT_SCALE))
        if bits == 8:
            # The reference's qgemv-8bit hands per-lane f32 partials to an f32 butterfly; it agrees
            # with the exact int32 sum while every partial stays below 2^24. Assert and report.
            xq = oracle.srq_codes(x.astype(np.float32), syn.IN_SCALE)
            worst = 0
            for r in range(0, n, 97):
                ref = oracle.qgemv_ref_lane_sum(8, w[r], xq, k)
                assert ref == np.float32(acc[r])
                worst = max(worst, abs(int(acc[r])))
            print(f"int8 down: max |acc| sampled {worst} (2^24 = {1 << 24})")
    gpu.qgemv_grouped(items)
    for it, want in zip(items, wants):
        assert np.array_equal(it.dst.download(), want)


def test_projection_batches_mix_scale_routing(gpu, oracle):
    # projectionBatch.ts:130-150: uncalibrated, SRQ and clamped SRQ in one dispatch.
    g = np.random.default_rng(31)
    k = 512
    rows = [8, 8, 8]
    scales_pairs = [(0.0, 0.0), (0.1875, 0.0625), (0.015625, 0.0)]
    x = (g.integers(-64, 65, size=k) / 8.0).astype(np.float32)
    ws = [g.integers(0, 256, size=(r, k // 2), dtype=np.uint8) for r in rows]
    ss = [g.uniform(0.005, 0.02, r).astype(np.float32) for r in rows]
    for count, name in ((3, "qkv-batch-4bit"), (2, "gate-up-batch-4bit")):
        for out_index in range(count):
            print(f"batch {name} output {out_index}", flush=True)
            inputs = {"x": dev(gpu, x)}
            params = {"k": k, "outputIndex": out_index}
            outs = []
            for i in range(count):
                inputs[f"w{i}"] = dev(gpu, ws[i])
                inputs[f"s{i}"] = dev(gpu, ss[i])
                params[f"rows{i}"] = rows[i]
                params[f"inScale{i}"], params[f"outScale{i}"] = scales_pairs[i]
                o = out_buf(gpu, (rows[i],), np.float32)
                outs.append(o)
                if i != out_index:
                    inputs[f"out{i}"] = o
            gpu.bind(name, inputs, outs[out_index], params)
            for i in range(count):
                want, _, _ = oracle.qgemv(4, ws[i], ss[i], x, rows[i], k, *scales_pairs[i])
                assert f32_equal(outs[i].download(), want), (name, out_index, i)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("splits", [2, 4, 8])
def test_split_and_folds(gpu, oracle, bits, splits):
    n, k = 1536, 1536 if bits == 4 else 1536
    print(f"split bits={bits} splits={splits}", flush=True)
    w = syn.weights("split", "w", n, k, bits)
    s = syn.row_scales("split", "w", n)
    x = syn.activations("split", "x", 1, k)[0]
    x32 = x.astype(np.float32)
    wb, sb, xb = dev(gpu, w), dev(gpu, s), dev(gpu, x)
    for exact in (False, True):
        part = out_buf(gpu, (n, splits), np.float32)
        gpu.bind(f"qgemv-{bits}bit-split", {"wq": wb, "scales": sb, "x": xb}, part,
                 {"k": k, "numRows": n, "kSplits": splits, "exact": int(exact),
                  "inScale": syn.IN_SCALE})
        want = oracle.qgemv_split(bits, w, s, x32, n, k, splits, exact, syn.IN_SCALE)
        got = part.download()
        assert f32_equal(got, want)
        dst = out_buf(gpu, (n,), np.float32)
        if exact:
            gpu.bind("qgemv-exact-merge", {"part": part, "scales": sb}, dst,
                     {"numRows": n, "kSplits": splits, "inScale": syn.IN_SCALE,
                      "outScale": syn.OUT_SCALE})
            fold = oracle.qgemv_exact_merge(want, s, syn.IN_SCALE, syn.OUT_SCALE)
            # The exact fold equals the unsplit GEMV, bit for bit.
            unsplit, _, _ = oracle.qgemv(bits, w, s, x32, n, k, syn.IN_SCALE, syn.OUT_SCALE)
            assert f32_equal(fold, unsplit)
        else:
            gpu.bind("qgemv-merge", {"part": part}, dst,
                     {"numRows": n, "kSplits": splits, "outScale": syn.OUT_SCALE})
            fold = oracle.qgemv_merge(want, syn.OUT_SCALE)
        assert f32_equal(dst.download(), fold)


@pytest.mark.parametrize("kind", ["f32", "f16"])
def test_srq_quantize_kernel(gpu, oracle, kind):
    g = np.random.default_rng(41)
    x = (g.standard_normal(1_000_003) * 3).astype(np.float32)
    x[:2000] = (np.arange(2000, dtype=np.float32) - 1000) * np.float32(0.025)  # exact ties
    if kind == "f16":
        x = x.astype(np.float16)
    codes = out_buf(gpu, (x.size,), np.int8)
    gpu.srq_quantize(dev(gpu, x), codes, x.size, syn.IN_SCALE)
    assert np.array_equal(codes.download(), oracle.srq_codes(x.astype(np.float32), syn.IN_SCALE))
