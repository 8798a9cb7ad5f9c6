"""GPU parity of the streaming decode GEMV (csrc/qgemv_stream.hip) against the oracle: every
compiled shape class, ragged row counts against the tile, every activation and output kind, the
per-call entry points that route to it, and the device-resident plan over a whole 35-layer
config-1 step."""
import numpy as np
import pytest

import g4synth as syn

pytestmark = pytest.mark.gpu


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(g4, shape, dtype):
    b = g4.DeviceBuffer.empty(shape, dtype)
    b.fill(0x7B)  # sentinel: an unwritten output cannot pass (registry.ts:89-98)
    return b


def f32_bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# (bits, K): one per compiled class (row chunks = K * bits / 128 = lanes per row * chunks per lane)
CLASS_SHAPES = [(4, 512), (4, 1024), (4, 1536), (4, 2048), (4, 3072), (4, 4096), (4, 6144),
                (4, 8192), (8, 256), (8, 512), (8, 768), (8, 1024), (8, 1536), (8, 2048),
                (8, 3072), (8, 4096), (8, 6144)]


@pytest.mark.parametrize("bits,k", CLASS_SHAPES)
def test_each_class_ragged_rows(gpu, oracle, bits, k):
    # 77 rows: not a multiple of any tile (16, 8 or 4 rows), so the clamped loads and the store
    # guard both run.
    n = 77
    print(f"stream class bits={bits} k={k} n={n}", flush=True)
    assert gpu.kernel_for_shape(bits, 1, n, k) == f"qgemv-{bits}bit-stream", \
        gpu.kernel_for_shape(bits, 1, n, k)
    w = syn.weights("stream", f"w{bits}.{k}", n, k, bits)
    s = syn.row_scales("stream", f"s{bits}.{k}", n)
    x = syn.activations("stream", f"x{k}", 1, k)[0]
    _, acc, codes = oracle.qgemv(bits, w, s, x.astype(np.float32), n, k, syn.IN_SCALE,
                                 syn.OUT_SCALE)
    out = out_buf(gpu, (n,), np.int8)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x), out, k, n, 1, syn.IN_SCALE,
              syn.OUT_SCALE)
    assert np.array_equal(out.download(), codes)
    acc_out = out_buf(gpu, (n,), np.int32)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, x), acc_out, k, n, 1, syn.IN_SCALE,
              syn.OUT_SCALE)
    assert np.array_equal(acc_out.download(), acc)


@pytest.mark.parametrize("x_kind", ["f16", "f32", "i8"])
@pytest.mark.parametrize("out_kind", ["i8", "f32", "i32"])
def test_activation_and_output_kinds(gpu, oracle, x_kind, out_kind):
    n, k, bits = 300, 1536, 4
    print(f"stream kinds x={x_kind} out={out_kind}", flush=True)
    w = syn.int4_weights("stream", "kinds.w", n, k)
    s = syn.row_scales("stream", "kinds.s", n)
    x16 = syn.activations("stream", "kinds.x", 1, k)[0]
    x32 = x16.astype(np.float32)
    y, acc, codes = oracle.qgemv(bits, w, s, x32, n, k, syn.IN_SCALE, syn.OUT_SCALE)
    xin = {"f16": x16, "f32": x32, "i8": oracle.srq_codes(x32, syn.IN_SCALE)}[x_kind]
    dt = {"i8": np.int8, "f32": np.float32, "i32": np.int32}[out_kind]
    out = out_buf(gpu, (n,), dt)
    gpu.qgemv(bits, dev(gpu, w), dev(gpu, s), dev(gpu, xin), out, k, n, 1, syn.IN_SCALE,
              syn.OUT_SCALE)
    got = out.download()
    if out_kind == "i8":
        assert np.array_equal(got, codes)
    elif out_kind == "i32":
        assert np.array_equal(got, acc)
    else:
        assert np.array_equal(f32_bits(got), f32_bits(y))


def test_output_snap_skipped_when_out_scale_zero(gpu, oracle):
    n, k = 64, 2048
    w = syn.int4_weights("stream", "noout.w", n, k)
    s = syn.row_scales("stream", "noout.s", n)
    x = syn.activations("stream", "noout.x", 1, k)[0].astype(np.float32)
    y, _, _ = oracle.qgemv(4, w, s, x, n, k, syn.IN_SCALE, 0.0)
    out = out_buf(gpu, (n,), np.float32)
    gpu.qgemv(4, dev(gpu, w), dev(gpu, s), dev(gpu, x), out, k, n, 1, syn.IN_SCALE, 0.0)
    assert np.array_equal(f32_bits(out.download()), f32_bits(y))


def test_outlier_saturation(gpu, oracle):
    # Activations at +-8 sigma saturate the 0.05 snap (8 / 0.05 = 160 > 127).
    n, k = 512, 1536
    w = syn.int4_weights("stream", "sat.w", n, k)
    s = syn.row_scales("stream", "sat.s", n)
    x = syn.activations("stream", "sat.x", 1, k, outlier_frac=0.05)[0]
    _, acc, codes = oracle.qgemv(4, w, s, x.astype(np.float32), n, k, syn.IN_SCALE, syn.OUT_SCALE)
    out = out_buf(gpu, (n,), np.int8)
    gpu.qgemv(4, dev(gpu, w), dev(gpu, s), dev(gpu, x), out, k, n, 1, syn.IN_SCALE, syn.OUT_SCALE)
    assert np.array_equal(out.download(), codes)


def _layer_items(g4, oracle, layer, down_bits=4, want=True):
    items, wants = [], []
    for name, n, k in syn.LAYER_PROJECTIONS:
        bits = down_bits if name == "down" else 4
        tag = f"{name}.L{layer}"
        w = syn.weights("bench", tag, n, k, bits)
        s = syn.row_scales("bench", tag, n)
        x = syn.activations("bench", tag, 1, k)[0]
        if want:
            wants.append(oracle.qgemv(bits, w, s, x.astype(np.float32), n, k, syn.IN_SCALE,
                                      syn.OUT_SCALE)[2])
        items.append(g4.Gemv(dev(g4, w), dev(g4, s), dev(g4, x), out_buf(g4, (n,), np.int8),
                             bits, k, n, syn.IN_SCALE, syn.OUT_SCALE))
    return items, wants


def test_plan_whole_step_35_layers(gpu, oracle):
    # The bench's workload: 35 layers x 7 projections in one plan (245 jobs, one launch). Layers
    # 0, 17 and 34 are checked against the oracle in full; every output is checked for the
    # sentinel (each row written exactly by its job).
    print("plan: 35-layer config-1 step", flush=True)
    all_items, checks = [], {}
    for layer in range(35):
        items, wants = _layer_items(gpu, oracle, layer, want=layer in (0, 17, 34))
        all_items.extend(items)
        if wants:
            checks[layer] = wants
    plan = gpu.GemvPlan(all_items)
    tiles, grid = plan.info()
    print(f"plan tiles {tiles} grid {grid}", flush=True)
    for _ in range(2):  # a replay reproduces the same bytes
        plan.launch()
        gpu.synchronize()
        for layer, wants in checks.items():
            for i, want in enumerate(wants):
                assert np.array_equal(all_items[layer * 7 + i].dst.download(), want), (layer, i)
    plan.close()


def test_plan_int8_down_and_graph_replay(gpu, oracle):
    items, wants = _layer_items(gpu, oracle, 3, down_bits=8)
    plan = gpu.GemvPlan(items)
    stream = gpu.Stream()
    graph = gpu.Graph(stream, lambda: plan.launch(stream.handle))
    for rep in range(3):
        for it in items:
            it.dst.fill(0x7B)
        gpu.synchronize()
        graph.launch()
        stream.synchronize()
        for it, want in zip(items, wants):
            assert np.array_equal(it.dst.download(), want), rep
    graph.close()
    plan.close()


def test_plan_refuses_unsupported_shapes(gpu):
    n, k = 16, 1280  # int4 K=1280: 40 chunks, no class
    items = [gpu.Gemv(dev(gpu, np.zeros((n, k // 2), np.uint8)), dev(gpu, np.ones(n, np.float32)),
                      dev(gpu, np.zeros(k, np.float16)), out_buf(gpu, (n,), np.int8), 4, k, n,
                      syn.IN_SCALE, syn.OUT_SCALE)]
    with pytest.raises(gpu.G4Error, match="no streaming shape class"):
        gpu.GemvPlan(items)
    uncal = [gpu.Gemv(items[0].wq, items[0].scales, items[0].x, items[0].dst, 4, 1536, 16, 0.0,
                      syn.OUT_SCALE)]
    with pytest.raises(gpu.G4Error):
        gpu.GemvPlan(uncal)
