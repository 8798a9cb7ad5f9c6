"""Benchmark of the wNa8o8 projection path on one MI355X (prints one JSON line).

The step: one E2B-shape decode projection stream at M = 1, i.e. BASELINE config 1 (a layer's
q, k, v, o, gate, up and down projections; int4 weights, f16 activations snapped on the static
input scale 0.05, int32 accumulation, int8 outputs on 0.1) for 35 layers with distinct seeded
weights (623.6 MB per step, more than twice the 256 MB Infinity Cache), one grouped GEMV launch per
layer. Inputs are resident in HBM before the timed region; the timed region is exactly `--steps`
steps between two HIP events on the launch stream, bracketed by device synchronizations.

Also reported (fields under "extra"): config 2's gate GEMM at M = 512 in int8 TOPS (MFMA), and
config 3's split PLE gather (5 slices, 2048 Zipf tokens, f16 out) in GB/s.

cpu_baseline: the oracle's C restatement (OpenMP over the host cores) timed on a bounded sample of
the same layer set, reported in the same unit. It is a baseline, not a target.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "gemma4-webgpu-engine_amd")
sys.path.insert(0, PKG)

import g4synth as syn  # noqa: E402
import g4w8a8 as g4  # noqa: E402

METRIC = "wNa8o8 GEMV GB/s (% HBM peak) M=1; int8 TOPS M=512; E2B-shape decode tok/s"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
LAYERS = 35


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_bytes():
    """Algorithmic bytes of one config-1 layer: N*K/2 weights + 4N scales + 2K f16 x + N int8."""
    return sum(n * k // 2 + 4 * n + 2 * k + n for _, n, k in syn.LAYER_PROJECTIONS)


def build_layers(stream):
    layers = []
    for layer in range(LAYERS):
        items = []
        for name, n, k in syn.LAYER_PROJECTIONS:
            tag = f"{name}.L{layer}"
            w = g4.DeviceBuffer.from_array(syn.int4_weights("bench", tag, n, k))
            s = g4.DeviceBuffer.from_array(syn.row_scales("bench", tag, n))
            x = g4.DeviceBuffer.from_array(syn.activations("bench", tag, 1, k)[0])
            d = g4.DeviceBuffer.empty((n,), np.int8)
            items.append(g4.Gemv(w, s, x, d, 4, k, n, syn.IN_SCALE, syn.OUT_SCALE))
        layers.append((items, g4.make_group(items)))
    return layers


def time_layers(layers, stream, steps, warmup):
    for _ in range(warmup):
        for _, arr in layers:
            g4.qgemv_grouped(arr, stream)
    g4.synchronize()
    e0, e1 = g4.Event(), g4.Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        for _, arr in layers:
            g4.qgemv_grouped(arr, stream)
    e1.record(stream)
    e1.synchronize()
    g4.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_ms(e1) / steps, wall


def per_launch_ms(layers, stream, reps=3):
    """Average duration of one grouped layer launch, each bracketed by its own event pair."""
    evs = [(g4.Event(), g4.Event()) for _ in layers]
    total, count = 0.0, 0
    for _ in range(reps):
        for (a, b), (_, arr) in zip(evs, layers):
            a.record(stream)
            g4.qgemv_grouped(arr, stream)
            b.record(stream)
        g4.synchronize()
        for a, b in evs:
            total += a.elapsed_ms(b)
            count += 1
    return total / count


def bench_gemm(stream, m=512, reps=50):
    n, k = syn.FFN, syn.HIDDEN
    w = g4.DeviceBuffer.from_array(syn.int4_weights("c2", "gate", n, k))
    s = g4.DeviceBuffer.from_array(syn.row_scales("c2", "gate", n))
    x = g4.DeviceBuffer.from_array(syn.activations("c2", f"x{m}", m, k, outlier_frac=0.01))
    d = g4.DeviceBuffer.empty((m, n), np.int8)
    for _ in range(5):
        g4.qgemm(4, w, s, x, d, k, n, m, syn.IN_SCALE, syn.OUT_SCALE, stream=stream)
    g4.synchronize()
    e0, e1 = g4.Event(), g4.Event()
    e0.record(stream)
    for _ in range(reps):
        g4.qgemm(4, w, s, x, d, k, n, m, syn.IN_SCALE, syn.OUT_SCALE, stream=stream)
    e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    return {"m": m, "n": n, "k": k, "ms": ms, "tops": 2.0 * m * n * k / (ms * 1e-3) / 1e12,
            "kernel": g4.kernel_for_shape(4, m, n, k), "includes": "activation snap + MFMA GEMM"}


def bench_gather(stream, tokens=2048, reps=20):
    rows, cols = syn.PLE_ROWS, syn.PLE_COLS
    codes = syn.ple_codes("c3", rows)
    scales = g4.DeviceBuffer.from_array(syn.ple_scales("c3", rows))
    plan, slices = g4.plan_table_split(rows, cols // 2, 1 << 30, 1 << 30, 10, 0)
    bufs = [g4.DeviceBuffer.from_array(codes[s.start_row:s.start_row + s.row_count])
            for s in slices]
    del codes
    ids = g4.DeviceBuffer.from_array(syn.zipf_ids("c3", tokens))
    out = g4.DeviceBuffer.empty((tokens, cols), np.float16)
    starts = [s.start_row for s in slices]
    counts = [s.row_count for s in slices]
    for _ in range(3):
        g4.ple_gather_split(bufs, starts, counts, scales, ids, out, tokens, cols, 256, stream)
    g4.synchronize()
    e0, e1 = g4.Event(), g4.Event()
    e0.record(stream)
    for _ in range(reps):
        g4.ple_gather_split(bufs, starts, counts, scales, ids, out, tokens, cols, 256, stream)
    e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    per_token = cols // 2 + 2 * (cols // 256) + 4 + 2 * cols  # codes + f16 scales + id + f16 out
    return {"tokens": tokens, "slices": len(slices), "ms": ms,
            "gbs": per_token * tokens / (ms * 1e-3) / 1e9}


def cpu_baseline(seconds=10.0):
    """The oracle (C, OpenMP) on the host cores over the config-1 layer set, in GB/s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # the checker's C restatement, used here only as the timed CPU baseline

    projs = []
    for name, n, k in syn.LAYER_PROJECTIONS:
        projs.append((n, k, syn.int4_weights("bench", f"{name}.L0", n, k),
                      syn.row_scales("bench", f"{name}.L0", n),
                      syn.activations("bench", f"{name}.L0", 1, k)[0].astype(np.float32)))
    done, t0 = 0, time.perf_counter()
    while True:
        for n, k, w, s, x in projs:
            oracle.qgemv(4, w, s, x, n, k, syn.IN_SCALE, syn.OUT_SCALE)
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(layer_bytes() * done / el / 1e9, 3), "unit": "GB/s",
            "cores": oracle.num_threads(), "kind": "port",
            "sample": f"{done} passes of the config-1 layer set (7 projections, int4, M=1) through "
                      f"the C oracle, {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this path is measured on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)
    if g4.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    g4.lib().g4_set_device(0)
    stream = g4.Stream()
    h = stream.handle
    log("building 35 layers of config-1 weights (623.6 MB)")
    layers = build_layers(h)
    log("timing")
    ms, wall = time_layers(layers, h, args.steps, args.warmup)
    step_bytes = layer_bytes() * LAYERS
    value = step_bytes / (ms * 1e-3) / 1e9
    launch_ms = per_launch_ms(layers, h)
    achieved = layer_bytes() / (launch_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded int4 weights U[-8,7], f32 scales U(0.005,0.02), f16 N(0,1) x)",
        "config": {
            "workload": "config1 decode projection set at M=1 (q 1536->2048, k/v 1536->256, "
                        "o 2048->1536, gate/up 1536->6144, down 6144->1536), int4 weights x int8 "
                        "activation codes, int32 accumulate, int8 out; 35 distinct layers per step, "
                        "one grouped GEMV launch per layer",
            "bytes_per_step": step_bytes,
            "launches_per_step": LAYERS,
            "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
            "wall_s": round(wall, 3),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "qgemv_int_kernel<1> (grouped layer GEMV)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_launch": layer_bytes(),
            "avg_launch_ms": round(launch_ms, 6),
        },
    }
    if not args.no_extra:
        log("config 2 gate GEMM at M=512")
        gm = bench_gemm(h)
        gm["frac_int8_peak"] = round(gm["tops"] / INT8_PEAK_TOPS, 4)
        log("config 3 split PLE gather")
        ga = bench_gather(h)
        ga["frac_hbm_peak"] = round(ga["gbs"] / HBM_PEAK_GBS, 4)
        result["extra"] = {"int8_gemm_m512": gm, "ple_gather": ga}
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle on host cores)")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
