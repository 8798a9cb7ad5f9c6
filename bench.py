"""Benchmark of the wNa8o8 projection path on one MI355X (prints one JSON line).

The step: BASELINE config 1 (one layer's q, k, v, o, gate, up and down projections; int4 weights,
f16 activations snapped on the static input scale 0.05, int32 accumulation, int8 outputs on 0.1)
for 35 layers with distinct seeded weights: 245 M = 1 GEMVs, 623.6 MB per step, more than twice the
256 MB Infinity Cache, so every step streams its weights from HBM. The step runs as one launch of
a device-resident GEMV plan (g4_qgemv_plan_launch: the streaming kernel over all 245 projections).
Inputs are resident in HBM before the timed region; the timed region is exactly `--steps` steps
between two HIP events on the launch stream, bracketed by device synchronizations.

Reported beside it (under "extra", not the headline):
  - the same 35 layers as one grouped launch per layer (7 projections per launch) and in the decode
    dependency shape (4 launches per layer: qkv batch, o, gate/up batch, down), which show what
    launch granularity costs;
  - config 0 (one 1536 x 1536 GEMV) as a single launch, warm and cold (512 rotated copies);
  - config 2's gate GEMM at M = 512 in int8 TOPS (MFMA), with and without the activation snap, and
    at every config-2 M with int8 and f16 input, M <= 128 also cold (a rotated 607 MB pool);
  - config 3's split PLE gather (5 slices, 2048 Zipf tokens, f16 out) in GB/s;
  - a measured HBM reference (a 1 GiB device-to-device copy) beside the 8 TB/s spec peak.

cpu_baseline: the oracle's C restatement (OpenMP over the host cores) on a bounded sample of the
same layer set, in the same unit. It is a baseline, not a target.

roofline.traffic: HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs
(`--traffic-probe` runs the same launches plus a plain device copy of known size that calibrates
the counters); the measured figure is read from profiles/traffic_qgemv_stream_config1.json when
that file exists, else null.
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_qgemv_stream_config1.json")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def proj_bytes(n, k, bits=4):
    """Algorithmic bytes of one M = 1 projection: weights + f32 scales + f16 x + int8 out."""
    return n * k * bits // 8 + 4 * n + 2 * k + n


def layer_bytes():
    return sum(proj_bytes(n, k) for _, n, k in syn.LAYER_PROJECTIONS)


def build_layers():
    """35 layers x 7 projections of seeded config-1 data, resident on the device."""
    layers = []
    for layer in range(LAYERS):
        items = {}
        for name, n, k in syn.LAYER_PROJECTIONS:
            tag = f"{name}.L{layer}"
            w = g4.DeviceBuffer.from_array(syn.int4_weights("bench", tag, n, k))
            s = g4.DeviceBuffer.from_array(syn.row_scales("bench", tag, n))
            x = g4.DeviceBuffer.from_array(syn.activations("bench", tag, 1, k)[0])
            d = g4.DeviceBuffer.empty((n,), np.int8)
            items[name] = g4.Gemv(w, s, x, d, 4, k, n, syn.IN_SCALE, syn.OUT_SCALE)
        layers.append(items)
    return layers


def timed(stream, fn, steps, warmup):
    """Average ms per call of fn() over `steps` calls between two events on `stream`."""
    for _ in range(warmup):
        fn()
    g4.synchronize()
    e0, e1 = g4.Event(), g4.Event()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    e1.synchronize()
    g4.synchronize()
    return e0.elapsed_ms(e1) / steps


def decode_shaped(layers, h):
    """The decode dependency shape: qkv batch, o, gate/up batch, down (4 launches per layer)."""
    def run():
        for L in layers:
            q, k_, v = L["q"], L["k"], L["v"]
            g4.projection_batch(4, [q.wq, k_.wq, v.wq], [q.scales, k_.scales, v.scales], q.x,
                                [q.dst, k_.dst, v.dst], [q.num_rows, k_.num_rows, v.num_rows],
                                [syn.IN_SCALE] * 3, [syn.OUT_SCALE] * 3, q.k, stream=h)
            g4.qgemv_grouped([L["o"]], h)
            gt, up = L["gate"], L["up"]
            g4.projection_batch(4, [gt.wq, up.wq], [gt.scales, up.scales], gt.x, [gt.dst, up.dst],
                                [gt.num_rows, up.num_rows], [syn.IN_SCALE] * 2,
                                [syn.OUT_SCALE] * 2, gt.k, stream=h)
            g4.qgemv_grouped([L["down"]], h)
    return run


def bench_gemm(h, m=512, reps=50):
    n, k = syn.FFN, syn.HIDDEN
    w = g4.DeviceBuffer.from_array(syn.int4_weights("c2", "gate", n, k))
    s = g4.DeviceBuffer.from_array(syn.row_scales("c2", "gate", n))
    xf = syn.activations("c2", f"x{m}", m, k, outlier_frac=0.01)
    x = g4.DeviceBuffer.from_array(xf)
    codes = g4.DeviceBuffer.empty((m, k), np.int8)
    g4.srq_quantize(x, codes, m * k, syn.IN_SCALE, stream=h)
    d = g4.DeviceBuffer.empty((m, n), np.int8)
    ops = 2.0 * m * n * k
    ms_f16 = timed(h, lambda: g4.qgemm(4, w, s, x, d, k, n, m, syn.IN_SCALE, syn.OUT_SCALE,
                                       stream=h), reps, 5)
    ms_i8 = timed(h, lambda: g4.qgemm(4, w, s, codes, d, k, n, m, syn.IN_SCALE, syn.OUT_SCALE,
                                      stream=h), reps, 5)
    return {"m": m, "n": n, "k": k, "kernel": g4.kernel_for_shape(4, m, n, k),
            "ms_f16_in": round(ms_f16, 6), "tops_f16_in": round(ops / (ms_f16 * 1e-3) / 1e12, 2),
            "ms_int8_in": round(ms_i8, 6), "tops_int8_in": round(ops / (ms_i8 * 1e-3) / 1e12, 2),
            "frac_int8_peak_int8_in": round(ops / (ms_i8 * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
            "note": "f16_in includes the activation snap; int8_in takes codes already snapped"}


POOL_BYTES = 512 << 20  # cold rows rotate weight copies totalling at least 2x the 256 MB MALL


def weight_pool(w_host, s_host, min_bytes=POOL_BYTES):
    """Copies of one weight matrix (and its scales) totalling at least `min_bytes`, so calls that
    rotate through them read their weights from HBM, not from the memory-side cache."""
    count = max(2, -(-min_bytes // w_host.nbytes))
    return [(g4.DeviceBuffer.from_array(w_host), g4.DeviceBuffer.from_array(s_host))
            for _ in range(count)]


def timed_pair(h, stream_obj, call, pool_len, reps):
    """Event-timed back-to-back calls (call(i) uses pool entry i) and the same calls captured as
    one graph and replayed: returns (us per call, us per call from a graph)."""
    i = [0]

    def one():
        call(i[0] % pool_len)
        i[0] += 1
    ms = timed(h, one, max(reps, pool_len), 3)
    per = pool_len if pool_len > 1 else 20
    graph = g4.Graph(stream_obj, lambda: [call(j % pool_len) for j in range(per)])
    ms_g = timed(h, graph.launch, max(2, reps // per), 2) / per
    graph.close()
    return ms * 1e3, ms_g * 1e3


def bench_gemm_sweep(h, stream_obj, ms=(4, 8, 16, 128, 512, 2048), reps=30):
    """Config 2: the gate projection (K=1536, N=6144, int4) at every BASELINE M. Each row gives
    the kernel that served it, with int8 codes in and with f16 activations in (the snap included),
    timed back to back and replayed from a graph. "warm" repeats one weight buffer (served from the
    256 MB memory-side cache after the first call); "cold" (M <= 128, where the weights are the
    bytes) rotates through a 607 MB pool of weight copies, so every call reads HBM. Bytes are
    weights + scales + x (1 B int8 or 2 B f16 per code) + int8 out."""
    n, k = syn.FFN, syn.HIDDEN
    w_host = syn.int4_weights("c2", "gate", n, k)
    s_host = syn.row_scales("c2", "gate", n)
    pool = weight_pool(w_host, s_host)
    rows = []
    for m in ms:
        xh = syn.activations("c2", f"x{m}", m, k, outlier_frac=0.01)
        x = g4.DeviceBuffer.from_array(xh)
        codes = g4.DeviceBuffer.empty((m, k), np.int8)
        g4.srq_quantize(x, codes, m * k, syn.IN_SCALE, stream=h)
        d = g4.DeviceBuffer.empty((m, n), np.int8)
        row = {"m": m, "kernel": g4.kernel_for_shape(4, m, n, k)}
        ops = 2.0 * m * n * k
        for src, xb, tag in ((codes, 1, "int8_in"), (x, 2, "f16_in")):
            by = n * k // 2 + 4 * n + xb * m * k + m * n
            temps = (("warm", 1), ("cold", len(pool))) if m <= 128 else (("warm", 1),)
            for temp, plen in temps:
                call = (lambda j, src=src: g4.qgemm(4, pool[j][0], pool[j][1], src, d, k, n, m,
                                                    syn.IN_SCALE, syn.OUT_SCALE, stream=h))
                us, us_g = timed_pair(h, stream_obj, call, plen, reps)
                key = f"{tag}_{temp}"
                row[key] = {"us": round(us, 3), "us_graph": round(us_g, 3),
                            "tops": round(ops / (us * 1e-6) / 1e12, 2),
                            "gbs": round(by / (us * 1e-6) / 1e9, 2),
                            "gbs_graph": round(by / (us_g * 1e-6) / 1e9, 2)}
        # the headline keys of earlier rounds: int8 in, warm, back to back
        row.update({"us": row["int8_in_warm"]["us"], "tops": row["int8_in_warm"]["tops"],
                    "us_graph": row["int8_in_warm"]["us_graph"]})
        rows.append(row)
    for wb, sb in pool:
        wb.close()
        sb.close()
    return rows


def bench_int8_down(h, stream_obj, reps=64):
    """Config 1's int8-weight variant of down (6144 -> 1536, I8 codes U[-127,127]) at M=1, warm
    (one weight buffer) and cold (a 604 MB pool of copies, rotated)."""
    n, k = syn.HIDDEN, syn.FFN
    pool = weight_pool(syn.int8_weights("c1", "down8", n, k), syn.row_scales("c1", "down8", n))
    x = g4.DeviceBuffer.from_array(syn.activations("c1", "down8", 1, k)[0])
    d = g4.DeviceBuffer.empty((n,), np.int8)
    out = {"n": n, "k": k, "kernel": g4.kernel_for_shape(8, 1, n, k), "pool_copies": len(pool)}
    for temp, plen in (("warm", 1), ("cold", len(pool))):
        call = lambda j: g4.qgemv(8, pool[j][0], pool[j][1], x, d, k, n, 1, syn.IN_SCALE,
                                  syn.OUT_SCALE, stream=h)
        us, us_g = timed_pair(h, stream_obj, call, plen, reps)
        out[temp] = {"us": round(us, 3), "gbs": round(proj_bytes(n, k, 8) / (us * 1e-6) / 1e9, 2),
                     "us_graph": round(us_g, 3),
                     "gbs_graph": round(proj_bytes(n, k, 8) / (us_g * 1e-6) / 1e9, 2)}
    for wb, sb in pool:
        wb.close()
        sb.close()
    out.update({"us": out["warm"]["us"], "gbs": out["warm"]["gbs"]})
    return out


def bench_config0(h, stream_obj, reps=512):
    """Config 0 (one 1536 x 1536 int4 GEMV) as a single launch, warm (one weight buffer, the
    memory-side cache serves it) and cold (512 copies, 609 MB, rotated)."""
    n = k = 1536
    pool = weight_pool(syn.int4_weights("c0", "w", n, k), syn.row_scales("c0", "w", n))
    x = g4.DeviceBuffer.from_array(syn.activations("c0", "x", 1, k)[0])
    d = g4.DeviceBuffer.empty((n,), np.int8)
    by = proj_bytes(n, k)
    out = {"bytes": by, "kernel": g4.kernel_for_shape(4, 1, n, k), "pool_copies": len(pool)}
    for temp, plen in (("warm", 1), ("cold", len(pool))):
        call = lambda j: g4.qgemv(4, pool[j][0], pool[j][1], x, d, k, n, 1, syn.IN_SCALE,
                                  syn.OUT_SCALE, stream=h)
        us, us_g = timed_pair(h, stream_obj, call, plen, reps)
        out[temp] = {"us": round(us, 3), "gbs": round(by / (us * 1e-6) / 1e9, 2),
                     "us_graph": round(us_g, 3), "gbs_graph": round(by / (us_g * 1e-6) / 1e9, 2)}
    for wb, sb in pool:
        wb.close()
        sb.close()
    out.update({"us": out["warm"]["us"], "gbs": out["warm"]["gbs"]})
    return out


def bench_tile8u(h, stream_obj, reps=64):
    """qgemv-4bit's tile8u geometry (qgemv.ts:870-1015) beside the classic routing, on config 1's
    gate (6144 x 1536) and down (1536 x 6144) shapes, f32 activations, calibrated, int8 out: each
    warm (one weight buffer) and graph-replayed. Bytes as the classic row: weights + scales + x
    (f32 here) + out."""
    rows = []
    for name, n, k in (("gate", syn.FFN, syn.HIDDEN), ("down", syn.HIDDEN, syn.FFN)):
        w = g4.DeviceBuffer.from_array(syn.int4_weights("t8b", name, n, k))
        s = g4.DeviceBuffer.from_array(syn.row_scales("t8b", name, n))
        tw = g4.DeviceBuffer(g4.tile8u_bytes(k, n), np.uint32)
        g4.tile8u_repack(w, tw, k, n, stream=h)
        x = g4.DeviceBuffer.from_array(syn.activations("t8b", name, 1, k)[0].astype(np.float32))
        d = g4.DeviceBuffer.empty((n,), np.int8)
        by = n * k // 2 + 4 * n + 4 * k + n
        row = {"shape": name, "n": n, "k": k, "bytes": by}
        for form, call in (
                ("classic", lambda j: g4.qgemv(4, w, s, x, d, k, n, 1, syn.IN_SCALE, syn.OUT_SCALE,
                                               stream=h)),
                ("tile8u", lambda j: g4.qgemv_tile8u(tw, s, x, d, k, n, syn.IN_SCALE, syn.OUT_SCALE,
                                                     stream=h))):
            us, us_g = timed_pair(h, stream_obj, call, 1, reps)
            row[form] = {"us": round(us, 3), "us_graph": round(us_g, 3),
                         "gbs_graph": round(by / (us_g * 1e-6) / 1e9, 2)}
        row["classic_kernel"] = g4.kernel_for_shape(4, 1, n, k)
        rows.append(row)
        for b in (w, s, tw, x, d):
            b.close()
    return rows


def cpu_extra(seconds=4.0):
    """The oracle on the host cores for the other rows (bounded samples): the config-2 GEMM at
    M=16 and the config-3 gather at 64 tokens."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # the checker's C restatement, used here only as the timed CPU baseline

    n, k, m = syn.FFN, syn.HIDDEN, 16
    w = syn.int4_weights("c2", "gate", n, k)
    s = syn.row_scales("c2", "gate", n)
    x = syn.activations("c2", f"x{m}", m, k, outlier_frac=0.01).astype(np.float32)
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.qgemm(4, w, s, x, n, k, m, syn.IN_SCALE, syn.OUT_SCALE)
        done += 1
    el = time.perf_counter() - t0
    gemm = {"tops": round(2.0 * m * n * k * done / el / 1e12, 4), "sample": f"{done} x M=16 gate GEMM, {el:.1f} s"}
    rows, cols, tokens = 4096, syn.PLE_COLS, 64
    codes = syn.ple_codes("c3cpu", rows)
    scales = syn.ple_scales("c3cpu", rows)
    ids = (syn.zipf_ids("c3", tokens) % rows).astype(np.int32)
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.embed_gather(codes, scales, ids, cols, 256, out_kind="f16")
        done += 1
    el = time.perf_counter() - t0
    per_token = cols // 2 + 2 * (cols // 256) + 4 + 2 * cols
    gather = {"gbs": round(per_token * tokens * done / el / 1e9, 3),
              "sample": f"{done} x 64-token gather over a 4096-row table, {el:.1f} s"}
    return {"cores": oracle.num_threads(), "kind": "port", "gemm_m16": gemm, "ple_gather": gather}


def bench_gather(h, stream_obj=None, tokens=2048, reps=20):
    """Config 3: the split PLE gather of `tokens` Zipf ids over the 5-slice table, f16 out. `ms`
    is event-timed over calls issued one by one from Python; with a stream object, `ms_graph` is
    the same call captured 20 times into one graph and replayed (launches back to back, no host
    gap between them), and the GB/s figures follow it."""
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
    def call(_=0):
        g4.ple_gather_split(bufs, starts, counts, scales, ids, out, tokens, cols, 256, h)
    ms = timed(h, call, reps, 3)
    per_token = cols // 2 + 2 * (cols // 256) + 4 + 2 * cols  # codes + f16 scales + id + f16 out
    r = {"tokens": tokens, "slices": len(slices), "ms": round(ms, 6)}
    if stream_obj is not None:
        _, us_g = timed_pair(h, stream_obj, call, 1, reps)
        r["ms_graph"] = round(us_g * 1e-3, 6)
        ms = us_g * 1e-3
    r["gbs"] = round(per_token * tokens / (ms * 1e-3) / 1e9, 2)
    r["frac_hbm_peak"] = round(per_token * tokens / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    return r


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


def traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t.get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def traffic_probe(plan, h):
    """Launches for the rocprofv3 --pmc runs: 3 copies of 256 MiB (the counter calibration: a
    plain copy reads and writes exactly that many bytes), then 5 plan launches."""
    n = 256 << 20
    a = g4.DeviceBuffer(n)
    b = g4.DeviceBuffer(n)
    a.fill(1)
    g4.synchronize()
    for _ in range(3):
        g4._check(g4.lib().g4_memcpy_d2d(g4._ptr(b), g4._ptr(a), n, h))
    g4.synchronize()
    for _ in range(5):
        plan.launch(h)
    g4.synchronize()
    log(f"traffic probe done: copy {n} B x3, plan x5")


def hbm_copy_rate(h, nbytes=1 << 30, reps=20):
    """A measured reference for the HBM peak: a device-to-device copy of 1 GiB (the runtime's copy,
    reading and writing every byte once, far past the 256 MB Infinity Cache); the rate counts
    both directions."""
    a = g4.DeviceBuffer(nbytes)
    b = g4.DeviceBuffer(nbytes)
    a.fill(1)
    g4.synchronize()
    ms = timed(h, lambda: g4._check(g4.lib().g4_memcpy_d2d(g4._ptr(b), g4._ptr(a), nbytes, h)),
               reps, 3)
    gbs = 2 * nbytes / (ms * 1e-3) / 1e9
    a.close()
    b.close()
    return {"bytes_moved": 2 * nbytes, "ms": round(ms, 4), "gbs": round(gbs, 1),
            "frac_of_spec": round(gbs / HBM_PEAK_GBS, 4),
            "note": "hipMemcpyAsync device to device, 1 GiB read + 1 GiB written"}


def decode_step_bytes(shape, pos):
    """Algorithmic HBM bytes of one E2B-shape decode step at `pos` for `batch` rows: every weight
    byte and row scale the step reads once (35 layers of q/k/v/o/gate/up/down int4 and the int8
    per-layer gate and projection, the per-layer model projection, the tied head), plus per row
    the KV each layer's attention reads (f32 K and V over its window) and writes (producers), the
    PLE row (4480 B of codes + 35 f32 scales) and the embedding row. Activations between kernels
    (a few KB per row per layer) are not counted."""
    s = shape
    H, F, QW, P, hd = s.hidden, s.ffn, s.q_heads * s.head_dim, s.ple_dim, s.head_dim

    def lin(n, k, bits):
        return n * k * bits // 8 + 4 * n

    w = 0
    for l in range(s.layers):
        prod = l < s.kv_producers
        w += lin(QW, H, 4) + lin(H, QW, 4) + 2 * lin(F, H, 4) + lin(H, F, 4)
        w += lin(P, H, 8) + lin(H, P, 8)
        if prod:
            w += 2 * lin(hd, H, 4)
    w += lin(s.layers * P, H, 4) + lin(s.vocab, H, 4)
    per_row = 0
    for l in range(s.layers):
        span = pos + 1 if s.is_global(l) else min(pos + 1, s.sliding_window)
        per_row += span * hd * 4 * 2
        if l < s.kv_producers:
            per_row += hd * 4 * 2
    per_row += s.layers * P // 2 + 4 * s.layers + H // 2 + 4 + 4 * s.vocab  # PLE row, embed row, logits
    return w + s.batch * per_row


def cpu_decode_step(shape, model, dec, pos, tokens):
    """The CPU composition of one decode step (oracle/decode_ref.py, C oracle kernels with OpenMP
    over the host cores) on the same model, KV and tokens: the weights are copied to the host
    before the timed region."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import decode_ref as ref
    import oracle as o
    W = ref.Weights(model)
    for name in model.buffers:
        if name != "ple_table":
            W[name]
    kv = {p: tuple(a.copy() for a in dec.download_kv(p)) for p in range(shape.kv_producers)}
    t0 = time.perf_counter()
    out = ref.step(shape, W, kv, list(tokens), pos)
    secs = time.perf_counter() - t0
    return {"value": round(len(tokens) / secs, 3), "unit": "tok/s", "cores": o.num_threads(),
            "kind": "port", "sample": f"one decode step at batch {len(tokens)} (position {pos})",
            "seconds": round(secs, 3), "next_tokens": [int(t) for t in out["next"]]}


def bench_decode(h, batch, steps=20, warmup=3, probe=False, cpu=False):
    """one E2B-shape decode step (35 layers, KV capacity 4096, position 4095, so
    global layers attend over 4096 positions and sliding ones over 512), greedy over 262144 rows,
    as one captured graph replayed per token; and the same step launched eagerly."""
    import g4decode as gd
    shape = gd.Shape(batch=batch, kv_capacity=4096)
    model = gd.SyntheticModel(shape, seed=4, stream=h)
    dec = gd.Decoder(shape, model)
    dec.fill_kv_history(stream=h)
    pos = shape.kv_capacity - 1
    dec.set_position(pos)
    toks = g4.DeviceBuffer.from_array(np.arange(batch, dtype=np.int32) * 7919 % shape.vocab)
    nxt = g4.DeviceBuffer.empty((batch,), np.int32)
    g4.synchronize()
    stream = g4.Stream()
    sh = stream.handle
    dec.step(toks, nxt, sh)
    stream.synchronize()
    graph = g4.Graph(stream, lambda: dec.step(toks, nxt, sh))
    if probe:
        for _ in range(steps):
            graph.launch()
        stream.synchronize()
        log(f"decode probe batch {batch}: {steps} graph replays")
        graph.close()
        dec.close()
        return None
    ms_graph = timed(sh, graph.launch, steps, warmup)
    ms_eager = timed(sh, lambda: dec.step(toks, nxt, sh), max(3, steps // 4), 1)
    nb = decode_step_bytes(shape, pos)
    out = {
        "batch": batch, "kv_positions": pos + 1, "ms_per_step_graph": round(ms_graph, 4),
        "tok_per_s": round(batch / (ms_graph * 1e-3), 1),
        "ms_per_step_eager": round(ms_eager, 4), "bytes_per_step": nb,
        "gbs": round(nb / (ms_graph * 1e-3) / 1e9, 1),
        "pct_hbm_peak": round(100 * nb / (ms_graph * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
        "next_tokens_head": [int(t) for t in nxt.download()[:4]],
        "model_bytes": model.nbytes(),
    }
    if cpu:
        log(f"config 4 CPU composition, batch {batch}")
        toks_host = [int(t) for t in toks.download()]
        dec.fill_kv_history()  # the timed replays rewrote the position's rows; restore the history
        g4.synchronize()
        c = cpu_decode_step(shape, model, dec, pos, toks_host)
        c["matches_gpu_next_tokens"] = c["next_tokens"] == out["next_tokens_head"][:batch]
        out["cpu"] = c
    graph.close()
    dec.close()
    stream.close()
    return out


def gemm_probe(h):
    """Launches for rocprofv3 --kernel-trace --stats: the config-2 gate GEMM 50 times at M=4, 8,
    16, 128 and 512 and 20 times at M=2048, first with f16 activations (above M=32: the activation
    snap + the tile kernel; up to 32 the small kernel snaps itself), then with int8 codes already
    snapped (one kernel)."""
    n, k = syn.FFN, syn.HIDDEN
    w = g4.DeviceBuffer.from_array(syn.int4_weights("c2", "gate", n, k))
    s = g4.DeviceBuffer.from_array(syn.row_scales("c2", "gate", n))
    for m, reps in ((4, 50), (8, 50), (16, 50), (128, 50), (512, 50), (2048, 20)):
        x = g4.DeviceBuffer.from_array(syn.activations("c2", f"x{m}", m, k, outlier_frac=0.01))
        codes = g4.DeviceBuffer.empty((m, k), np.int8)
        g4.srq_quantize(x, codes, m * k, syn.IN_SCALE, stream=h)
        d = g4.DeviceBuffer.empty((m, n), np.int8)
        for src, name in ((x, "f16"), (codes, "int8")):
            for _ in range(reps):
                g4.qgemm(4, w, s, src, d, k, n, m, syn.IN_SCALE, syn.OUT_SCALE, stream=h)
            g4.synchronize()
            log(f"gemm probe M={m} {name} in: {reps} launches")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only the config-2 GEMM launches (M=4..2048, f16 then int8 in), for rocprofv3")
    ap.add_argument("--decode-probe", type=int, default=0, metavar="BATCH",
                    help="only config-4 decode steps at this batch (graph replays), for rocprofv3")
    ap.add_argument("--gather-probe", action="store_true",
                    help="only the config-3 gather launches (2048 tokens, 5 slices), for rocprofv3")
    ap.add_argument("--tile8u-probe", action="store_true",
                    help="only the tile8u and classic GEMV launches on config 1's gate and down")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this path is measured on one GPU; --gpus {args.gpus} is not supported "
              "(how the path would shard is a design note only)", file=sys.stderr)
        sys.exit(2)
    if g4.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    g4.lib().g4_set_device(0)
    stream = g4.Stream()
    h = stream.handle
    if args.gemm_probe:
        gemm_probe(h)
        return
    if args.tile8u_probe:
        print(json.dumps(bench_tile8u(h, stream)))
        return
    if args.decode_probe:
        bench_decode(h, args.decode_probe, steps=10, probe=True)
        return
    if args.gather_probe:
        r = bench_gather(h, stream, reps=50)
        log(f"gather probe: {r['ms'] * 1e3:.2f} us per call issued from Python, "
            f"{r['ms_graph'] * 1e3:.2f} us graph-replayed")
        return
    log("building 35 layers of config-1 weights (623.6 MB)")
    layers = build_layers()
    items = [L[name] for L in layers for name, _, _ in syn.LAYER_PROJECTIONS]
    plan = g4.GemvPlan(items)
    tiles, grid = plan.info()
    if args.traffic_probe:
        traffic_probe(plan, h)
        return
    log(f"timing the plan ({len(items)} projections, {tiles} tiles, {grid} blocks)")
    ms = timed(h, lambda: plan.launch(h), args.steps, args.warmup)
    t_wall = time.perf_counter()
    step_bytes = layer_bytes() * LAYERS
    value = step_bytes / (ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded int4 weights U[-8,7], f32 scales U(0.005,0.02), f16 N(0,1) x)",
        "config": {
            "workload": "config1 decode projection set at M=1 (q 1536->2048, k/v 1536->256, "
                        "o 2048->1536, gate/up 1536->6144, down 6144->1536), int4 weights x int8 "
                        "activation codes, int32 accumulate, int8 out; 35 distinct layers per step "
                        "(245 GEMVs) as one streaming-plan launch",
            "bytes_per_step": step_bytes,
            "launches_per_step": 1,
            "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "qgemv_stream_kernel<true, 0> (plan launch, 245 projections)",
            "achieved": round(value, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": traffic(),
            "bytes_per_launch": step_bytes,
            "avg_launch_ms": round(ms, 6),
            "plan_tiles": tiles,
            "plan_blocks": grid,
        },
    }
    if not args.no_extra:
        log("per-layer grouped launches")
        groups = [g4.make_group([L[name] for name, _, _ in syn.LAYER_PROJECTIONS]) for L in layers]
        ms_layer = timed(h, lambda: [g4.qgemv_grouped(a, h) for a in groups], 20, 3)
        log("decode-shaped launches")
        ms_dec = timed(h, decode_shaped(layers, h), 20, 3)
        log("config 0 single GEMV, warm and cold")
        c0 = bench_config0(h, stream)
        log("config 2 gate GEMM at M=512")
        gm = bench_gemm(h)
        log("config 3 split PLE gather")
        ga = bench_gather(h, stream)
        log("config 2 sweep over M, config 1 int8 down")
        sweep = bench_gemm_sweep(h, stream)
        down8 = bench_int8_down(h, stream)
        log("qgemv-4bit tile8u geometry beside the classic loop")
        t8 = bench_tile8u(h, stream)
        log("measured HBM copy rate")
        hbm = hbm_copy_rate(h)
        log("config 4 decode step, batch 1 and 32")
        dec1 = bench_decode(h, 1, cpu=not args.no_cpu_baseline)
        dec32 = bench_decode(h, 32)
        result["extra"] = {
            "decode_step_config4": {"batch1": dec1, "batch32": dec32},
            "per_layer_grouped": {"launches_per_step": LAYERS, "ms_per_step": round(ms_layer, 6),
                                  "gbs": round(step_bytes / (ms_layer * 1e-3) / 1e9, 2)},
            "decode_shaped": {"launches_per_step": 4 * LAYERS, "ms_per_step": round(ms_dec, 6),
                              "gbs": round(step_bytes / (ms_dec * 1e-3) / 1e9, 2)},
            "config0_single_gemv": c0,
            "int8_gemm_m512": gm,
            "gemm_sweep_config2": sweep,
            "config1_int8_down": down8,
            "tile8u_config1": t8,
            "ple_gather": ga,
            "hbm_measured": hbm,
        }
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle on host cores)")
        result["cpu_baseline"] = cpu_baseline()
        if not args.no_extra:
            result.setdefault("extra", {})["cpu_other_rows"] = cpu_extra()
    result["config"]["wall_s_after_timing"] = round(time.perf_counter() - t_wall, 3)
    plan.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
