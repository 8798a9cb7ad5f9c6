"""GPU parity of the decode-step glue kernels and of the native decode step (include/g4decode.h)
against the CPU restatement (oracle/g4_decode_oracle.c, oracle/decode_ref.py): bit-exact on every
f32, int8 and index output. Every kernel runs the fixed reduction order the oracle states, so the
contract is identity, not a tolerance; the oracle itself is held to the reference's f64 oracles
within their stated tolerances in tests/test_oracle_decode.py."""
import ctypes

import numpy as np
import pytest

import decode_oracle as d

pytestmark = pytest.mark.gpu

IN, OUT, EPS = float(np.float32(0.05)), float(np.float32(0.1)), 1e-6


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(g4, shape, dtype):
    b = g4.DeviceBuffer.empty(shape, dtype)
    b.fill(0x7B)
    return b


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        return a.shape == b.shape and np.array_equal(a.view(np.uint32), np.asarray(b, np.float32).view(np.uint32))
    return np.array_equal(a, b)


def test_fill_hash_matches_numpy(gpu):
    import g4decode as gd
    n = 100003
    b = gpu.DeviceBuffer.empty((n,), np.float32)
    gpu._check(gpu.lib().g4_fill_hash_f32(b.ptr, n, 12345, -1.7, 1.7, None))
    assert same(b.download(), gd.hash_f32(n, 12345, -1.7, 1.7))
    u = gpu.DeviceBuffer.empty((n,), np.uint8)
    gpu._check(gpu.lib().g4_fill_hash_u8(u.ptr, n, 777, None))
    assert same(u.download(), gd.hash_u8(n, 777))


@pytest.mark.parametrize("width", [1536, 256, 2048, 640])
def test_rms_join_forms(gpu, width):
    print(f"rms_join width={width}", flush=True)
    L = gpu.lib()
    rng = np.random.default_rng(width)
    rows = 3
    x = rng.standard_normal((rows, width)).astype(np.float32) * np.float32(2.0)
    codes_src = rng.integers(-128, 128, (rows, width)).astype(np.int8)
    resid = rng.standard_normal((rows, width)).astype(np.float32)
    gain = rng.uniform(0.5, 1.5, width).astype(np.float32)
    gain2 = rng.uniform(-2, 2, width).astype(np.float32)
    dx, dcodes_src, dresid = dev(gpu, x), dev(gpu, codes_src), dev(gpu, resid)
    dgain, dgain2 = dev(gpu, gain), dev(gpu, gain2)
    hid = out_buf(gpu, (rows, width), np.float32)
    cod = out_buf(gpu, (rows, width), np.int8)
    # rms-norm with the consumer's snap, weighted and weightless
    for g_host, g_dev in ((gain, dgain.ptr), (None, None)):
        gpu._check(L.g4_rms_join(dx.ptr, gpu.KIND_F32, 1.0, g_dev, None, 1.0, None, rows, width, EPS,
                                 IN, hid.ptr, cod.ptr, None))
        assert same(hid.download(), d.rms_norm(x, g_host, EPS))
        assert same(cod.download(), d.rms_norm_codes(x, g_host, EPS, IN))
    # norm-residual from a projection's int8 output, snapped for the next linear
    src = codes_src.astype(np.float32) * np.float32(OUT)
    gpu._check(L.g4_rms_join(dcodes_src.ptr, gpu.KIND_I8, OUT, dgain.ptr, dresid.ptr, 1.0, None,
                             rows, width, EPS, IN, hid.ptr, cod.ptr, None))
    want = d.norm_residual(src, gain, resid, EPS)
    assert same(hid.download(), want)
    assert same(cod.download(), np.stack([o_codes(r) for r in want]))
    # norm-residual-norm with a layer scalar, in place on the residual
    for alpha in (1.0, 0.3671875, 0.77):
        dres2 = dev(gpu, resid)
        gpu._check(L.g4_rms_join(dcodes_src.ptr, gpu.KIND_I8, OUT, dgain.ptr, dres2.ptr, alpha,
                                 dgain2.ptr, rows, width, EPS, IN, dres2.ptr, cod.ptr, None))
        wh, wc = d.norm_residual_norm(src, gain, resid, gain2, alpha, EPS, IN)
        assert same(dres2.download(), wh)
        assert same(cod.download(), wc)


def o_codes(row):
    import oracle as o
    return o.srq_codes(row, IN)


@pytest.mark.parametrize("producer", [False, True])
@pytest.mark.parametrize("use_dev_pos", [False, True])
def test_attn_prologue(gpu, producer, use_dev_pos):
    print(f"attn_prologue producer={producer} dev_pos={use_dev_pos}", flush=True)
    import g4decode as gd
    L = gpu.lib()
    rng = np.random.default_rng(3 + producer)
    rows, heads, hd, cap, pos = 2, 8, 256, 1024, 777
    cos, sin = gd.rope_tables(cap, hd, 1e6, 0.25)
    qc = rng.integers(-128, 128, (rows, heads, hd)).astype(np.int8)
    kc = rng.integers(-128, 128, (rows, hd)).astype(np.int8)
    vc = rng.integers(-128, 128, (rows, hd)).astype(np.int8)
    qg = rng.uniform(0.1, 0.4, hd).astype(np.float32)
    kg = rng.uniform(0.1, 0.4, hd).astype(np.float32)
    dq, dk, dv = dev(gpu, qc), dev(gpu, kc), dev(gpu, vc)
    dqg, dkg, dcos, dsin = dev(gpu, qg), dev(gpu, kg), dev(gpu, cos), dev(gpu, sin)
    qout = out_buf(gpu, (rows, heads, hd), np.float32)
    cache = np.full((rows, 2, cap, hd), 5.0, np.float32)
    dcache = dev(gpu, cache)
    stride = 2 * cap * hd
    vbase = dcache.ptr + cap * hd * 4
    pos_buf = dev(gpu, np.array([pos], np.int32))
    gpu._check(L.g4_attn_prologue(dq.ptr, OUT, dk.ptr if producer else None, OUT,
                                  dv.ptr if producer else None, OUT, dqg.ptr,
                                  dkg.ptr if producer else None, dcos.ptr, dsin.ptr, rows, heads, hd,
                                  EPS, qout.ptr, dcache.ptr if producer else None,
                                  vbase if producer else None, stride, cap - 1 if use_dev_pos else pos,
                                  pos_buf.ptr if use_dev_pos else None, None))
    got = qout.download()
    got_cache = dcache.download()
    for r in range(rows):
        assert same(got[r], d.q_norm_rope(qc[r], OUT, qg, cos[pos], sin[pos], EPS))
        if producer:
            kr, vr = d.kv_norm_rope(kc[r], OUT, vc[r], OUT, kg, cos[pos], sin[pos], EPS)
            assert same(got_cache[r, 0, pos], kr)
            assert same(got_cache[r, 1, pos], vr)
    # nothing but row `pos` of each cache changed
    mask = np.ones(cap, bool)
    if producer:
        mask[pos] = False
    assert np.all(got_cache[:, :, mask] == 5.0)


# rows 2: two halves of four heads with K staged in LDS (grids up to 256 blocks); at position
# 4095 (128 chunks) rows 5 stage K with one half (640 blocks) and rows 7 load per-lane K segments
# (896 blocks)
@pytest.mark.parametrize("pos,window,rows", [(0, 0, 2), (1, 0, 2), (255, 0, 2), (256, 0, 2),
                                             (700, 0, 2), (4095, 0, 2), (4095, 512, 2),
                                             (511, 512, 2), (512, 512, 2), (1000, 512, 2),
                                             (4095, 0, 5), (4095, 0, 7)])
def test_attention_decode(gpu, pos, window, rows):
    print(f"attention pos={pos} window={window} rows={rows}", flush=True)
    L = gpu.lib()
    rng = np.random.default_rng(pos * 3 + window + 1000 * (rows - 2))
    heads, hd = 8, 256
    cap = max(pos + 1, 300)
    q = (rng.standard_normal((rows, heads, hd)) * 0.25).astype(np.float32)
    kv = rng.uniform(-1.7, 1.7, (rows, 2, cap, hd)).astype(np.float32)
    dq, dkv = dev(gpu, q), dev(gpu, kv)
    stride = 2 * cap * hd
    for use_dev_pos in (False, True):
        # with the device word, the grid is sized for the largest position
        bound = cap - 1 if use_dev_pos else pos
        ws_bytes = L.g4_attention_workspace_bytes(rows, heads, bound, window)
        ws = gpu.DeviceBuffer(ws_bytes, np.uint8)
        codes = out_buf(gpu, (rows, heads, hd), np.int8)
        f = out_buf(gpu, (rows, heads, hd), np.float32)
        pos_buf = dev(gpu, np.array([pos], np.int32))
        gpu._check(L.g4_attention_decode(dq.ptr, dkv.ptr, dkv.ptr + cap * hd * 4, stride, rows,
                                         heads, hd, bound, pos_buf.ptr if use_dev_pos else None,
                                         window, ws.ptr, ws_bytes, IN, codes.ptr, f.ptr, None))
        got, got_c = f.download(), codes.download()
        for r in range(rows):
            want = d.attention_decode(q[r], kv[r, 0], kv[r, 1], pos, window)
            assert same(got[r], want), (r, use_dev_pos)
            assert same(got_c[r].ravel(), o_codes(want.ravel()))


@pytest.mark.parametrize("n,ple", [(6144, False), (256, True), (1000, False)])
def test_gelu_mul(gpu, n, ple):
    print(f"gelu_mul n={n} ple={ple}", flush=True)
    L = gpu.lib()
    rng = np.random.default_rng(n)
    rows = 3
    g = rng.integers(-128, 128, (rows, n)).astype(np.int8)
    u = rng.integers(-128, 128, (rows, n)).astype(np.int8)
    stride = n * 5
    up = rng.uniform(-3, 3, (rows, stride)).astype(np.float32)
    dg, du, dup = dev(gpu, g), dev(gpu, u), dev(gpu, up)
    codes = out_buf(gpu, (rows, n), np.int8)
    gpu._check(L.g4_gelu_mul(dg.ptr, OUT, None if ple else du.ptr, OUT, dup.ptr if ple else None,
                             stride, rows, n, IN, codes.ptr, None))
    got = codes.download()
    for r in range(rows):
        want = d.gelu_mul_codes(g[r], OUT, None if ple else u[r], OUT, IN,
                                up_f32=up[r, :n] if ple else None)
        assert same(got[r], want)


def test_embed_tokens(gpu):
    L = gpu.lib()
    rng = np.random.default_rng(8)
    vocab, cols = 1000, 1536
    table = rng.integers(0, 256, (vocab, cols // 2)).astype(np.uint8)
    scales = rng.uniform(0.005, 0.02, vocab).astype(np.float32)
    ids = np.array([0, 999, 17, 17, 512, -1, 1000], np.int32)  # the last two are out of range
    es = float(np.float32(np.sqrt(1536.0)))
    dt, ds, di = dev(gpu, table), dev(gpu, scales), dev(gpu, ids)
    x = out_buf(gpu, (ids.size, cols), np.float32)
    c = out_buf(gpu, (ids.size, cols), np.int8)
    gpu._check(L.g4_embed_tokens(dt.ptr, ds.ptr, di.ptr, ids.size, vocab, cols, es, IN, x.ptr,
                                 c.ptr, None))
    gx, gc = x.download(), c.download()
    for r, t in enumerate(ids):
        if not 0 <= t < vocab:
            assert np.all(gx[r] == 0.0) and np.all(gc[r] == 0)
            continue
        want = d.embed_row(table[t], scales[t], cols, es)
        assert same(gx[r], want)
        assert same(gc[r], o_codes(want))


def test_ple_combine(gpu):
    L = gpu.lib()
    rng = np.random.default_rng(9)
    rows, groups, group = 3, 35, 256
    pc = rng.integers(-128, 128, (rows, groups * group)).astype(np.int8)
    gain = rng.uniform(0.5, 1.5, group).astype(np.float32)
    ident = rng.uniform(-2, 2, (rows, groups * group)).astype(np.float32)
    alpha = float(np.float32(1536 ** -0.5))
    dpc, dg, di = dev(gpu, pc), dev(gpu, gain), dev(gpu, ident)
    out = out_buf(gpu, (rows, groups * group), np.float32)
    gpu._check(L.g4_ple_combine(dpc.ptr, OUT, alpha, dg.ptr, di.ptr, rows, groups, group, EPS,
                                out.ptr, None))
    got = out.download()
    for r in range(rows):
        assert same(got[r], d.ple_combine(pc[r], OUT, alpha, gain, ident[r], group, EPS))


@pytest.mark.parametrize("vocab,cap", [(262144, 30.0), (5000, 30.0), (4096, 0.0), (1, 30.0)])
def test_softcap_argmax(gpu, vocab, cap):
    print(f"softcap_argmax vocab={vocab} cap={cap}", flush=True)
    L = gpu.lib()
    rng = np.random.default_rng(vocab)
    rows = 4
    x = rng.integers(-40, 41, (rows, vocab)).astype(np.float32)  # many ties
    if vocab > 5000:
        x[1, 7] = x[1].max()           # tie across partial blocks: the lowest index wins
        x[1, vocab - 3] = x[1].max()
        x[2, :] = np.nan
        x[2, 4097] = 1.0               # NaN never wins
    if vocab == 5000:
        x[3, :] = np.nan               # nothing wins: -1
    if cap == 0.0:
        x[3, :] = -np.inf              # uncapped, nothing exceeds -inf: -1 (capped, -inf is -30)
    dx = dev(gpu, x)
    capped = out_buf(gpu, (rows, vocab), np.float32)
    ws_bytes = L.g4_argmax_workspace_bytes(rows, vocab)
    ws = gpu.DeviceBuffer(ws_bytes, np.uint8)
    tok = out_buf(gpu, (rows,), np.int32)
    gpu._check(L.g4_softcap_argmax(dx.ptr, rows, vocab, cap, capped.ptr, ws.ptr, ws_bytes, tok.ptr,
                                   None))
    gc, gt = capped.download(), tok.download()
    for r in range(rows):
        want = d.softcap(x[r], cap)
        assert same(gc[r], want), r
        assert gt[r] == d.argmax(want), (r, gt[r], d.argmax(want))
    if vocab == 5000 or cap == 0.0:
        assert gt[3] == -1


# ---- the decode step --------------------------------------------------------------------------

def tiny_shape(batch, **kw):
    import g4decode as gd
    base = dict(layers=7, kv_producers=4, hidden=512, ffn=1024, q_heads=8, global_period=3,
                sliding_window=512, kv_capacity=1024, batch=batch, vocab=3000)
    base.update(kw)
    return gd.Shape(**base)


def run_steps(gpu, shape, tokens_list, pos0, stop=None, seed=4):
    """Device and oracle side by side for consecutive steps; returns both results per step."""
    import decode_ref as ref
    import g4decode as gd
    model = gd.SyntheticModel(shape, seed=seed)
    dec = gd.Decoder(shape, model)
    if stop is not None:
        dec.set_stop(stop)
    dec.fill_kv_history()
    gpu.synchronize()
    kv = {p: dec.download_kv(p) for p in range(shape.kv_producers)}
    W = ref.Weights(model)
    out = []
    nxt = gpu.DeviceBuffer.empty((shape.batch,), np.int32)
    for i, toks in enumerate(tokens_list):
        pos = pos0 + i
        dtoks = dev(gpu, np.asarray(toks, np.int32))
        dec.set_position(pos)
        dec.step(dtoks, nxt)
        gpu.synchronize()
        got = {"hidden": dec.download("hidden", np.float32),
               "codes": dec.download("codes" if stop is not None else "head_codes", np.int8),
               "per_layer": dec.download("per_layer", np.float32)}
        if stop is None:
            got["logits"] = dec.download("logits", np.float32)
            got["next"] = nxt.download()
        want = ref.step(shape, W, kv, list(toks), pos, stop=stop)
        if stop is None:
            want["codes"] = want["head_codes"]
        out.append((got, want, {p: dec.download_kv(p) for p in range(shape.kv_producers)}, {p: (k.copy(), v.copy()) for p, (k, v) in kv.items()}))
    dec.close()
    return out


def check_step(got, want, dev_kv, ref_kv):
    for key in got:
        assert same(got[key], want[key]), key
    for p in ref_kv:
        for a, b in zip(dev_kv[p], ref_kv[p]):
            assert same(a, b), f"kv layer {p}"


# batch 1: the streaming plans with carried joins; 3: the small-M kernel on 16-row tiles; 20 and
# 32: on 32-row tiles, with the gelu-mul epilogues on 16-wave (FFN 1024: 64 blocks) and 4-wave
# (FFN 6144: 384 blocks) grids. Attention grids (chunks x batch): two halves with K staged in LDS
# up to 256 blocks, K staged up to 768 (batch 20 and 32 at position 700: 22 x 32 = 704), and the
# per-lane K segments beyond (batch 32 at position 1000: 32 x 32 = 1024).
@pytest.mark.parametrize("batch,ffn,pos0", [(1, 1024, 700), (3, 1024, 700), (20, 1024, 700),
                                            (32, 6144, 700), (32, 1024, 1000)])
def test_decode_step_tiny(gpu, batch, ffn, pos0):
    print(f"decode tiny batch={batch} ffn={ffn} pos0={pos0}", flush=True)
    shape = tiny_shape(batch, ffn=ffn)
    rng = np.random.default_rng(batch)
    extra = [int(t) for t in rng.integers(0, 3000, max(0, batch - 3))]
    toks = [([5, 2999, 1234] + extra)[:batch], ([7, 0, 1] + extra[::-1])[:batch]]
    for got, want, dkv, rkv in run_steps(gpu, shape, toks, pos0=pos0):
        check_step(got, want, dkv, rkv)
        if "next" in got:
            print("next tokens", got["next"], flush=True)


# Fewer than eight query heads: the split kernel's prologue waves past the last head (and the
# waves that build no K / V row) load stand-in rows whose values go unused; the scores and P.V
# take the guarded forms. Batch 1 (two halves, K in LDS), batch 32 at position 700 (K in LDS) and
# at 1000 (per-lane K segments).
@pytest.mark.parametrize("batch,pos0", [(1, 700), (32, 700), (32, 1000)])
def test_decode_step_six_heads(gpu, batch, pos0):
    print(f"decode 6 heads batch={batch} pos0={pos0}", flush=True)
    shape = tiny_shape(batch, q_heads=6)
    toks = [[(97 * i + 5) % 3000 for i in range(batch)]]
    for got, want, dkv, rkv in run_steps(gpu, shape, toks, pos0=pos0):
        check_step(got, want, dkv, rkv)


# Batch 1 folds o_proj into the attention merge (bit 0), gate / up / gelu-mul / down into the FFN
# block (bit 1) and the per-layer-input pair into its block (bit 2) wherever they fit; each mix of
# folded and plan forms hands its int32 accumulators or codes to a different join. Hidden 512 fits
# all three, so fold_off walks every combination; hidden 768 (not a multiple of 512) leaves the FFN
# block out by shape, with the merge and per-layer-input folds on, then with the latter off.
@pytest.mark.parametrize("hidden,fold_off", [(512, f) for f in range(1, 8)] + [(768, 0), (768, 4)])
def test_decode_batch1_fold_combinations(gpu, hidden, fold_off):
    print(f"decode batch 1 hidden={hidden} fold_off={fold_off}", flush=True)
    shape = tiny_shape(1, hidden=hidden, fold_off=fold_off)
    for got, want, dkv, rkv in run_steps(gpu, shape, [[5], [2999]], pos0=700):
        check_step(got, want, dkv, rkv)


def test_decode_fold_off_range(gpu):
    import g4decode as gd
    shape = tiny_shape(1, fold_off=8)
    with pytest.raises(gpu.G4Error, match="fold_off 8"):
        gd.Decoder(shape, gd.SyntheticModel(tiny_shape(1), seed=4))


def test_decode_stop_after_each_layer(gpu):
    shape = tiny_shape(1, layers=5, kv_producers=3)
    for stop in range(shape.layers - 1):
        print(f"stop={stop}", flush=True)
        (got, want, dkv, rkv), = run_steps(gpu, shape, [[11]], pos0=600, stop=stop)
        check_step(got, want, dkv, rkv)


def test_decode_batch_rows_match_batch1(gpu):
    """Rows are independent: row 0 of a batch-3 step equals the batch-1 step on the same token,
    though the linears run on different kernels (the M = 1 plan vs the small-M MFMA path)."""
    import g4decode as gd
    res = []
    for batch in (1, 3):
        shape = tiny_shape(batch)
        model = gd.SyntheticModel(shape, seed=4)
        dec = gd.Decoder(shape, model)
        # the fill hashes the element index, and row 0 is the first 2 * capacity * head_dim
        # elements of every cache in both layouts: row 0 starts from the same history
        dec.fill_kv_history()
        dec.set_position(300)
        nxt = gpu.DeviceBuffer.empty((batch,), np.int32)
        dec.step(dev(gpu, np.array([42, 9, 9][:batch], np.int32)), nxt)
        gpu.synchronize()
        res.append((dec.download("logits", np.float32), nxt.download(),
                    dec.download("hidden", np.float32)))
        dec.close()
    assert same(res[1][0][0], res[0][0][0])
    assert res[1][1][0] == res[0][1][0]
    assert same(res[1][2][0], res[0][2][0])


def test_decode_graph_replay(gpu):
    """One captured step replays the following tokens: positions come from the device word."""
    import g4decode as gd
    shape = tiny_shape(1)
    eager, graph = [], []
    for mode in ("eager", "graph"):
        model = gd.SyntheticModel(shape, seed=5)
        dec = gd.Decoder(shape, model)
        dec.fill_kv_history()
        st = gpu.Stream()
        toks = dev(gpu, np.array([17], np.int32))
        nxt = gpu.DeviceBuffer.empty((1,), np.int32)
        dec.set_position(800)
        dec.step(toks, nxt, st.handle)      # warm (plans and library state ready before capture)
        st.synchronize()
        g = gpu.Graph(st, lambda: dec.step(toks, nxt, st.handle)) if mode == "graph" else None
        seq = []
        for i in range(4):
            dec.set_position(801 + i)
            gpu._check(gpu.lib().g4_memcpy_d2d(toks.ptr, nxt.ptr, 4, None))
            gpu.synchronize()
            if g is not None:
                g.launch()
            else:
                dec.step(toks, nxt, st.handle)
            st.synchronize()
            seq.append((int(nxt.download()[0]), dec.download("logits", np.float32).copy()))
        (eager if mode == "eager" else graph).extend(seq)
        if g is not None:
            g.close()
        dec.close()
        st.close()
    for (te, le), (tg, lg) in zip(eager, graph):
        assert te == tg
        assert same(le, lg)


@pytest.mark.parametrize("batch", [1, 3, 32])
def test_decode_step_e2b_full(gpu, batch):
    """BASELINE config 4 at its real shape: 35 layers (15 KV producers), hidden 1536, FFN 6144,
    8 query heads over one KV head of 256, tied int4 head over 262144 rows, a 4096-position seeded
    KV, decoding position 4095 (global layers attend over all 4096 positions, sliding ones over
    512). Every output of the step is compared bit for bit: next tokens, capped logits, the final
    residual row, the per-layer inputs and each producer's KV row at the position."""
    import decode_ref as ref
    import g4decode as gd
    print(f"decode e2b full batch={batch}", flush=True)
    shape = gd.Shape(batch=batch, kv_capacity=4096)
    model = gd.SyntheticModel(shape, seed=4)
    dec = gd.Decoder(shape, model)
    dec.fill_kv_history()
    gpu.synchronize()
    pos = 4095
    kv = {}
    for p in range(shape.kv_producers):
        k, v = dec.download_kv(p)
        kv[p] = (k.copy(), v.copy())
    # batch 32 adds seeded ids over the whole vocabulary (the rows run different kernels than at
    # batch 1 and 3: 16-wave small-M grids, split down_proj accumulators, the 64-row tile head)
    toks = ([1234, 262143, 7] + [int(t) for t in np.random.default_rng(32).integers(
        0, 262144, 29)])[:batch]
    nxt = gpu.DeviceBuffer.empty((batch,), np.int32)
    dec.set_position(pos)
    dec.step(dev(gpu, np.array(toks, np.int32)), nxt)
    gpu.synchronize()
    got = {"next": nxt.download(), "logits": dec.download("logits", np.float32),
           "hidden": dec.download("hidden", np.float32),
           "per_layer": dec.download("per_layer", np.float32),
           "head_codes": dec.download("head_codes", np.int8)}
    dkv = {p: dec.download_kv(p) for p in range(shape.kv_producers)}
    dec.close()
    print("device step done; running the CPU composition", flush=True)
    want = ref.step(shape, ref.Weights(model), kv, toks, pos)
    print("next tokens", got["next"], want["next"], flush=True)
    for key in got:
        assert same(got[key], want[key]), key
    for p in kv:
        assert same(dkv[p][0][:, pos], kv[p][0][:, pos]) and same(dkv[p][1][:, pos], kv[p][1][:, pos]), p


def test_decode_step_e2b_split_ple_table(gpu):
    """The E2B-shape step with the 1.17 GB PLE table carried as the 5 slices of the default-cap
    plan at 1 GiB bindings (tableSplit.ts planTableSplit; plan.ts:709-725 one gather step per
    slice, one fused launch here): the same next tokens, logits, residual and per-layer inputs as
    the same model with the table whole."""
    import g4decode as gd
    shape = gd.Shape(batch=3, kv_capacity=4096)
    model = gd.SyntheticModel(shape, seed=4)
    plan, slices = gpu.plan_table_split(shape.vocab, shape.layers * shape.ple_dim // 2, 1 << 30,
                                        1 << 30, 10, 0)
    assert plan.num_slices == 5
    toks = dev(gpu, np.array([59903, 59904, 262143], np.int32))  # both sides of a slice boundary
    outs = []
    for split in (False, True):
        if split:
            model.split_ple(slices, drop_whole=True)
        dec = gd.Decoder(shape, model)
        dec.fill_kv_history()
        dec.set_position(4095)
        nxt = gpu.DeviceBuffer.empty((shape.batch,), np.int32)
        dec.step(toks, nxt)
        gpu.synchronize()
        outs.append([nxt.download(), dec.download("logits", np.float32),
                     dec.download("hidden", np.float32), dec.download("per_layer", np.float32)])
        dec.close()
    for a, b in zip(*outs):
        assert same(a, b)
