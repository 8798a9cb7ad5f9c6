"""The CPU composition of the decode step (oracle/decode_ref.py) on a small synthetic model built
by the host restatement of the device fill: it runs end to end, updates exactly the KV rows of the
position, and the synthetic scales keep every projection's int8 codes in range (neither zero nor
saturated), so the bit-exact GPU comparison exercises real values rather than clamps."""
import numpy as np

import decode_ref as ref
import g4decode as gd


def tiny(batch=1):
    return gd.Shape(layers=4, kv_producers=3, hidden=512, ffn=512, q_heads=8, global_period=2,
                    sliding_window=512, kv_capacity=640, batch=batch, vocab=600)


def test_reference_step_runs_and_writes_the_position():
    s = tiny(batch=2)
    model = gd.HostReplica(s, seed=4)
    kv = {p: tuple(np.array(a) for a in gd.kv_history(s, p).transpose(1, 0, 2, 3))
          for p in range(s.kv_producers)}
    before = {p: (kv[p][0].copy(), kv[p][1].copy()) for p in kv}
    out = ref.step(s, ref.Weights(model), kv, [3, 599], pos=600)
    assert out["next"].shape == (2,)
    assert np.all((out["next"] >= 0) & (out["next"] < s.vocab))
    assert np.all(np.abs(out["logits"]) <= 30.0)
    for p in kv:
        for a, b in zip(kv[p], before[p]):
            changed = np.any(a != b, axis=2)  # [batch][capacity]
            assert changed[:, 600].all() and changed.sum() == 2
    # the codes the head reads are live: mostly unsaturated and not all zero
    hc = out["head_codes"].astype(int)
    assert 0.0 < np.mean(hc != 0) and np.mean(np.abs(hc) >= 127) < 0.05
    # determinism: the same inputs give the same bits
    kv2 = {p: (before[p][0].copy(), before[p][1].copy()) for p in before}
    again = ref.step(s, ref.Weights(model), kv2, [3, 599], pos=600)
    assert np.array_equal(again["logits"].view(np.uint32), out["logits"].view(np.uint32))


def test_layer_outputs_in_range():
    s = tiny()
    model = gd.HostReplica(s, seed=7)
    kv = {p: tuple(np.array(a) for a in gd.kv_history(s, p).transpose(1, 0, 2, 3))
          for p in range(s.kv_producers)}
    for stop in range(s.layers - 1):
        kvc = {p: (kv[p][0].copy(), kv[p][1].copy()) for p in kv}
        out = ref.step(s, ref.Weights(model), kvc, [17], pos=300, stop=stop)
        c = out["codes"].astype(int)
        h = out["hidden"]
        print(f"layer {stop}: hidden rms {np.sqrt(np.mean(h * h)):.3f}, "
              f"codes nonzero {np.mean(c != 0):.2f}, saturated {np.mean(np.abs(c) >= 127):.3f}")
        assert np.all(np.isfinite(h))
        assert np.mean(c != 0) > 0.5 and np.mean(np.abs(c) >= 127) < 0.05


def test_host_replica_rows_match_whole_tensor():
    s = tiny()
    m = gd.HostReplica(s, seed=4)
    whole = m.host("ple_table")
    assert np.array_equal(m.host_rows("ple_table", [0, 599, 17]), whole[[0, 599, 17]])
