"""The whole decode step on the CPU, composed from the pinned oracle functions.

TEST INFRASTRUCTURE ONLY: tests/ and bench.py's cpu_baseline leg use it as the checker. It walks
the reference's decode plan (src/plan.ts:487-665 planLayer, :720-729 planEmbed, :768-777 planHead)
for one position, with the same per-kernel arithmetic the oracle restates:
  linears           oracle.qgemm (qgemvOracle, qgemv.ts:1131-1176): int8 codes in, int8 out
  joins, norms      decode_oracle (rmsNorm.ts, mlpEpilogue.ts, blockJoin.ts)
  prologue, rope    decode_oracle (attnPrologue.ts, rope.ts)
  attention         decode_oracle (attention.ts:858-918, split form)
  gelu-mul          decode_oracle (geluMul.ts), embed and PLE combine (embedGather.ts, plan.ts)
  head              oracle.qgemm with outScale 0 (f32 logits), softcap, argmax
Inputs are host arrays read back from the device model, so both sides see the same bytes.
"""
from __future__ import annotations

import math

import numpy as np

import decode_oracle as d
import oracle as o


def _f32(x):
    return np.float32(x)


def linear(bits, w, s, codes, n, k, in_scale, out_scale):
    """int8 codes in: x = codes * in_scale rounds back to the same codes in the oracle's own snap
    (|code| <= 128 keeps the f32 product within 2^-22 of the integer), so this is exactly the
    reference linear fed pre-snapped codes."""
    x = codes.astype(np.float32).reshape(-1, k) * _f32(in_scale)
    dst, _, out = o.qgemm(bits, w, s, x, n, k, x.shape[0], in_scale, out_scale)
    return out if out_scale != 0.0 else dst


class Weights:
    """Host copies of a SyntheticModel's tensors, fetched lazily (the PLE table by row)."""

    def __init__(self, model):
        self.model = model
        self.cache = {}

    def __getitem__(self, name):
        if name not in self.cache:
            self.cache[name] = self.model.host(name)
        return self.cache[name]


def step(shape, W, kv, tokens, pos, stop=None):
    """One decode step for rows `tokens` at position `pos`.

    kv: {producer: (K [batch][cap][hd], V [batch][cap][hd])} f32 arrays, updated in place at `pos`.
    Returns a dict: hidden, codes (the next projection input when stopped early), head_codes,
    logits (capped), next (tokens), per_layer."""
    s = shape
    H, F, QW, P, hd = s.hidden, s.ffn, s.q_heads * s.head_dim, s.ple_dim, s.head_dim
    PL = s.layers * P
    ins, outs, eps = s.in_scale, s.out_scale, s.eps
    B = len(tokens)
    last = s.layers - 1 if stop is None else stop
    res = {k: [] for k in ("hidden", "codes", "head_codes", "logits", "next", "per_layer")}
    embed_scale = _f32(math.sqrt(H))
    cos_l, sin_l = W["rope_local_cos"], W["rope_local_sin"]
    cos_g, sin_g = W["rope_global_cos"], W["rope_global_sin"]
    ple_rows = W.model.host_rows("ple_table", tokens)
    ple_s = W["ple_table_s"]
    for b, tok in enumerate(tokens):
        # embedding phase (plan.ts:720-729)
        x = d.embed_row(W["embed"][tok], W["embed_s"][tok], H, embed_scale)
        ecodes = o.srq_codes(x, ins)
        identity = o.embed_gather(ple_rows[b:b + 1], ple_s[tok:tok + 1], np.zeros(1, np.int32), PL,
                                  P, out_kind="f32")[0]
        pm = linear(4, W["ple_model_proj"], W["ple_model_proj_s"], ecodes, PL, H, ins, outs)[0]
        per_layer = d.ple_combine(pm, outs, _f32(H ** -0.5), W["ple_proj_norm"], identity, P, eps)
        hidden = x
        xc = d.rms_norm_codes(hidden[None], W["l0.input_norm"], eps, ins)[0]
        for l in range(last + 1):
            pre = f"l{l}."
            prod = l < s.kv_producers
            glob = s.is_global(l)
            cos, sin = (cos_g, sin_g) if glob else (cos_l, sin_l)
            qc = linear(4, W[pre + "q"], W[pre + "q_s"], xc, QW, H, ins, outs)[0]
            q = d.q_norm_rope(qc.reshape(s.q_heads, hd), outs, W[pre + "q_norm"], cos[pos],
                              sin[pos], eps)
            src = s.kv_source(l)
            K, V = kv[src]
            if prod:
                kc = linear(4, W[pre + "k"], W[pre + "k_s"], xc, hd, H, ins, outs)[0]
                vc = linear(4, W[pre + "v"], W[pre + "v_s"], xc, hd, H, ins, outs)[0]
                K[b, pos], V[b, pos] = d.kv_norm_rope(kc, outs, vc, outs, W[pre + "k_norm"],
                                                      cos[pos], sin[pos], eps)
            att = d.attention_decode(q, K[b, :pos + 1], V[b, :pos + 1], pos, s.window(l))
            ac = o.srq_codes(att.reshape(-1), ins)
            oc = linear(4, W[pre + "o"], W[pre + "o_s"], ac, H, QW, ins, outs)[0]
            h2, xc = d.norm_residual_norm((oc.astype(np.float32) * _f32(outs))[None],
                                          W[pre + "post_attn_norm"], hidden[None],
                                          W[pre + "pre_ffn_norm"], 1.0, eps, ins)
            hidden, xc = h2[0], xc[0]
            gc = linear(4, W[pre + "gate"], W[pre + "gate_s"], xc, F, H, ins, outs)[0]
            uc = linear(4, W[pre + "up"], W[pre + "up_s"], xc, F, H, ins, outs)[0]
            act = d.gelu_mul_codes(gc, outs, uc, outs, ins)
            dc = linear(4, W[pre + "down"], W[pre + "down_s"], act, H, F, ins, outs)[0]
            hidden = d.norm_residual((dc.astype(np.float32) * _f32(outs))[None],
                                     W[pre + "post_ffn_norm"], hidden[None], eps)[0]
            xc = o.srq_codes(hidden, ins)
            pg = linear(8, W[pre + "ple_gate"], W[pre + "ple_gate_s"], xc, P, H, ins, outs)[0]
            pac = d.gelu_mul_codes(pg, outs, None, 0.0, ins, up_f32=per_layer[l * P:(l + 1) * P])
            pp = linear(8, W[pre + "ple_proj"], W[pre + "ple_proj_s"], pac, H, P, ins, outs)[0]
            nxt = W["final_norm"] if l + 1 == s.layers else W[f"l{l + 1}.input_norm"]
            h2, xc = d.norm_residual_norm((pp.astype(np.float32) * _f32(outs))[None],
                                          W[pre + "post_ple_norm"], hidden[None], nxt,
                                          float(W.model.layer_scalar[l]), eps, ins)
            hidden, xc = h2[0], xc[0]
        res["hidden"].append(hidden)
        res["codes"].append(xc)
        res["per_layer"].append(per_layer)
        if last == s.layers - 1:
            logits = linear(4, W["embed"], W["embed_s"], xc, s.vocab, H, ins, 0.0)[0]
            capped = d.softcap(logits, s.final_softcap)
            res["head_codes"].append(xc)
            res["logits"].append(capped)
            res["next"].append(d.argmax(capped))
    return {k: np.array(v) for k, v in res.items() if v}
