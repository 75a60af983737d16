"""Extract oracle-form (per-projection, decoded) weights from product objects."""

from __future__ import annotations

import torch


def _dec(lw):
    from ltx_amd.kernels import gemm

    return gemm.dequantize(lw).float().cpu()


def _bias(lw, n):
    return torch.zeros(n) if lw.bias is None else lw.bias.float().cpu()


def attention_weights(a) -> dict:
    inner, heads = a.inner_dim, a.heads
    pq = _dec(a.proj_q)
    bq = _bias(a.proj_q, pq.shape[0])
    w = {}
    if a.self_attention:
        names = [("to_q", 0, inner), ("to_k", inner, 2 * inner), ("to_v", 2 * inner, 3 * inner),
                 ("to_gate_logits", 3 * inner, 3 * inner + heads)]
        for n, s, e in names:
            w[n], w[n + "_b"] = pq[s:e], bq[s:e]
    else:
        w["to_q"], w["to_q_b"] = pq[:inner], bq[:inner]
        w["to_gate_logits"], w["to_gate_logits_b"] = pq[inner:], bq[inner:]
        pkv = _dec(a.proj_kv)
        bkv = _bias(a.proj_kv, pkv.shape[0])
        w["to_k"], w["to_k_b"] = pkv[:inner], bkv[:inner]
        w["to_v"], w["to_v_b"] = pkv[inner:], bkv[inner:]
    w["to_out"], w["to_out_b"] = _dec(a.to_out), _bias(a.to_out, a.to_out.out_features)
    for n in ("to_q", "to_k", "to_v", "to_gate_logits"):
        w[n + "_qlinear"] = (a.proj_q if n in ("to_q", "to_gate_logits") or a.self_attention
                             else a.proj_kv).qlinear
    w["to_out_qlinear"] = a.to_out.qlinear
    w["q_norm"], w["k_norm"] = a.q_norm.float().cpu(), a.k_norm.float().cpu()
    return w


def ff_weights(f) -> dict:
    return {"w1": _dec(f.project_in), "b1": _bias(f.project_in, f.inner_dim),
            "w2": _dec(f.project_out), "b2": _bias(f.project_out, f.dim_out),
            "w1_qlinear": f.project_in.qlinear, "w2_qlinear": f.project_out.qlinear}


def block_weights(b) -> dict:
    W = {}
    for name in ("attn1", "attn2", "audio_attn1", "audio_attn2", "audio_to_video_attn", "video_to_audio_attn"):
        a = getattr(b, name)
        if a is not None:
            W[name] = attention_weights(a)
    if b.ff is not None:
        W["ff"] = ff_weights(b.ff)
    if b.audio_ff is not None:
        W["audio_ff"] = ff_weights(b.audio_ff)
    return W


def mlp_weights(m) -> dict:
    return {"w1": m.w1.float().cpu(), "b1": m.b1.float().cpu(), "w2": m.w2.float().cpu(), "b2": m.b2.float().cpu(),
            "w": m.w.float().cpu(), "b": m.b.float().cpu()}
