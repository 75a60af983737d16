"""Oracle for the audio+video transformer block and the denoise step.

A float32 torch-CPU restatement of model/transformer/transformer.py:389-674,
attention.py:528-603, feed_forward.py:64-112, model.py:285-497, :1312-1342,
:1489-1542 and diffusion_steps.py:58-69, with every bf16 rounding of the
reference (``bf`` marks them).  Weights are plain per-projection tensors
(to_q, to_k, to_v, to_gate_logits, to_out, ...), decoded to their bf16
values, as in the reference's modules; ``<name>_qlinear`` marks a projection
that the reference runs as a quantised linear (bias added after the bf16
rounding of the product).

AdaLN follows the reference's dispatch default (transformer.py:85-110): the
compiled inline form ``(rms_norm(x) * (1 + scale) + shift).astype(bf16)``
whose rms_norm output is bf16 (``fused_adaln=False``); ``fused_adaln=True``
is the single-rounding fused kernel (fused_ops.py:172-175).

Pinning: built from the pinned pieces (oracle.fused_ops, oracle.rope,
oracle.attention, oracle.quant.linear semantics), and checked in
tests/test_oracle_block.py by properties that a wiring mistake breaks:
zero gates make every sub-layer vanish; a zero A2V gate decouples audio from
video; the FF path is per token; each of the 12 (scale, shift) row pairs
feeds its own sub-layer input (scale -1 / shift c turns that input into the
constant c, so the update becomes one shared row), including the AV tables'
scale-before-shift order, and the mirrored assignment fails; V2A reads the
norm taken before A2V (the A2V weights cannot reach the audio output); each
cross-PE table rotates its own side in both directions (a 90-degree table
equals rotated projection rows); text cross-attention rounds twice, the
self-attention residual once.  Test infrastructure only: the product never
imports this module.
"""

from __future__ import annotations

import math

import torch

EPS = 1e-6


def bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


def rms_inv(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    return torch.rsqrt(x.double().square().mean(-1, keepdim=True) + eps).float()


def rms_norm_bf(x, eps=EPS):
    """mx.fast.rms_norm(x) on bf16 x (no weight): bf16 output."""
    return bf(x * rms_inv(x, eps))


def adaln(x, scale, shift, eps=EPS, fused=False):
    if fused:
        return bf(x * rms_inv(x, eps) * (1 + scale) + shift)
    return bf(rms_norm_bf(x, eps) * (1 + scale) + shift)


def linear(x, w, b=None, qlinear=False):
    """nn.Linear / mx.addmm on bf16: fp32 accumulation, bf16 output.  With
    ``qlinear`` nn.QuantizedLinear's form (loader/transformer_cache.py:
    177-193): the product is rounded to bf16 before the bias add."""
    y = x @ w.T
    if qlinear:
        y = bf(y)
    if b is not None:
        y = y + b
    return bf(y)


def _proj(w: dict, name: str, x):
    return linear(x, w[name], w[name + "_b"], w.get(name + "_qlinear", False))


def gelu_tanh(x):
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def rope(x, cos, sin, heads):
    """Split RoPE (rope.py:37-89) with token-major (T, D/2) tables."""
    t, d = x.shape
    dh = d // heads
    xh = x.view(t, heads, dh)
    c = cos.view(t, heads, dh // 2)
    s = sin.view(t, heads, dh // 2)
    x1, x2 = xh[..., : dh // 2], xh[..., dh // 2:]
    return bf(torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], -1).reshape(t, d))


def sdpa(q, k, v, heads):
    tq, d = q.shape
    tk = k.shape[0]
    dh = d // heads
    qh = q.view(tq, heads, dh).transpose(0, 1)
    kh = k.view(tk, heads, dh).transpose(0, 1)
    vh = v.view(tk, heads, dh).transpose(0, 1)
    p = torch.softmax(torch.matmul(qh, kh.transpose(1, 2).contiguous()) / math.sqrt(dh), -1)
    return bf(torch.matmul(p, vh.contiguous()).transpose(0, 1).reshape(tq, d))


def attention(w: dict, x, context=None, pe=None, k_pe=None, heads=32, eps=EPS):
    """Attention.__call__ (attention.py:528-603)."""
    context = x if context is None else context
    g = bf(2.0 * bf(torch.sigmoid(_proj(w, "to_gate_logits", x))))
    v = _proj(w, "to_v", context)
    q = _proj(w, "to_q", x)
    k = _proj(w, "to_k", context)
    q = bf(q * rms_inv(q, eps) * w["q_norm"])
    k = bf(k * rms_inv(k, eps) * w["k_norm"])
    if pe is not None:
        q = rope(q, pe[0], pe[1], heads)
        kp = pe if k_pe is None else k_pe
        k = rope(k, kp[0], kp[1], heads)
    o = sdpa(q, k, v, heads)
    t, d = o.shape
    o = bf(o.view(t, heads, d // heads) * g[:, :, None]).reshape(t, d)
    return _proj(w, "to_out", o)


def feed_forward(w: dict, x):
    h = bf(gelu_tanh(linear(x, w["w1"], w["b1"], w.get("w1_qlinear", False))))
    return linear(h, w["w2"], w["b2"], w.get("w2_qlinear", False))


def block(W: dict, vx, ax, v_ada, a_ada, vctx, actx, vpe, vxpe, ape, axpe, *, fused_adaln=False, eps=EPS,
          skips=frozenset()):
    """BasicAVTransformerBlock.__call__ (transformer.py:389-674) on 2-D
    streams; ``*_ada`` are the (16, D) modulation rows
    [sst(9) | prompt(2) | av(5)] + timestep rows, or (16, T, D) per video
    token (per-token timesteps; the prompt rows are then the sample's on
    every token).  ``skips`` holds the
    perturbation kinds applying to this block ("skip_video_self_attn",
    "skip_audio_self_attn", "skip_a2v_cross_attn", "skip_v2a_cross_attn"):
    the sub-layer's whole residual update is skipped (transformer.py:430-470,
    :576-625)."""
    r = v_ada
    vh, ah = 32, 32
    if vx is not None:
        if "skip_video_self_attn" not in skips:
            h = adaln(vx, r[1], r[0], eps, fused_adaln)
            vx = bf(vx + attention(W["attn1"], h, pe=vpe, heads=vh) * r[2])
        a = adaln(vx, r[7], r[6], eps)
        # the context's prompt rows belong to the sample, not to a video token
        # (per-token rows (16, T, D) carry the same prompt rows on every token)
        pk = r[:, 0] if r.dim() == 3 else r
        c = bf(vctx * (1 + pk[10]) + pk[9])
        vx = bf(vx + bf(attention(W["attn2"], a, c, heads=vh) * r[8]))
    if ax is not None:
        q = a_ada
        if "skip_audio_self_attn" not in skips:
            h = adaln(ax, q[1], q[0], eps, fused_adaln)
            ax = bf(ax + attention(W["audio_attn1"], h, pe=ape, heads=ah) * q[2])
        a = adaln(ax, q[7], q[6], eps)
        c = bf(actx * (1 + q[10]) + q[9])
        ax = bf(ax + bf(attention(W["audio_attn2"], a, c, heads=ah) * q[8]))
    if vx is not None and ax is not None:
        vn, an = rms_norm_bf(vx, eps), rms_norm_bf(ax, eps)
        q = a_ada
        if "skip_a2v_cross_attn" not in skips:
            vs = bf(vn * (1 + r[11]) + r[12])
            as_ = bf(an * (1 + q[11]) + q[12])
            vx = bf(vx + attention(W["audio_to_video_attn"], vs, as_, pe=vxpe, k_pe=axpe, heads=ah) * r[15])
        if "skip_v2a_cross_attn" not in skips:
            as2 = bf(an * (1 + q[13]) + q[14])
            vs2 = bf(vn * (1 + r[13]) + r[14])
            ax = bf(ax + attention(W["video_to_audio_attn"], as2, vs2, pe=axpe, k_pe=vxpe, heads=ah) * q[15])
    if vx is not None:
        h = adaln(vx, r[4], r[3], eps, fused_adaln)
        vx = bf(vx + feed_forward(W["ff"], h) * r[5])
    if ax is not None:
        q = a_ada
        h = adaln(ax, q[4], q[3], eps, fused_adaln)
        ax = bf(ax + feed_forward(W["audio_ff"], h) * q[5])
    return vx, ax


# ---- step glue -------------------------------------------------------------
def timestep_sinusoid(t: float, dim: int = 256) -> torch.Tensor:
    """get_timestep_embedding(flip_sin_to_cos=True, shift=0) in float64 args."""
    half = dim // 2
    i = torch.arange(half, dtype=torch.float32)
    expo = (torch.tensor(-math.log(10000.0), dtype=torch.float32) * i) / half
    arg = torch.tensor(t, dtype=torch.float32) * torch.exp(expo.double()).float()
    arg = arg.double()
    return torch.cat([torch.cos(arg), torch.sin(arg)]).float()


def adaln_mlp(w: dict, t: float):
    """AdaLayerNormSingle (timestep_embedding.py:165-201) in fp32 with bf16
    weights -> (emb (N*D), embedded_timestep (D))."""
    s = timestep_sinusoid(t)
    h = torch.nn.functional.silu(s @ w["w1"].T + w["b1"])
    e = h @ w["w2"].T + w["b2"]
    return torch.nn.functional.silu(e) @ w["w"].T + w["b"], e


def output_head(x, table, emb, w, b, eps=EPS):
    """model.py:1312-1326: bf16 arithmetic modulation, then proj_out; ``emb``
    (D) or per token (T, D)."""
    ss = bf(table + emb[None, :]) if emb.dim() == 1 else bf(table[:, None, :] + emb[None])
    shift, scale = ss[0], ss[1]
    mu = x.double().mean(-1, keepdim=True)
    var = (x.double() - mu).square().mean(-1, keepdim=True)
    n = bf(((x.double() - mu) / torch.sqrt(var + eps)).float())
    y = bf(bf(n * bf(1 + scale)) + shift)
    return linear(y, w, b)


def euler_x0(latent, velocity, sigma: float, sigma_next: float):
    """model.py:1519-1525 + diffusion_steps.py:58-69 in fp32."""
    s = torch.tensor(sigma, dtype=torch.float32)
    ratio = torch.tensor(sigma_next / sigma, dtype=torch.float32)
    x0 = latent - s * velocity
    return bf(x0 + ratio * (latent - x0))


def model_velocity(MW: dict, vlat, alat, vctx, actx, sigma: float, pes, *, av_ca_mult=1000.0, ts_mult=1000.0,
                   eps=EPS, skips=None, video_token_sigmas=None):
    """LTXModel.__call__ (model.py:1344-1486): (video velocity, audio velocity)
    bf16 values.  ``skips(block_index) -> set of perturbation kinds``.

    ``video_token_sigmas`` (T,): per-token video timesteps (model.py:160-187,
    :418-497 -- the image-conditioned denoise mask): the video AdaLN rows 0-8,
    the cross scale / shift rows 11-14 and the output head's embedded
    timestep follow each token's value; the prompt rows and both cross gates
    keep ``sigma`` (each modality's sample sigma).  The blocks then see
    (16, T, D) modulation rows, broadcast per token.

    MW: {"patchify": (w, b), "audio_patchify": (w, b), "mlps_v": [4 mlp dicts],
    "mlps_a": [...], "tables_v": (L, 16, D), "tables_a": ..., "blocks": [block
    dicts], "sst_out_v": (2, D), "proj_out_v": (w, b), ...}.
    """
    vpe, vxpe, ape, axpe = pes
    t = sigma * ts_mult
    vx = linear(vlat, *MW["patchify"])
    ax = linear(alat, *MW["audio_patchify"]) if alat is not None else None

    def temb(mlps, d):
        e9, emb = adaln_mlp(mlps[0], t)
        e2, _ = adaln_mlp(mlps[1], t)
        e4, _ = adaln_mlp(mlps[2], t)
        e1, _ = adaln_mlp(mlps[3], sigma * av_ca_mult)
        return torch.cat([e9, e2, e4, e1]).view(16, d), emb

    tv, emb_v = temb(MW["mlps_v"], vx.shape[1])
    ta, emb_a = temb(MW["mlps_a"], ax.shape[1]) if ax is not None else (None, None)
    if video_token_sigmas is not None:
        ts_tok = torch.as_tensor(video_token_sigmas, dtype=torch.float32).reshape(-1)
        d = vx.shape[1]
        rows = tv[:, None, :].repeat(1, ts_tok.numel(), 1)  # prompt rows and the gate: the sample's
        emb_tok = emb_v[None, :].repeat(ts_tok.numel(), 1)
        for u in torch.unique(ts_tok).tolist():
            sel = ts_tok == u
            e9, emb_u = adaln_mlp(MW["mlps_v"][0], u * ts_mult)
            e4, _ = adaln_mlp(MW["mlps_v"][2], u * ts_mult)
            rows[0:9, sel] = e9.view(9, 1, d)
            rows[11:15, sel] = e4.view(4, 1, d)
            emb_tok[sel] = emb_u
        tv, emb_v = rows, emb_tok
    for i, W in enumerate(MW["blocks"]):
        v_ada = (MW["tables_v"][i][:, None, :] if tv.dim() == 3 else MW["tables_v"][i]) + tv
        a_ada = MW["tables_a"][i] + ta if ax is not None else None
        vx, ax = block(W, vx, ax, v_ada, a_ada, vctx, actx, vpe, vxpe, ape, axpe, eps=eps,
                       skips=frozenset() if skips is None else frozenset(skips(i)))
    vvel = output_head(vx, MW["sst_out_v"], emb_v, *MW["proj_out_v"], eps=eps)
    avel = output_head(ax, MW["sst_out_a"], emb_a, *MW["proj_out_a"], eps=eps) if ax is not None else None
    return vvel, avel


def model_step(MW: dict, vlat, alat, vctx, actx, sigma: float, sigma_next: float, pes, *, av_ca_mult=1000.0,
               ts_mult=1000.0, eps=EPS):
    """One distilled AV denoise step: LTXModel.__call__ (model.py:1344-1486)
    + X0Model (:1489-1542) + Euler (diffusion_steps.py:58-69)."""
    vvel, avel = model_velocity(MW, vlat, alat, vctx, actx, sigma, pes, av_ca_mult=av_ca_mult, ts_mult=ts_mult,
                                eps=eps)
    new_v = euler_x0(vlat, vvel, sigma, sigma_next)
    new_a = euler_x0(alat, avel, sigma, sigma_next) if avel is not None else None
    return new_v, new_a
