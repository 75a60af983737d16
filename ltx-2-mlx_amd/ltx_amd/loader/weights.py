"""Resident weights of the transformer: random initialisation in the three
weight formats, laid out for the fused kernels.

The reference loads real checkpoints through its transformer cache
(loader/transformer_cache.py); the benchmarked configurations here are
random-init (no checkpoints are available offline), drawn as documented for
them: linear weights ~N(0, 0.02) bf16 with zero biases, RMSNorm weights 1,
AdaLN tables ~N(0, 0.02) fp32.

Fused projection layouts (rows of the (N, K) weight):
  self-attention  [to_q; to_k; to_v; to_gate_logits]
  cross-attention [to_q; to_gate_logits]  and  [to_k; to_v]
Quantised formats quantise each output row on its own (MXFP8 blocks run along
K), so a fused weight quantises bit-identically to its separate projections.
"""

from __future__ import annotations

import torch

from ..kernels import gemm
from ..model.transformer.attention import Attention
from ..model.transformer.feed_forward import FeedForward

WEIGHT_STD = 0.02


def _randn(shape, gen, device, std=WEIGHT_STD, dtype=torch.bfloat16):
    return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)


def linear_weight(n: int, k: int, *, gen, device, weight_format: str, bias: bool = True) -> gemm.LinearWeight:
    w = _randn((n, k), gen, device)
    b = torch.zeros(n, dtype=torch.float32, device=device) if bias else None
    out = gemm.make_weight(w, b, kind=weight_format)
    if weight_format != "bf16":
        del w
    return out


def build_attention(query_dim: int, context_dim: int | None, heads: int, dim_head: int, *, gen, device,
                    weight_format: str, norm_eps: float = 1e-6) -> Attention:
    inner = heads * dim_head
    kdim = query_dim if context_dim is None else context_dim
    if context_dim is None:
        proj_q = linear_weight(3 * inner + heads, query_dim, gen=gen, device=device, weight_format=weight_format)
        proj_kv = None
    else:
        proj_q = linear_weight(inner + heads, query_dim, gen=gen, device=device, weight_format=weight_format)
        proj_kv = linear_weight(2 * inner, kdim, gen=gen, device=device, weight_format=weight_format)
    to_out = linear_weight(query_dim, inner, gen=gen, device=device, weight_format=weight_format)
    ones = torch.ones(inner, dtype=torch.float32, device=device)
    return Attention(query_dim, context_dim, heads, dim_head, proj_q, proj_kv, to_out, ones, ones.clone(),
                     norm_eps=norm_eps)


def build_ff(dim: int, mult: int = 4, *, gen, device, weight_format: str) -> FeedForward:
    return FeedForward(linear_weight(dim * mult, dim, gen=gen, device=device, weight_format=weight_format),
                       linear_weight(dim, dim * mult, gen=gen, device=device, weight_format=weight_format))


def build_block(video_config, audio_config, *, device="cuda", weight_format: str = "bf16",
                generator: torch.Generator | None = None, norm_eps: float = 1e-6,
                video_tables: torch.Tensor | None = None, audio_tables: torch.Tensor | None = None) -> dict:
    """Random weights of one BasicAVTransformerBlock (transformer.py:192-284)."""
    gen = generator
    if gen is None:
        gen = torch.Generator(device=device)
        gen.manual_seed(0)
    w: dict = {}
    kw = dict(gen=gen, device=device, weight_format=weight_format, norm_eps=norm_eps)
    if video_config is not None:
        vc = video_config
        w["attn1"] = build_attention(vc.dim, None, vc.heads, vc.d_head, **kw)
        w["attn2"] = build_attention(vc.dim, vc.context_dim, vc.heads, vc.d_head, **kw)
        w["ff"] = build_ff(vc.dim, gen=gen, device=device, weight_format=weight_format)
        t = _randn((16, vc.dim), gen, device, dtype=torch.float32)
        if video_tables is not None:
            video_tables.copy_(t)
            t = video_tables
        w["video_tables"] = t
    if audio_config is not None:
        ac = audio_config
        w["audio_attn1"] = build_attention(ac.dim, None, ac.heads, ac.d_head, **kw)
        w["audio_attn2"] = build_attention(ac.dim, ac.context_dim, ac.heads, ac.d_head, **kw)
        w["audio_ff"] = build_ff(ac.dim, gen=gen, device=device, weight_format=weight_format)
        t = _randn((16, ac.dim), gen, device, dtype=torch.float32)
        if audio_tables is not None:
            audio_tables.copy_(t)
            t = audio_tables
        w["audio_tables"] = t
    if video_config is not None and audio_config is not None:
        vc, ac = video_config, audio_config
        # Q from video (dim 4096) / K,V from audio (2048), audio heads (transformer.py:259-267)
        w["audio_to_video_attn"] = build_attention(vc.dim, ac.dim, ac.heads, ac.d_head, **kw)
        # Q from audio / K,V from video (:270-278)
        w["video_to_audio_attn"] = build_attention(ac.dim, vc.dim, ac.heads, ac.d_head, **kw)
    return w
