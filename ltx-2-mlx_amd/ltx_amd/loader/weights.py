"""Resident weights of the transformer: random initialisation in the three
weight formats, laid out for the fused kernels.

The reference loads real checkpoints through its transformer cache
(loader/transformer_cache.py); the benchmarked configurations here are
random-init (no checkpoints are available offline), drawn as documented for
them: linear weights ~N(0, 0.02) bf16 with zero biases, RMSNorm weights 1,
AdaLN tables ~N(0, 0.02) fp32.  ``init="empty"`` allocates the same storage
uninitialised for the checkpoint / cache loaders (loader.resident).

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


def linear_weight(n: int, k: int, *, gen, device, weight_format: str, bias: bool = True,
                  init: str = "random") -> gemm.LinearWeight:
    """A resident (N, K) projection: random (``init="random"``) or
    uninitialised storage of the format, to be filled by a loader
    (``init="empty"``)."""
    if init == "empty":
        b = torch.zeros(n, dtype=torch.float32, device=device) if bias else None
        if weight_format == "bf16":
            return gemm.LinearWeight("bf16", torch.empty((n, k), dtype=torch.bfloat16, device=device), None, b)
        if weight_format == "int8":
            return gemm.LinearWeight("int8", torch.empty((n, k), dtype=torch.int8, device=device),
                                     torch.empty((n,), dtype=torch.float32, device=device), b)
        if weight_format == "mxfp8":
            return gemm.LinearWeight("mxfp8", torch.empty((n, k), dtype=torch.uint8, device=device),
                                     torch.empty((n, k // 32), dtype=torch.uint8, device=device), b, qlinear=True)
        raise ValueError(f"unknown weight format {weight_format!r}")
    if init != "random":
        raise ValueError(f"init must be 'random' or 'empty', got {init!r}")
    w = _randn((n, k), gen, device)
    b = torch.zeros(n, dtype=torch.float32, device=device) if bias else None
    out = gemm.make_weight(w, b, kind=weight_format)
    if weight_format != "bf16":
        del w
    return out


def build_attention(query_dim: int, context_dim: int | None, heads: int, dim_head: int, *, gen, device,
                    weight_format: str, norm_eps: float = 1e-6, init: str = "random") -> Attention:
    inner = heads * dim_head
    kdim = query_dim if context_dim is None else context_dim
    kw = dict(gen=gen, device=device, weight_format=weight_format, init=init)
    if context_dim is None:
        proj_q = linear_weight(3 * inner + heads, query_dim, **kw)
        proj_kv = None
    else:
        proj_q = linear_weight(inner + heads, query_dim, **kw)
        proj_kv = linear_weight(2 * inner, kdim, **kw)
    to_out = linear_weight(query_dim, inner, **kw)
    ones = torch.ones(inner, dtype=torch.float32, device=device)
    return Attention(query_dim, context_dim, heads, dim_head, proj_q, proj_kv, to_out, ones, ones.clone(),
                     norm_eps=norm_eps)


def build_ff(dim: int, mult: int = 4, *, gen, device, weight_format: str, init: str = "random") -> FeedForward:
    kw = dict(gen=gen, device=device, weight_format=weight_format, init=init)
    return FeedForward(linear_weight(dim * mult, dim, **kw), linear_weight(dim, dim * mult, **kw))


def build_block(video_config, audio_config, *, device="cuda", weight_format: str = "bf16",
                generator: torch.Generator | None = None, norm_eps: float = 1e-6,
                video_tables: torch.Tensor | None = None, audio_tables: torch.Tensor | None = None,
                init: str = "random") -> dict:
    """Weights of one BasicAVTransformerBlock (transformer.py:192-284):
    random, or uninitialised storage for a loader (``init="empty"``)."""
    gen = generator
    if gen is None and init == "random":
        gen = torch.Generator(device=device)
        gen.manual_seed(0)
    w: dict = {}
    kw = dict(gen=gen, device=device, weight_format=weight_format, norm_eps=norm_eps, init=init)
    fkw = dict(gen=gen, device=device, weight_format=weight_format, init=init)

    def table(d, dst):
        t = (_randn((16, d), gen, device, dtype=torch.float32) if init == "random"
             else torch.zeros((16, d), dtype=torch.float32, device=device))
        if dst is not None:
            dst.copy_(t)
            t = dst
        return t

    if video_config is not None:
        vc = video_config
        w["attn1"] = build_attention(vc.dim, None, vc.heads, vc.d_head, **kw)
        w["attn2"] = build_attention(vc.dim, vc.context_dim, vc.heads, vc.d_head, **kw)
        w["ff"] = build_ff(vc.dim, **fkw)
        w["video_tables"] = table(vc.dim, video_tables)
    if audio_config is not None:
        ac = audio_config
        w["audio_attn1"] = build_attention(ac.dim, None, ac.heads, ac.d_head, **kw)
        w["audio_attn2"] = build_attention(ac.dim, ac.context_dim, ac.heads, ac.d_head, **kw)
        w["audio_ff"] = build_ff(ac.dim, **fkw)
        w["audio_tables"] = table(ac.dim, audio_tables)
    if video_config is not None and audio_config is not None:
        vc, ac = video_config, audio_config
        # Q from video (dim 4096) / K,V from audio (2048), audio heads (transformer.py:259-267)
        w["audio_to_video_attn"] = build_attention(vc.dim, ac.dim, ac.heads, ac.d_head, **kw)
        # Q from audio / K,V from video (:270-278)
        w["video_to_audio_attn"] = build_attention(ac.dim, vc.dim, ac.heads, ac.d_head, **kw)
    return w
