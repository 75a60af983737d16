"""Gemma feature extractor V2 (model/text_encoder/feature_extractor.py:9-79).

The hidden states of the ``num_layers`` Gemma layers are RMS-normalised per
token and per layer over ``hidden_dim``, padding tokens zeroed, scaled by
sqrt(inner_dim / hidden_dim) and projected by one linear per modality to the
transformer's widths (4096 video, 2048 audio).  The normalisation runs in
``ltx_gemma_features_bf16`` with the reference's bf16 rounding points; the
projections in the bf16 GEMM.  The features are laid out layer-major (index
l * hidden_dim + d), so the projection weights are stored with their input
columns permuted from the checkpoint's d * num_layers + l order
(``permute_aggregate_weight``).
"""

from __future__ import annotations

import math

import torch

from ... import _lib
from ...kernels import gemm
from ...loader.weights import linear_weight


def _bf16_value(v: float) -> float:
    return float(torch.tensor(v, dtype=torch.float32).bfloat16().float())


def permute_aggregate_weight(w: torch.Tensor, hidden_dim: int, num_layers: int) -> torch.Tensor:
    """(N, D*L) columns in the reference's d*L + l order -> l*D + d order."""
    n = w.shape[0]
    return w.reshape(n, hidden_dim, num_layers).transpose(1, 2).reshape(n, num_layers * hidden_dim).contiguous()


class GemmaFeaturesExtractorV2:
    def __init__(self, hidden_dim: int = 3840, num_layers: int = 49, video_inner_dim: int = 4096,
                 audio_inner_dim: int = 2048, *, device="cuda", init: str = "random", seed: int = 0):
        self.hidden_dim = hidden_dim
        self.num_layers = num_layers
        self.embedding_dim = hidden_dim
        flat = hidden_dim * num_layers
        gen = None
        if init == "random":
            gen = torch.Generator(device=device)
            gen.manual_seed(seed)
        # layer-major input columns (see the module docstring)
        self.video_aggregate_embed = linear_weight(video_inner_dim, flat, gen=gen, device=device,
                                                   weight_format="bf16", init=init)
        self.audio_aggregate_embed = linear_weight(audio_inner_dim, flat, gen=gen, device=device,
                                                   weight_format="bf16", init=init)

    def extract_from_hidden_states(self, hidden_states, attention_mask: torch.Tensor | None,
                                   padding_side: str = "left"):
        """``hidden_states``: list of ``num_layers`` (1, T, D) / (T, D) bf16
        tensors, or one (L, T, D) tensor; ``attention_mask`` (1, T) / (T,)
        binary.  Returns (video (1, T, 4096), audio (1, T, 2048)) bf16."""
        if isinstance(hidden_states, (list, tuple)):
            hs = torch.stack([h.reshape(h.shape[-2], h.shape[-1]) for h in hidden_states], 0)
        else:
            hs = hidden_states
        hs = hs.to(torch.bfloat16).contiguous()
        L, T, D = hs.shape
        if L != self.num_layers or D != self.hidden_dim:
            raise ValueError(f"expected {self.num_layers} layers of width {self.hidden_dim}, got {tuple(hs.shape)}")
        mask = None
        if attention_mask is not None:
            mask = attention_mask.reshape(-1).to(device=hs.device, dtype=torch.int32).contiguous()
            if mask.numel() != T:
                raise ValueError("attention mask length differs from the token count")
        v_dim = self.video_aggregate_embed.out_features
        a_dim = self.audio_aggregate_embed.out_features
        sv = _bf16_value(math.sqrt(v_dim / self.embedding_dim))
        sa = _bf16_value(math.sqrt(a_dim / self.embedding_dim))
        fv = torch.empty((T, L * D), dtype=torch.bfloat16, device=hs.device)
        fa = torch.empty_like(fv)
        _lib.call("ltx_gemma_features_bf16", _lib.ptr(hs), L, T, D, T * D, D, _lib.ptr(mask),
                  _bf16_value(1e-6), sv, sa, _lib.ptr(fv), _lib.ptr(fa), L * D, _lib.stream_of(hs))
        video = gemm.linear(fv, self.video_aggregate_embed)
        audio = gemm.linear(fa, self.audio_aggregate_embed)
        return video[None], audio[None]
