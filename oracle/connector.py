"""Oracle for the text conditioning after Gemma (test infrastructure only).

A CPU restatement of model/text_encoder/feature_extractor.py:9-79 (per-token
RMS normalisation of every Gemma layer in bf16 arithmetic, padding zeroed,
scaled by the bf16 value of sqrt(inner / hidden), one linear per modality) and
model/text_encoder/connector.py:12-281 (learnable registers appended to a
multiple of the register count of at least 1024 tokens, 1-D RoPE over the
token index, pre-norm self-attention and feed-forward blocks with bf16
residual adds, final RMSNorm), built on oracle.block's attention, feed-forward
and rms_norm.

Pinning (tests/test_oracle_connector.py): masked tokens give zero features;
each normalised layer row has mean square 1 up to bf16 rounding; the scale is
the bf16 rounding of sqrt(inner / hidden) (1.03125 for 4096 / 3840); register
row i of the extension is register i mod R and the original rows are kept;
with zero attention and feed-forward output projections a block reduces to
the identity.  The bf16 rounding points of the feature normalisation (power,
mean, rsqrt) follow the reference's bf16 array operations; MLX's own
reduction order and transcendental rounding are not reproducible here, so the
feature normalisation is parity unpinned below one bf16 ulp.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import block as ob
from .bf16 import bf16r


def _bf(x):
    return bf16r(np.asarray(x, np.float32))


def bf16_value(v: float) -> float:
    return float(bf16r(np.float32(v)))


def gemma_features(hidden, mask, scale: float, eps: float = 1e-6) -> np.ndarray:
    """hidden (L, T, D) bf16 values -> (T, L*D) layer-major features."""
    h = np.asarray(hidden, np.float32)
    L, T, D = h.shape
    sq = _bf(h * h)
    mean = _bf(sq.sum(-1, dtype=np.float64).astype(np.float32) / np.float32(D))  # (L, T)
    var = _bf(mean + np.float32(bf16_value(eps)))
    r = _bf(np.float32(1.0) / np.sqrt(var.astype(np.float64)).astype(np.float32))
    y = _bf(h * r[..., None])
    if mask is not None:
        y = y * (np.asarray(mask).reshape(1, T, 1) != 0)
    y = _bf(y * np.float32(bf16_value(scale)))
    return np.ascontiguousarray(y.transpose(1, 0, 2).reshape(T, L * D))


def aggregate_scale(inner: int, hidden: int) -> float:
    return math.sqrt(inner / hidden)


def extend_with_registers(x: torch.Tensor, registers: torch.Tensor) -> torch.Tensor:
    t = x.shape[0]
    r = registers.shape[0]
    total = math.ceil(max(1024, t) / r) * r
    if total == t:
        return x
    idx = torch.arange(t, total) % r
    return torch.cat([x, registers[idx]], 0)


def block1d(W: dict, x: torch.Tensor, pe, heads: int, eps: float = ob.EPS) -> torch.Tensor:
    h = ob.rms_norm_bf(x, eps)
    x = ob.bf(x + ob.attention(W["attn1"], h, pe=pe, heads=heads, eps=eps))
    h = ob.rms_norm_bf(x, eps)
    return ob.bf(x + ob.feed_forward(W["ff"], h))


def connector(Wc: dict, x: torch.Tensor, pe, heads: int, eps: float = ob.EPS) -> torch.Tensor:
    """Wc: {"registers": (R, D) or None, "blocks": [block dicts]}; x (T, D)."""
    if Wc.get("registers") is not None:
        x = extend_with_registers(x, Wc["registers"])
    for W in Wc["blocks"]:
        x = block1d(W, x, pe, heads, eps)
    return ob.rms_norm_bf(x, eps)
