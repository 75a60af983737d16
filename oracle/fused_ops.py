"""Oracle for the bandwidth-bound row operators and the per-step glue.

All inputs are numpy float32 arrays whose values are bf16-representable where
the reference holds bf16 tensors; reductions run in float64 (the reference
accumulates in fp32; the difference is far below one bf16 ulp of the result).
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import bf16r


def rms_inv(x: np.ndarray, eps: float) -> np.ndarray:
    """rsqrt(mean(x^2) + eps) per row (mx.fast.rms_norm normaliser,
    kernels/fused_ops.py:132-163)."""
    x64 = x.astype(np.float64)
    return 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)


def adaln(x, scale, shift, eps: float = 1e-6, *, round_norm: bool = False, no_norm: bool = False):
    """AdaLN modulation.

    Fused kernel (kernels/fused_ops.py:163-176): out = bf16(x*inv*(1+scale)+shift).
    round_norm=True is the inline form ``(mx.fast.rms_norm(x) * (1 + scale) +
    shift).astype(bf16)`` (model/transformer/transformer.py:21-37, :374; and
    the fallback fused_ops.py:192-201) whose rms_norm output is bf16 first.
    no_norm=True is the context modulation ``(ctx*(1+scale)+shift).astype``
    (transformer.py:375).
    """
    x64 = np.asarray(x, dtype=np.float64)
    if no_norm:
        n = x64
    else:
        n = x64 * rms_inv(x, eps)
        if round_norm:
            n = bf16r(n).astype(np.float64)
    s = np.asarray(scale, dtype=np.float64)
    h = np.asarray(shift, dtype=np.float64)
    return bf16r(n * (1.0 + s) + h)


def gated_add(residual, branch, gate, *, round_product: bool = False):
    """out = bf16(residual + branch*gate) in fp32 (fused_ops.py:340-349,
    transformer.py:40-50).  round_product=True: the text cross-attention form
    ``vx + (attn_out*gate).astype(bf16)`` (transformer.py:387, :484)."""
    r = np.asarray(residual, dtype=np.float64)
    b = np.asarray(branch, dtype=np.float64)
    g = np.asarray(gate, dtype=np.float64)
    if round_product:
        return bf16r(r + bf16r(b * g).astype(np.float64))
    return bf16r(r + b * g)


def rms_norm_weighted(x, w, eps: float = 1e-6):
    """``RMSNorm.__call__`` (model/transformer/attention.py:320-329):
    bf16(x * rsqrt(mean(x^2)+eps) * w) with fp32 weight."""
    x64 = np.asarray(x, dtype=np.float64)
    return bf16r(x64 * rms_inv(x, eps) * np.asarray(w, dtype=np.float64))


def layer_norm_bf16(x, eps: float = 1e-6):
    """``nn.LayerNorm(affine=False)`` on bf16 x: bf16((x-mean)/sqrt(var+eps))."""
    x64 = np.asarray(x, dtype=np.float64)
    mu = x64.mean(axis=-1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=-1, keepdims=True)
    return bf16r((x64 - mu) / np.sqrt(var + eps))


def output_norm_modulate(x, table, emb, eps: float = 1e-6):
    """Output head before proj_out (model/transformer/model.py:1312-1326):
    ss = bf16(table + emb); out = norm_out(x) * (1 + scale) + shift, all in
    bf16 arithmetic (every op rounds to bf16)."""
    ss = bf16r(np.asarray(table, np.float32) + np.asarray(emb, np.float32)[None, :])
    shift, scale = ss[0], ss[1]
    n = layer_norm_bf16(x, eps)
    ops = bf16r(1.0 + scale)
    return bf16r(bf16r(n * ops) + shift)


def euler_x0_step(latent, velocity, sigma: float, sigma_next: float):
    """X0 (model.py:1510-1525) then Euler (components/diffusion_steps.py:58-69),
    in fp32 with each product and sum rounded (numpy float32 arithmetic)."""
    l = np.asarray(latent, np.float32)
    v = np.asarray(velocity, np.float32)
    s = np.float32(sigma)
    ratio = np.float32(sigma_next / sigma)
    x0 = (l - (s * v).astype(np.float32)).astype(np.float32)
    return bf16r(x0 + (ratio * (l - x0).astype(np.float32)).astype(np.float32))


def timestep_embedding(values, dim: int = 256, multiplier: float = 1000.0):
    """get_timestep_embedding(t*multiplier, dim, flip_sin_to_cos=True,
    downscale_freq_shift=0) (timestep_embedding.py:9-59, :140-144), fp32
    argument construction, transcendental in float64."""
    half = dim // 2
    i = np.arange(half, dtype=np.float32)
    expo = (np.float32(-math.log(10000.0)) * i).astype(np.float32) / np.float32(half)
    freqs = np.exp(expo.astype(np.float64)).astype(np.float32)
    t = (np.asarray(values, np.float32) * np.float32(multiplier)).astype(np.float32)
    arg = (t[:, None] * freqs[None, :]).astype(np.float32).astype(np.float64)
    emb = np.concatenate([np.cos(arg), np.sin(arg)], axis=-1).astype(np.float32)
    if dim % 2:
        emb = np.pad(emb, [(0, 0), (0, 1)])
    return emb


def silu(v):
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def linear_f32(x, W, b=None, *, silu_in: bool = False, silu_out: bool = False):
    """fp32 Linear with bf16 weights (AdaLN MLP layers,
    timestep_embedding.py:111-123, :186-201)."""
    x64 = np.asarray(x, dtype=np.float64)
    if silu_in:
        x64 = silu(x64)
    y = x64 @ np.asarray(W, dtype=np.float64).T
    if b is not None:
        y = y + np.asarray(b, dtype=np.float64)
    if silu_out:
        y = silu(y)
    return y.astype(np.float32)
