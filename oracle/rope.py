"""Oracle for positions, RoPE tables and the split-RoPE rotation.

Follows model/transformer/rope.py (frequency grid :92-133, fractional
positions :169-244, split tables :247-336, rotation :37-89),
components/patchifiers.py (video bounds :127-218, audio timings :233-287) and
conditioning/tools.py:37-85 (seconds conversion).  Float32 steps are done in
numpy float32 in the reference's operation order; the float64 frequency grid
follows ``generate_freq_grid_float64_cpu`` (the LTX-2.3 setting).
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import bf16r

VIDEO_MAX_POS = (20, 2048, 2048)
AUDIO_MAX_POS = (20,)
SCALE_FACTORS = (8, 32, 32)  # (time, height, width), types.py:36-41


def freq_grid_f64(theta: float, n_pos_dims: int, inner_dim: int) -> np.ndarray:
    """rope.py:92-133: float32(theta ** linspace(0, 1, n) * pi/2), n = inner_dim // (2*n_pos_dims)."""
    n = inner_dim // (2 * n_pos_dims)
    if n <= 0:
        return np.zeros((0,), np.float32)
    e = np.linspace(0.0, 1.0, n, dtype=np.float64)
    return (np.power(np.float64(theta), e) * (math.pi / 2)).astype(np.float32)


def video_positions(frames: int, height: int, width: int, fps: float, causal_fix: bool = True) -> np.ndarray:
    """(1, 3, T, 2) float32 [start, end) bounds in (seconds, pixels, pixels)
    for a patch-size-1 latent grid (patchifiers.py:127-218, tools.py:62-76)."""
    f, h, w = np.meshgrid(np.arange(frames), np.arange(height), np.arange(width), indexing="ij")
    starts = np.stack([f, h, w], 0).reshape(3, -1).astype(np.int64)
    coords = np.stack([starts, starts + 1], -1)  # (3, T, 2), patch size (1,1,1)
    scale = np.array(SCALE_FACTORS, np.int64).reshape(3, 1, 1)
    pix = coords * scale
    if causal_fix:
        pix[0] = np.maximum(pix[0] + 1 - SCALE_FACTORS[0], 0)
    pos = pix.astype(np.float32)
    pos[0] = (pos[0] / np.float32(fps)).astype(np.float32)
    return pos[None]


def audio_positions(num_steps: int, shift: int = 0, hop_length: int = 160, sample_rate: int = 16000,
                    downsample: int = 4, causal: bool = True) -> np.ndarray:
    """(1, 1, T, 2) float32 start/end seconds (patchifiers.py:233-287)."""

    def secs(start: int, end: int) -> np.ndarray:
        frame = np.arange(start, end).astype(np.float32)
        mel = (frame * np.float32(downsample)).astype(np.float32)
        if causal:
            mel = np.maximum((mel + np.float32(1) - np.float32(downsample)).astype(np.float32), np.float32(0))
        return ((mel * np.float32(hop_length)).astype(np.float32) / np.float32(sample_rate)).astype(np.float32)

    s = secs(shift, num_steps + shift)
    e = secs(shift + 1, num_steps + shift + 1)
    return np.stack([s, e], -1)[None, None]


def fractional_freqs(indices: np.ndarray, positions: np.ndarray, max_pos) -> np.ndarray:
    """rope.py:197-244 with use_middle_indices_grid=True: (B, T, n_freq*n_dims)
    with entry [f*n_dims + d] = indices[f] * ((mid_d / max_pos[d]) * 2 - 1)."""
    mid = ((positions[..., 0] + positions[..., 1]).astype(np.float32) / np.float32(2.0)).astype(np.float32)
    n_dims = positions.shape[1]
    frac = np.stack([(mid[:, d, :] / np.float32(max_pos[d])).astype(np.float32) for d in range(n_dims)], -1)
    scaled = ((frac * np.float32(2)).astype(np.float32) - np.float32(1)).astype(np.float32)  # (B,T,n_dims)
    freqs = (indices[None, None, None, :] * scaled[..., None]).astype(np.float32)  # (B,T,n_dims,n_freq)
    freqs = freqs.transpose(0, 1, 3, 2)
    return freqs.reshape(freqs.shape[0], freqs.shape[1], -1)


def rope_tables(positions: np.ndarray, dim: int, heads: int, max_pos, theta: float = 10000.0):
    """Token-major cos/sin tables (T, dim/2) float32 for batch 0.

    Equivalent to precompute_freqs_cis (rope.py:286-336): cos/sin of the
    fractional freqs, front-padded with (1, 0) up to dim/2 entries; the
    reference's (1, H, T, dh/2) tensor is this table reshaped (T, H, dh/2)
    and transposed.  cos/sin are evaluated in float64 and rounded to fp32
    (the reference evaluates them in fp32 on the GPU).
    """
    n_dims = positions.shape[1]
    idx = freq_grid_f64(theta, n_dims, dim)
    fr = fractional_freqs(idx, positions, max_pos)[0].astype(np.float64)
    pad = dim // 2 - fr.shape[-1]
    cos = np.cos(fr).astype(np.float32)
    sin = np.sin(fr).astype(np.float32)
    if pad:
        cos = np.concatenate([np.ones((cos.shape[0], pad), np.float32), cos], -1)
        sin = np.concatenate([np.zeros((sin.shape[0], pad), np.float32), sin], -1)
    assert cos.shape[-1] == dim // 2 and (dim // 2) % heads == 0
    return np.ascontiguousarray(cos), np.ascontiguousarray(sin)


def apply_split_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, heads: int) -> np.ndarray:
    """Split RoPE (rope.py:37-89) on token-major x (T, heads*dh) with tables
    (T, heads*dh/2); fp32 arithmetic, bf16 output."""
    t, d = x.shape
    dh = d // heads
    xh = x.reshape(t, heads, dh).astype(np.float64)
    c = cos.reshape(t, heads, dh // 2).astype(np.float64)
    s = sin.reshape(t, heads, dh // 2).astype(np.float64)
    x1, x2 = xh[..., : dh // 2], xh[..., dh // 2:]
    out = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], -1)
    return bf16r(out.reshape(t, d))


def qknorm_rope(x: np.ndarray, w: np.ndarray, cos, sin, heads: int, eps: float = 1e-6) -> np.ndarray:
    """q_norm / k_norm (attention.py:578-579) then RoPE (:582-584)."""
    from .fused_ops import rms_norm_weighted

    n = rms_norm_weighted(x, w, eps)
    if cos is None:
        return n
    return apply_split_rope(n, cos, sin, heads)
