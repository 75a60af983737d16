"""Positions and RoPE cos/sin tables (built once per stage on the host).

Follows the reference's LTX-2.3 setting: float64 frequency grid
(rope.py:92-133, ``use_double_precision``), middle-of-patch fractional
positions mapped to [-1, 1] (rope.py:169-244), split layout with front
identity padding (rope.py:247-336).  Positions come from the patch bounds of
components/patchifiers.py:127-218 (video, causal time fix, seconds) and
:233-287 (audio).

Tables are token-major fp32 (T, D/2): the reference's (1, H, T, dh/2) tensor
reshaped (T, H, dh/2) -- the layout the QK-norm + RoPE kernel reads -- or
that table factored over the position axes (a few rows per axis and a row
index per token and axis), which the kernel recombines exactly.  The
reference recomputes them every step unless ``LTX_ROPE_PRECOMPUTE`` is set;
positions are fixed for a stage, so this build computes them once.
"""

from __future__ import annotations

import math
from enum import Enum

import numpy as np
import torch

VIDEO_MAX_POS = (20, 2048, 2048)
AUDIO_MAX_POS = (20,)
SCALE_FACTORS = (8, 32, 32)  # time, height, width (types.py:36-41)


class LTXRopeType(Enum):
    SPLIT = "split"


def freq_grid(theta: float, n_pos_dims: int, inner_dim: int) -> np.ndarray:
    n = inner_dim // (2 * n_pos_dims)
    if n <= 0:
        return np.zeros((0,), np.float32)
    e = np.linspace(0.0, 1.0, n, dtype=np.float64)
    return (np.power(np.float64(theta), e) * (math.pi / 2)).astype(np.float32)


def video_positions(frames: int, height: int, width: int, fps: float, causal_fix: bool = True) -> np.ndarray:
    """(1, 3, T, 2) float32 patch bounds in (seconds, pixel y, pixel x)."""
    f, h, w = np.meshgrid(np.arange(frames), np.arange(height), np.arange(width), indexing="ij")
    starts = np.stack([f, h, w], 0).reshape(3, -1).astype(np.int64)
    bounds = np.stack([starts, starts + 1], -1)
    pix = bounds * np.array(SCALE_FACTORS, np.int64).reshape(3, 1, 1)
    if causal_fix:
        pix[0] = np.maximum(pix[0] + 1 - SCALE_FACTORS[0], 0)
    pos = pix.astype(np.float32)
    pos[0] = (pos[0] / np.float32(fps)).astype(np.float32)
    return pos[None]


def audio_positions(num_steps: int, shift: int = 0, hop_length: int = 160, sample_rate: int = 16000,
                    downsample: int = 4, causal: bool = True) -> np.ndarray:
    """(1, 1, T, 2) float32 start/end seconds of audio latent frames."""

    def secs(a: int, b: int) -> np.ndarray:
        mel = (np.arange(a, b).astype(np.float32) * np.float32(downsample)).astype(np.float32)
        if causal:
            mel = np.maximum((mel + np.float32(1 - downsample)).astype(np.float32), np.float32(0))
        return ((mel * np.float32(hop_length)).astype(np.float32) / np.float32(sample_rate)).astype(np.float32)

    return np.stack([secs(shift, num_steps + shift), secs(shift + 1, num_steps + shift + 1)], -1)[None, None]


def rope_tables_np(positions: np.ndarray, dim: int, max_pos, theta: float = 10000.0) -> tuple[np.ndarray, np.ndarray]:
    """Token-major (T, dim/2) fp32 cos/sin for batch 0 of ``positions``."""
    n_dims = positions.shape[1]
    idx = freq_grid(theta, n_dims, dim)
    mid = ((positions[0, :, :, 0] + positions[0, :, :, 1]).astype(np.float32) / np.float32(2.0)).astype(np.float32)
    frac = np.stack([(mid[d] / np.float32(max_pos[d])).astype(np.float32) for d in range(n_dims)], -1)
    scaled = ((frac * np.float32(2)).astype(np.float32) - np.float32(1)).astype(np.float32)  # (T, n_dims)
    freqs = (idx[None, None, :] * scaled[:, :, None]).astype(np.float32)  # (T, n_dims, n_freq)
    freqs = freqs.transpose(0, 2, 1).reshape(freqs.shape[0], -1).astype(np.float64)
    pad = dim // 2 - freqs.shape[-1]
    cos = np.cos(freqs).astype(np.float32)
    sin = np.sin(freqs).astype(np.float32)
    if pad:
        cos = np.concatenate([np.ones((cos.shape[0], pad), np.float32), cos], -1)
        sin = np.concatenate([np.zeros((sin.shape[0], pad), np.float32), sin], -1)
    return np.ascontiguousarray(cos), np.ascontiguousarray(sin)


def factor_tables_np(positions: np.ndarray, cos: np.ndarray, sin: np.ndarray):
    """Token-major tables factored over the position axes, or None if that
    saves nothing.

    Column c of a (T, D/2) table depends on one axis only: the identity pad
    columns and, after them, frequency f of axis (c - pad) % n_dims.  For
    each axis the distinct (start, end) bounds give the distinct rows; the
    factored form stacks, per axis, one row per distinct bound holding that
    axis' columns (axis 0 also the pad columns) and exactly 1 / -0 in every
    other column, plus idx (T, n_dims) int32 rows into the stack.  The token
    row is cos = prod_a cos_f[idx[t, a]], sin = sum_a sin_f[idx[t, a]] in
    axis order -- bit-identical to the full table (x * 1 = x and x + -0 = x
    for every float), which is checked here before the form is used.
    """
    n_dims = positions.shape[1]
    t, half = cos.shape
    pad = half - (half // n_dims) * n_dims
    col_axis = np.zeros(half, np.int64)
    col_axis[pad:] = np.arange(half - pad) % n_dims
    reps, inv = [], []
    for a in range(n_dims):
        _, first, inverse = np.unique(positions[0, a], axis=0, return_index=True, return_inverse=True)
        reps.append(first)
        inv.append(inverse.reshape(-1))
    rows = sum(len(r) for r in reps)
    if rows >= t:
        return None
    cos_f = np.ones((rows, half), np.float32)
    sin_f = np.full((rows, half), -0.0, np.float32)
    idx = np.empty((t, n_dims), np.int32)
    off = 0
    for a in range(n_dims):
        cols = col_axis == a
        cos_f[off:off + len(reps[a])][:, cols] = cos[reps[a]][:, cols]
        sin_f[off:off + len(reps[a])][:, cols] = sin[reps[a]][:, cols]
        idx[:, a] = off + inv[a]
        off += len(reps[a])
    c_exp, s_exp = expand_tables_np(cos_f, sin_f, idx)
    if not (np.array_equal(c_exp.view(np.uint32), cos.view(np.uint32))
            and np.array_equal(s_exp.view(np.uint32), sin.view(np.uint32))):
        return None
    return cos_f, sin_f, idx


def expand_tables_np(cos_f: np.ndarray, sin_f: np.ndarray, idx: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-token (T, D/2) tables of a factored form, combined in the order the
    QK-norm + RoPE kernel uses (fp32 products and sums, axis 0 first)."""
    c = cos_f[idx[:, 0]].copy()
    s = sin_f[idx[:, 0]].copy()
    for a in range(1, idx.shape[1]):
        c = (c * cos_f[idx[:, a]]).astype(np.float32)
        s = (s + sin_f[idx[:, a]]).astype(np.float32)
    return c, s


def rope_tables(positions: np.ndarray, dim: int, max_pos, device, theta: float = 10000.0,
                factored: bool = False) -> tuple:
    """Device tables: (cos, sin) token-major, or with ``factored`` the
    (cos_f, sin_f, idx) form of :func:`factor_tables_np` when it is smaller."""
    cos, sin = rope_tables_np(positions, dim, max_pos, theta)
    if factored:
        f = factor_tables_np(positions, cos, sin)
        if f is not None:
            return tuple(torch.from_numpy(a).to(device) for a in f)
    return torch.from_numpy(cos).to(device), torch.from_numpy(sin).to(device)


def expand_tables(pe: tuple) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) per-token CPU tables of either device form."""
    if len(pe) == 2:
        return pe[0].cpu(), pe[1].cpu()
    c, s = expand_tables_np(*(a.cpu().numpy() for a in pe))
    return torch.from_numpy(c), torch.from_numpy(s)
