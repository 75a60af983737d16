"""Positions and RoPE cos/sin tables (built once per stage on the host).

Follows the reference's LTX-2.3 setting: float64 frequency grid
(rope.py:92-133, ``use_double_precision``), middle-of-patch fractional
positions mapped to [-1, 1] (rope.py:169-244), split layout with front
identity padding (rope.py:247-336).  Positions come from the patch bounds of
components/patchifiers.py:127-218 (video, causal time fix, seconds) and
:233-287 (audio).

Tables are token-major fp32 (T, D/2): the reference's (1, H, T, dh/2) tensor
reshaped (T, H, dh/2) -- the layout the QK-norm + RoPE kernel reads.  The
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


def rope_tables(positions: np.ndarray, dim: int, max_pos, device, theta: float = 10000.0) -> tuple[torch.Tensor, torch.Tensor]:
    cos, sin = rope_tables_np(positions, dim, max_pos, theta)
    return torch.from_numpy(cos).to(device), torch.from_numpy(sin).to(device)
