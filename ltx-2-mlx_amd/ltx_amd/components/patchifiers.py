"""Latent shapes and token counts (types.py:44-157, patchifiers.py)."""

from __future__ import annotations

import math

VIDEO_SCALE = (8, 32, 32)  # time, height, width
NATIVE_FPS = 24.0


def video_latent_grid(height: int, width: int, frames: int) -> tuple[int, int, int]:
    """(frames, h, w) latent grid of a pixel shape (types.py:75-90)."""
    return (frames - 1) // VIDEO_SCALE[0] + 1, height // VIDEO_SCALE[1], width // VIDEO_SCALE[2]


def audio_latent_frames(frames: int, fps: float = NATIVE_FPS, sample_rate: int = 16000, hop_length: int = 160,
                        downsample: int = 4) -> int:
    """ceil(duration * latents_per_second) (types.py:118-157)."""
    per_second = float(sample_rate) / float(hop_length) / float(downsample)
    return math.ceil(float(frames) / float(fps) * per_second)
