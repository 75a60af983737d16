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


AUDIO_LATENT_CHANNELS = 8
AUDIO_MEL_BINS = 16


def _swap_axes(x, a: int, b: int, r: int, shape):
    """out[b, a, r] = in[a, b, r] on the device (``ltx_swap_axes``)."""
    import torch

    from .. import _lib

    x = x.contiguous()
    if x.numel() != a * b * r:
        raise ValueError(f"{tuple(x.shape)} does not hold ({a}, {b}, {r}) elements")
    out = torch.empty(shape, dtype=x.dtype, device=x.device)
    _lib.call("ltx_swap_axes", _lib.ptr(x), a, b, r, x.element_size(), _lib.ptr(out), _lib.stream_of(x))
    return out


class VideoLatentPatchifier:
    """(B=1, C, F, H, W) <-> (1, F*H*W, C) token rows (patchifiers.py:14-124)
    for the LTX-2 patch size 1 (temporal and spatial)."""

    def __init__(self, patch_size: int = 1):
        if patch_size != 1:
            raise NotImplementedError("LTX-2 latents use patch size 1 (av_pipeline.py:207)")
        self._patch_size = (1, patch_size, patch_size)

    @property
    def patch_size(self) -> tuple[int, int, int]:
        return self._patch_size

    def patchify(self, latents):
        b, c, f, h, w = latents.shape
        if b != 1:
            raise NotImplementedError("batch size 1")
        n = f * h * w
        return _swap_axes(latents, c, n, 1, (1, n, c))

    def unpatchify(self, latents, output_shape):
        """``output_shape``: (C, F, H, W) or (1, C, F, H, W)."""
        c, f, h, w = tuple(output_shape)[-4:]
        n = f * h * w
        if latents.shape[-2:] != (n, c):
            raise ValueError(f"{tuple(latents.shape)} tokens do not match {(c, f, h, w)}")
        return _swap_axes(latents, n, c, 1, (1, c, f, h, w))


class AudioPatchifier:
    """(B=1, C, T, M) <-> (1, T, C*M) (patchifiers.py:221-374)."""

    def __init__(self, patch_size: int = 1):
        self._patch_size = (1, patch_size, patch_size)

    @property
    def patch_size(self) -> tuple[int, int, int]:
        return self._patch_size

    def patchify(self, audio_latents):
        b, c, t, m = audio_latents.shape
        if b != 1:
            raise NotImplementedError("batch size 1")
        return _swap_axes(audio_latents, c, t, m, (1, t, c * m))

    def unpatchify(self, audio_latents, output_shape):
        """``output_shape``: (C, T, M) or (1, C, T, M)."""
        c, t, m = tuple(output_shape)[-3:]
        if audio_latents.shape[-2:] != (t, c * m):
            raise ValueError(f"{tuple(audio_latents.shape)} tokens do not match {(c, t, m)}")
        return _swap_axes(audio_latents, t, c, m, (1, c, t, m))
