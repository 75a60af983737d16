"""Sigma schedules (components/schedulers.py:10-115).

``DISTILLED_SIGMA_VALUES`` / ``STAGE_2_DISTILLED_SIGMA_VALUES`` are the fixed
schedules of the distilled checkpoint; ``LTX2Scheduler`` is the
token-count-shifted schedule of the dev checkpoint used by the guided loops,
evaluated with the reference's fp32 array arithmetic (python scalars meet the
fp32 array as fp32 values); ``linspace`` is numpy's (each point the fp32
rounding of the exact value).  Host-side, once per generation.
"""

from __future__ import annotations

import math

import numpy as np

DISTILLED_SIGMA_VALUES = [1.0, 0.99375, 0.9875, 0.98125, 0.975, 0.909375, 0.725, 0.421875, 0.0]
STAGE_2_DISTILLED_SIGMA_VALUES = [0.909375, 0.725, 0.421875, 0.0]

BASE_SHIFT_ANCHOR = 1024
MAX_SHIFT_ANCHOR = 4096


class LTX2Scheduler:
    """Shifted schedule: ``s' = e^shift / (e^shift + (1/s - 1))`` over
    ``linspace(1, 0, steps + 1)``, the shift linear in the token count between
    the two anchors, then stretched so the last non-zero sigma is
    ``terminal``."""

    def execute(self, steps: int, latent=None, max_shift: float = 2.05, base_shift: float = 0.95,
                stretch: bool = True, terminal: float = 0.1, **_kwargs) -> np.ndarray:
        f32 = np.float32
        if latent is not None:
            tokens = math.prod(latent.shape[2:])
        else:
            tokens = MAX_SHIFT_ANCHOR
        sigmas = np.linspace(1.0, 0.0, steps + 1, dtype=np.float32)
        mm = (max_shift - base_shift) / (MAX_SHIFT_ANCHOR - BASE_SHIFT_ANCHOR)
        b = base_shift - mm * BASE_SHIFT_ANCHOR
        exp_shift = f32(math.exp(tokens * mm + b))
        with np.errstate(divide="ignore"):
            inv = (f32(1.0) / sigmas) - f32(1.0)
            shifted = np.where(sigmas != 0, exp_shift / (exp_shift + inv), f32(0.0)).astype(np.float32)
        sigmas = shifted
        if stretch and steps > 0:
            one_minus = (f32(1.0) - sigmas).astype(np.float32)
            scale_factor = float(one_minus[steps - 1]) / (1.0 - terminal)
            # steps == 1: scale_factor is 0 and the first sigma becomes 0/0 = NaN,
            # as the reference's array division gives
            with np.errstate(divide="ignore", invalid="ignore"):
                stretched = (f32(1.0) - one_minus / f32(scale_factor)).astype(np.float32)
            sigmas = np.where(sigmas != 0, stretched, sigmas).astype(np.float32)
        return sigmas.astype(np.float32)


def get_sigma_schedule(num_steps: int, distilled: bool = False, latent=None) -> np.ndarray:
    """The distilled schedule, or the shifted one for ``num_steps`` steps (fp32)."""
    if distilled:
        return np.asarray(DISTILLED_SIGMA_VALUES, dtype=np.float32)
    return LTX2Scheduler().execute(steps=num_steps, latent=latent)
