"""Euler step fused with the X0 conversion (diffusion_steps.py:8-69,
model.py:1489-1542): ``x0 = latent - sigma * v``; ``next = bf16(x0 +
(sigma_next/sigma) * (latent - x0))`` in fp32, one HIP launch."""

from __future__ import annotations

import numpy as np
import torch

from .. import _lib


class EulerDiffusionStep:
    def step_from_velocity(self, sample: torch.Tensor, velocity: torch.Tensor, sigma: float, sigma_next: float,
                           out: torch.Tensor | None = None) -> torch.Tensor:
        """Next latent from the model velocity; ``out`` may be ``sample``."""
        if sample.dtype != torch.bfloat16 or velocity.dtype != torch.bfloat16 or sample.shape != velocity.shape:
            raise ValueError("bf16 sample/velocity of one shape expected")
        if not (sample.is_contiguous() and velocity.is_contiguous()):
            raise ValueError("contiguous tensors expected")
        if out is None:
            out = torch.empty_like(sample)
        ratio = float(np.float32(sigma_next / sigma))  # Python-float ratio rounded to fp32, as the reference
        _lib.call("ltx_euler_x0_step_bf16", sample.data_ptr(), velocity.data_ptr(), float(sigma), ratio,
                  out.data_ptr(), sample.numel(), _lib.stream_of(sample))
        return out
