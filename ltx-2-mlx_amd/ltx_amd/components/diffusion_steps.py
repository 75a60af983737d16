"""Euler stepping (components/diffusion_steps.py:8-69) and the X0 conversion
(X0Model, model/transformer/model.py:1489-1542).

* ``step_from_velocity``: the distilled loop's fused form, ``x0 = latent -
  sigma * v`` and ``next = bf16(x0 + (sigma_next/sigma) * (latent - x0))`` in
  fp32, one HIP launch;
* ``step``: the reference's signature, from an fp32 denoised latent (the
  guided loops, after guidance);
* ``to_denoised``: the X0 prediction ``latent - sigma * v`` in fp32.
"""

from __future__ import annotations

import numpy as np
import torch

from .. import _lib


def _ratio(sigma: float, sigma_next: float) -> float:
    return float(np.float32(sigma_next / sigma))  # Python-float ratio rounded to fp32, as the reference


def to_denoised(latent: torch.Tensor, velocity: torch.Tensor, sigma: float) -> torch.Tensor:
    """fp32 ``latent - sigma * velocity`` (X0Model.denoise, model.py:1519-1525)."""
    if latent.dtype != torch.bfloat16 or velocity.dtype != torch.bfloat16 or latent.shape != velocity.shape:
        raise ValueError("bf16 latent/velocity of one shape expected")
    latent, velocity = latent.contiguous(), velocity.contiguous()
    out = torch.empty(latent.shape, dtype=torch.float32, device=latent.device)
    _lib.call("ltx_x0_from_velocity_f32", _lib.ptr(latent), _lib.ptr(velocity), float(sigma), _lib.ptr(out),
              latent.numel(), _lib.stream_of(latent))
    return out


class EulerDiffusionStep:
    def step(self, sample: torch.Tensor, denoised_sample: torch.Tensor, sigmas, step_index: int, *,
             sigma: float | None = None, sigma_next: float | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor:
        """``bf16(denoised + (sigma_next/sigma) * (sample - denoised))`` in fp32
        (diffusion_steps.py:19-69); ``out`` may be ``sample``."""
        if sigma is None:
            sigma = float(sigmas[step_index])
        if sigma_next is None:
            sigma_next = float(sigmas[step_index + 1])
        if sample.dtype != torch.bfloat16 or not sample.is_contiguous():
            raise ValueError("contiguous bf16 sample expected")
        d = denoised_sample if denoised_sample.dtype == torch.float32 else denoised_sample.float()
        d = d.contiguous()
        if d.shape != sample.shape:
            raise ValueError("sample and denoised shapes differ")
        if out is None:
            out = torch.empty_like(sample)
        _lib.call("ltx_euler_step_bf16", _lib.ptr(sample), _lib.ptr(d), _ratio(sigma, sigma_next), _lib.ptr(out),
                  sample.numel(), _lib.stream_of(sample))
        return out

    def step_from_velocity(self, sample: torch.Tensor, velocity: torch.Tensor, sigma: float, sigma_next: float,
                           out: torch.Tensor | None = None) -> torch.Tensor:
        """Next latent from the model velocity; ``out`` may be ``sample``."""
        if sample.dtype != torch.bfloat16 or velocity.dtype != torch.bfloat16 or sample.shape != velocity.shape:
            raise ValueError("bf16 sample/velocity of one shape expected")
        if not (sample.is_contiguous() and velocity.is_contiguous()):
            raise ValueError("contiguous tensors expected")
        if out is None:
            out = torch.empty_like(sample)
        _lib.call("ltx_euler_x0_step_bf16", sample.data_ptr(), velocity.data_ptr(), float(sigma),
                  _ratio(sigma, sigma_next), out.data_ptr(), sample.numel(), _lib.stream_of(sample))
        return out
