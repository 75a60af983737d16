"""Guidance strategies (components/guiders.py:10-190) on device tensors.

Same classes and methods as the reference: ``CFGGuider``,
``CFGStarRescalingGuider``, ``STGGuider`` (``delta`` / ``guide`` /
``enabled``), ``MultiModalGuiderParams``, ``MultiModalGuider``
(``calculate``, ``do_unconditional_generation``,
``do_isolated_modality_generation``) and ``projection_coef``.  The operands
are the fp32 denoised latents of the transformer passes; the arithmetic runs
in the HIP kernels ``ltx_guidance_f32`` / ``ltx_guidance_stats_f32`` with the
reference's fp32 operation order (each scale enters as the fp32 value of the
python float expression, as MLX casts weakly typed scalars).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .. import _lib

GUIDE_DELTA_ONLY = 1
STATS_PROJECTION = 1
STATS_STD_RATIO = 2


def _check(*ts: torch.Tensor) -> None:
    shape = ts[0].shape
    for t in ts:
        if t.dtype != torch.float32 or not t.is_contiguous() or t.shape != shape:
            raise ValueError("guidance operands are contiguous fp32 tensors of one shape")


def _guide(base, terms=(), scales=(), coef=None, factor=None, delta_only=False) -> torch.Tensor:
    """Launch ``ltx_guidance_f32``: base + sum_k c_k * (base - u_k) [* factor]."""
    ts = list(terms) + [None] * (3 - len(terms))
    cs = list(scales) + [0.0] * (3 - len(scales))
    _check(base, *[t for t in ts if t is not None])
    out = torch.empty_like(base)
    _lib.call("ltx_guidance_f32", _lib.ptr(base), _lib.ptr(ts[0]), _lib.ptr(ts[1]), _lib.ptr(ts[2]),
              cs[0], cs[1], cs[2], _lib.ptr(coef), _lib.ptr(factor), _lib.ptr(out), base.numel(),
              GUIDE_DELTA_ONLY if delta_only else 0, _lib.stream_of(base))
    return out


def _stats(a: torch.Tensor, b: torch.Tensor, mode: int, rescale: float = 0.0) -> torch.Tensor:
    _check(a, b)
    out = torch.empty((1,), dtype=torch.float32, device=a.device)
    _lib.call("ltx_guidance_stats_f32", _lib.ptr(a), _lib.ptr(b), a.numel(), mode, rescale, 1.0 - rescale,
              _lib.ptr(out), _lib.stream_of(a))
    return out


def projection_coef(to_project: torch.Tensor, project_onto: torch.Tensor) -> torch.Tensor:
    """sum(a*b) / (sum(b*b) + 1e-8) over the whole (batch-1) latent, as a
    device fp32 scalar of shape (1,) (guiders.py:175-190)."""
    return _stats(to_project, project_onto, STATS_PROJECTION)


@dataclass(frozen=True)
class CFGGuider:
    """Classifier-free guidance: ``cond + (scale - 1) * (cond - uncond)``."""

    scale: float

    def delta(self, cond: torch.Tensor, uncond: torch.Tensor) -> torch.Tensor:
        return _guide(cond, (uncond,), (self.scale - 1,), delta_only=True)

    def guide(self, cond: torch.Tensor, uncond: torch.Tensor) -> torch.Tensor:
        return _guide(cond, (uncond,), (self.scale - 1,))

    def enabled(self) -> bool:
        return self.scale != 1.0


@dataclass(frozen=True)
class CFGStarRescalingGuider:
    """CFG with the unconditioned prediction rescaled by its projection
    coefficient onto the conditioned one."""

    scale: float

    def delta(self, cond: torch.Tensor, uncond: torch.Tensor) -> torch.Tensor:
        return _guide(cond, (uncond,), (self.scale - 1,), coef=projection_coef(cond, uncond), delta_only=True)

    def guide(self, cond: torch.Tensor, uncond: torch.Tensor) -> torch.Tensor:
        return _guide(cond, (uncond,), (self.scale - 1,), coef=projection_coef(cond, uncond))

    def enabled(self) -> bool:
        return self.scale != 1.0


@dataclass(frozen=True)
class STGGuider:
    """Spatio-temporal guidance: ``pos + scale * (pos - perturbed)``."""

    scale: float

    def delta(self, pos_denoised: torch.Tensor, perturbed_denoised: torch.Tensor) -> torch.Tensor:
        return _guide(pos_denoised, (perturbed_denoised,), (self.scale,), delta_only=True)

    def guide(self, pos_denoised: torch.Tensor, perturbed_denoised: torch.Tensor) -> torch.Tensor:
        return _guide(pos_denoised, (perturbed_denoised,), (self.scale,))

    def enabled(self) -> bool:
        return self.scale != 0.0


@dataclass(frozen=True)
class MultiModalGuiderParams:
    cfg_scale: float = 1.0
    stg_scale: float = 0.0
    stg_blocks: list | None = field(default_factory=list)
    rescale_scale: float = 0.0
    modality_scale: float = 1.0


@dataclass(frozen=True)
class MultiModalGuider:
    """CFG + STG + modality-isolated guidance with the optional std rescale
    (guiders.py:106-172); absent passes are given as the float 0.0."""

    params: MultiModalGuiderParams
    negative_context: torch.Tensor | None = None

    def calculate(self, cond: torch.Tensor, uncond_text, uncond_perturbed, uncond_modality) -> torch.Tensor:
        p = self.params
        dtype = cond.dtype
        if dtype != torch.float32:
            raise ValueError("the denoised predictions are fp32")
        terms, scales = [], []
        for t, c in ((uncond_text, p.cfg_scale - 1), (uncond_perturbed, p.stg_scale),
                     (uncond_modality, p.modality_scale - 1)):
            if isinstance(t, torch.Tensor):
                terms.append(t)
                scales.append(c)
            else:
                terms.append(None)
                scales.append(0.0)
        pred = _guide(cond, terms, scales)
        if p.rescale_scale != 0:
            factor = _stats(cond, pred, STATS_STD_RATIO, p.rescale_scale)
            pred = _guide(pred, (), (), factor=factor)
        return pred

    def do_unconditional_generation(self) -> bool:
        return not math.isclose(self.params.cfg_scale, 1.0)

    def do_isolated_modality_generation(self) -> bool:
        return not math.isclose(self.params.modality_scale, 1.0)
