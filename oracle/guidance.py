"""Oracle for the guided loops' elementwise math (test infrastructure only).

A numpy restatement, one correctly rounded fp32 operation at a time in the
reference's order, of:
  X0Model.denoise              model/transformer/model.py:1519-1525
  CFGGuider / CFGStarRescalingGuider / STGGuider delta and guide,
  MultiModalGuider.calculate, projection_coef
                               components/guiders.py:10-190
  GE velocity correction       pipelines/av_pipeline.py:722-728
  EulerDiffusionStep.step      components/diffusion_steps.py:19-69
Python-float scalars enter as their fp32 values (MLX casts a weakly typed
scalar to the array's dtype).  The two reductions (projection coefficient,
variance) are summed in float64 from the fp32 products and rounded once; the
reference's fp32 tree sums differ by their own summation error, so those two
are compared with a tolerance.

Pinning (tests/test_oracle_guidance.py): neutral scales give the conditioned
prediction exactly; an unconditioned prediction equal to the conditioned one
cancels; CFG-star with uncond = 2 * cond rescales it back onto cond and
cancels exactly; the std rescale of pred = 2 * cond halves it; Euler with
sigma_next = 0 returns the denoised latent; GE with gamma = 1 reproduces the
current velocity; and every guide form agrees with torch's float32 evaluation
of the reference's expressions.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16r

f32 = np.float32


def x0(latent, velocity, sigma: float) -> np.ndarray:
    """``latent - sigma * velocity`` (bf16 inputs as float32 values)."""
    return (np.asarray(latent, f32) - (f32(sigma) * np.asarray(velocity, f32)).astype(f32)).astype(f32)


def guide(base, terms=(), scales=(), coef=None, factor=None, delta_only=False) -> np.ndarray:
    """base + sum_k c_k * (base - u_k), u_0 = coef * term_0 when coef is
    given, absent (None) terms skipped; then * factor.  ``delta_only``:
    c_0 * (base - u_0)."""
    base = np.asarray(base, f32)
    def u(k, t):
        t = np.asarray(t, f32)
        return (f32(coef) * t).astype(f32) if (k == 0 and coef is not None) else t
    if delta_only:
        return (f32(scales[0]) * (base - u(0, terms[0])).astype(f32)).astype(f32)
    pred = base.copy()
    for k, (t, c) in enumerate(zip(terms, scales)):
        if t is None:
            continue
        d = (base - u(k, t)).astype(f32)
        pred = (pred + (f32(c) * d).astype(f32)).astype(f32)
    if factor is not None:
        pred = (pred * f32(factor)).astype(f32)
    return pred


def projection_coef(a, b) -> np.float32:
    """sum(a*b) / (sum(b*b) + 1e-8), products in fp32, sums in float64."""
    a, b = np.asarray(a, f32).ravel(), np.asarray(b, f32).ravel()
    dot = f32(np.sum((a * b).astype(f32), dtype=np.float64))
    sq = f32(np.sum((b * b).astype(f32), dtype=np.float64))
    return f32(dot / f32(sq + f32(1e-8)))


def std_ratio(a, b, rescale: float) -> np.float32:
    """rescale * std(a) / std(b) + (1 - rescale), std = sqrt(var + 1e-8)."""
    def std(x):
        x = np.asarray(x, np.float64).ravel()
        return f32(np.sqrt(f32(f32(x.var()) + f32(1e-8))))
    f = f32(std(a) / std(b))
    return f32(f32(f32(rescale) * f) + f32(1.0 - rescale))


def ge_correct(latent, denoised, prev, prev_valid: bool, sigma: float, gamma: float):
    """-> (denoised', current velocity)."""
    x = np.asarray(latent, f32)
    d = np.asarray(denoised, f32)
    cur = ((x - d).astype(f32) / f32(sigma)).astype(f32)
    if prev_valid:
        p = np.asarray(prev, f32)
        total = ((f32(gamma) * (cur - p).astype(f32)).astype(f32) + p).astype(f32)
        d = (x - (total * f32(sigma)).astype(f32)).astype(f32)
    return d, cur


def euler(sample, denoised, sigma: float, sigma_next: float) -> np.ndarray:
    """bf16(denoised + fp32(sigma_next / sigma) * (sample - denoised))."""
    x = np.asarray(sample, f32)
    d = np.asarray(denoised, f32)
    ratio = f32(sigma_next / sigma)
    return bf16r((d + (ratio * (x - d).astype(f32)).astype(f32)).astype(f32))
