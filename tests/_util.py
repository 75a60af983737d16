"""Comparison helpers shared by the parity tests."""

from __future__ import annotations

import numpy as np


def cos_sim(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(a) * np.linalg.norm(b)
    return float(a @ b / den) if den else float(np.array_equal(a, b))


def max_rel_err(got, ref) -> float:
    """max|got - ref| / max|ref|: the normwise relative error used for the
    bf16 tolerance gate (<= 1e-2)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / scale) if scale else float(np.max(np.abs(got)))


def ulp_diff_bf16(got, ref) -> np.ndarray:
    """Distance in bf16 ulps between two arrays of bf16-representable values."""
    def line(a):
        b = (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.int64)
        # sign-magnitude bf16 bits -> monotone integer line
        return np.where(b & 0x8000, -(b & 0x7FFF), b)

    return np.abs(line(got) - line(ref))


def bf16_from_torch(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()
