"""Fused AdaLN and gated-residual operators on gfx950.

Drop-in for ``LTX_2_MLX/kernels/fused_ops.py``: same function names,
argument meaning, shape/dtype gates and fallbacks.

* ``adaln_norm_fused(x, scale, shift, eps)`` (reference :237-287) computes
  ``(rms_norm(x) * (1 + scale) + shift).astype(x.dtype)`` with one rounding,
  like the reference Metal kernel (:172-175).
* ``gated_add_fused(residual, branch, gate)`` (reference :398-442) computes
  ``(residual + branch * gate).astype(residual.dtype)``.

When the gate predicate (reference :204-234 and :369-395) accepts the call,
the HIP kernel in libltx_hip.so runs on the tensors' device and current
stream.  Otherwise the stock-framework expression runs, exactly as the
reference falls back to its MLX expression (:192-201, :362-366).  The gate
never depends on whether the library is present: a missing library raises.

``LTX_FUSED_PROBE=1`` tallies kernel vs fallback dispatches per operator and
prints the kernel share at exit (the reference's switch, :12-69).
"""

from __future__ import annotations

import atexit
import collections
import os

import torch

from .. import _lib

class _DispatchTally:
    """Counts, per operator, how many calls took the HIP kernel and how many
    the fallback expression, when ``$LTX_FUSED_PROBE`` is set (the reference's
    probe switch, kernels/fused_ops.py:12-69); the per-operator kernel share is
    printed once at interpreter exit."""

    PATHS = ("kernel", "fallback")

    def __init__(self, ops: tuple[str, ...]):
        self.enabled = bool(os.environ.get("LTX_FUSED_PROBE"))
        self.ops = ops
        self.tally = collections.Counter()
        if self.enabled:
            atexit.register(self.report)

    def hit(self, op: str, path: str) -> None:
        if self.enabled:
            self.tally[op, path] += 1

    def counts(self) -> dict[str, int]:
        return {f"{op}_{path}": self.tally[op, path] for op in self.ops for path in self.PATHS}

    def report(self) -> None:
        lines = []
        for op in self.ops:
            k, f = self.tally[op, "kernel"], self.tally[op, "fallback"]
            if k + f:
                lines.append(f"  {op}: {k} on the HIP kernel, {f} on the fallback "
                             f"({k / (k + f):.1%} kernel)")
        if lines:
            print("LTX_FUSED_PROBE dispatch tally", *lines, sep="\n")


_TALLY = _DispatchTally(("adaln", "gated_add"))


def get_dispatch_counts() -> dict[str, int]:
    """``{op_path: calls}`` for op in (adaln, gated_add) and path in (kernel,
    fallback); all zero unless ``$LTX_FUSED_PROBE`` is set."""
    return _TALLY.counts()


_ADALN_FUSED_EPS = 1e-6
# Channel counts with a registered kernel.  The reference registers C=4096
# (video) and C=2048 (audio) only (:98-101); the gate keeps that set so the
# dispatch decisions are the reference's.
_ADALN_FUSED_CONFIGS: tuple[int, ...] = (4096, 2048)
_GATED_ADD_FUSED_CONFIGS: tuple[int, ...] = (4096, 2048)


def _rms_norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    """``mx.fast.rms_norm(x, None, eps)``: fp32 reduction, output in x.dtype."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)).to(x.dtype)


def _adaln_norm_torch(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float) -> torch.Tensor:
    """Fallback expression, the reference's ``_adaln_norm_mlx`` (:192-201)."""
    normed = _rms_norm(x, eps)
    return (normed * (1 + scale) + shift).to(x.dtype)


def _adaln_t2v_broadcast_compatible(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor) -> bool:
    """Reference gate (:204-234): x 3-D bf16 with a registered C; scale and
    shift fp32 with last dim C and all-singleton leading dims."""
    if x.dtype != torch.bfloat16 or x.dim() != 3:
        return False
    c = x.shape[-1]
    if c not in _ADALN_FUSED_CONFIGS:
        return False
    if scale.dtype != torch.float32 or shift.dtype != torch.float32:
        return False
    if scale.shape[-1] != c or shift.shape[-1] != c:
        return False
    if any(d != 1 for d in scale.shape[:-1]) or any(d != 1 for d in shift.shape[:-1]):
        return False
    return True


def adaln_rows(x2d: torch.Tensor, x_stride: int, scale: torch.Tensor, shift: torch.Tensor,
               out2d: torch.Tensor, out_stride: int, rows: int, c: int, eps: float, flags: int) -> None:
    """Launch the AdaLN kernel on row views (no gate, no allocation)."""
    _lib.call(
        "ltx_adaln_norm_fused_bf16",
        _lib.ptr(x2d), x_stride, _lib.ptr(scale), _lib.ptr(shift), _lib.ptr(out2d), out_stride,
        rows, c, float(eps), flags, _lib.stream_of(x2d),
        detail=f"rows={rows} C={c}",
    )


def adaln_rows2(x2d: torch.Tensor, x_stride: int, scale: torch.Tensor, shift: torch.Tensor, out2d: torch.Tensor,
                scale2: torch.Tensor, shift2: torch.Tensor, out2_2d: torch.Tensor, rows: int, c: int, eps: float,
                flags: int) -> None:
    """Two modulations of one row norm (one read of x): out = AdaLN(x, scale,
    shift), out2 = AdaLN(x, scale2, shift2), both with row stride c."""
    _lib.call(
        "ltx_adaln_norm_fused2_bf16",
        _lib.ptr(x2d), x_stride, _lib.ptr(scale), _lib.ptr(shift), _lib.ptr(out2d), c, _lib.ptr(scale2),
        _lib.ptr(shift2), _lib.ptr(out2_2d), c, rows, c, float(eps), flags, _lib.stream_of(x2d),
        detail=f"rows={rows} C={c} (two outputs)",
    )


def adaln_norm_fused(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float) -> torch.Tensor:
    """Fused RMSNorm + AdaLN modulation: ``rms_norm(x) * (1+scale) + shift``.

    Returns ``(rms_norm(x) * (1 + scale) + shift).astype(x.dtype)``; the
    kernel path rounds once, like the reference kernel.
    """
    if eps != _ADALN_FUSED_EPS or not _adaln_t2v_broadcast_compatible(x, scale, shift):
        _TALLY.hit("adaln", "fallback")
        return _adaln_norm_torch(x, scale, shift, eps)
    _TALLY.hit("adaln", "kernel")
    b, t, c = x.shape
    xv, xs = _lib.row_view(x, c)
    out = torch.empty((b, t, c), dtype=torch.bfloat16, device=x.device)
    adaln_rows(xv, xs, scale.reshape(-1).contiguous(), shift.reshape(-1).contiguous(),
               out, c, b * t, c, eps, 0)
    return out


def _gated_add_torch(residual: torch.Tensor, branch: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """Fallback expression, the reference's ``_gated_add_mlx`` (:362-366)."""
    return (residual + branch * gate).to(residual.dtype)


def _gated_add_t2v_broadcast_compatible(residual: torch.Tensor, branch: torch.Tensor, gate: torch.Tensor) -> bool:
    """Reference gate (:369-395)."""
    if residual.dtype != torch.bfloat16 or branch.dtype != torch.bfloat16:
        return False
    if residual.dim() != 3:
        return False
    c = residual.shape[-1]
    if c not in _GATED_ADD_FUSED_CONFIGS:
        return False
    if residual.shape != branch.shape:
        return False
    if gate.dtype != torch.float32 or gate.shape[-1] != c:
        return False
    if any(d != 1 for d in gate.shape[:-1]):
        return False
    return True


def gated_add_rows(res2d: torch.Tensor, res_stride: int, br2d: torch.Tensor, br_stride: int,
                   gate: torch.Tensor, out2d: torch.Tensor, out_stride: int, rows: int, c: int,
                   flags: int) -> None:
    """Launch the gated-add kernel on row views (no gate, no allocation)."""
    _lib.call(
        "ltx_gated_add_fused_bf16",
        _lib.ptr(res2d), res_stride, _lib.ptr(br2d), br_stride, _lib.ptr(gate), _lib.ptr(out2d),
        out_stride, rows, c, flags, _lib.stream_of(res2d),
        detail=f"rows={rows} C={c}",
    )


def gated_add_fused(residual: torch.Tensor, branch: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """Fused gated add: ``residual + branch * gate``, cast to residual.dtype."""
    if not _gated_add_t2v_broadcast_compatible(residual, branch, gate):
        _TALLY.hit("gated_add", "fallback")
        return _gated_add_torch(residual, branch, gate)
    _TALLY.hit("gated_add", "kernel")
    b, t, c = residual.shape
    rv, rs = _lib.row_view(residual, c)
    bv, bs = _lib.row_view(branch, c)
    out = torch.empty((b, t, c), dtype=torch.bfloat16, device=residual.device)
    gated_add_rows(rv, rs, bv, bs, gate.reshape(-1).contiguous(), out, c, b * t, c, 0)
    return out
