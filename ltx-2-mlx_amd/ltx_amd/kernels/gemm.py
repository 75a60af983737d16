"""Projection GEMMs: ``y = epilogue(x @ W.T + b)`` on gfx950 matrix cores.

One entry point, :func:`linear`, for the three resident weight formats of
:class:`LinearWeight` (bf16, int8 W8A16, MXFP8).  It replaces ``nn.Linear`` /
``mx.addmm`` (model/transformer/attention.py:425-437,
feed_forward.py:91-112) and ``mx.quantized_matmul`` for the mxfp8 cache
(loader/transformer_cache.py:177-193).  The epilogues fuse what the reference
evaluates right after the projection:

* ``EPI_BIAS``            ``bf16(x W^T + b)``
* ``EPI_GELU``            ``bf16(gelu_tanh(bf16(x W^T + b)))`` (feed_forward.py:101-102)
* ``EPI_RESIDUAL``        ``bf16(res + gate * bf16(x W^T + b))``, the gated residual add
                          of fused_ops.py:345-348 / transformer.py:598, :625
* ``EPI_RESIDUAL_ROUND``  ``bf16(res + bf16(gate * bf16(x W^T + b)))`` (transformer.py:387, :484)
* ``EPI_SIGMOID2``        ``bf16(2 * bf16(sigmoid(bf16(x W^T + b))))``, the per-head gate
                          (attention.py:563-569)

Opt-in (``MX_ACTIVATIONS``, environment ``LTX_MX_ACTIVATIONS=1``): MXFP8
weights multiply MXFP8-quantised activations on the scaled fp8 MFMA
(:func:`linear_mx`) instead of bf16 activations.  That is not the reference's
arithmetic -- its MXFP8 path keeps the activations in bf16 -- and the
activations' E4M3 rounding moves outputs by a few percent of their range.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch

from .. import _lib

EPI_BIAS = _lib.GEMM_EPI_BIAS
EPI_GELU = _lib.GEMM_EPI_GELU
EPI_RESIDUAL = _lib.GEMM_EPI_RESIDUAL
EPI_RESIDUAL_ROUND = _lib.GEMM_EPI_RESIDUAL_ROUND
EPI_SIGMOID2 = _lib.GEMM_EPI_SIGMOID2
TILE_AUTO, TILE_256, TILE_128, TILE_256_DMA, TILE_256x128, TILE_G8, TILE_G8_128 = 0, 1, 2, 3, 4, 5, 6


FORMATS = ("bf16", "int8", "mxfp8")

# Opt-in quantised-activation path for MXFP8 weights (see the module text):
# products with at least this many 256x256 tiles quantise their activations
# and run ltx_gemm_mx_bf16.
MX_ACTIVATIONS = os.environ.get("LTX_MX_ACTIVATIONS", "0") == "1"
MX_MIN_TILES = 100

# Optional launch observer: called as hook(phase, info) with phase "pre" /
# "post" around every GEMM launch on the launching stream (used by bench.py
# to time chosen launches with stream events).  None in normal operation.
LAUNCH_HOOK = None


@dataclass
class LinearWeight:
    """A projection weight resident in HBM.

    ``w`` is (N, K) in nn.Linear layout: bf16, int8 codes, or E4M3 codes
    (uint8).  ``scale`` is fp32 (N) for int8 and E8M0 uint8 (N, K/32) for
    mxfp8.  ``bias`` is fp32 (N) or None.

    ``qlinear`` selects the reference module whose arithmetic the GEMM
    reproduces: False for ``nn.Linear`` (``mx.addmm``: bias added to the fp32
    accumulator, one rounding), True for ``nn.QuantizedLinear`` /
    ``_PretransposedQuantizedLinear`` (loader/transformer_cache.py:177-193:
    ``quantized_matmul(x, w) + bias``, the product rounded to bf16 before the
    bias add).  MXFP8 weights are the reference's quantised linears, so
    ``make_weight(kind="mxfp8")`` sets it; a quantised cache weight decoded
    to bf16 keeps it.
    """

    kind: str
    w: torch.Tensor
    scale: torch.Tensor | None = None
    bias: torch.Tensor | None = None
    qlinear: bool = False

    @property
    def out_features(self) -> int:
        return self.w.shape[0]

    @property
    def in_features(self) -> int:
        return self.w.shape[1]

    def nbytes(self) -> int:
        n = self.w.numel() * self.w.element_size()
        for t in (self.scale, self.bias):
            if t is not None:
                n += t.numel() * t.element_size()
        return n


def _quantize(kind: str, w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    n, k = w.shape
    w = w.contiguous()
    stream = _lib.stream_of(w)
    if kind == "int8":
        q = torch.empty((n, k), dtype=torch.int8, device=w.device)
        s = torch.empty((n,), dtype=torch.float32, device=w.device)
        _lib.call("ltx_quantize_w8_bf16", w.data_ptr(), k, n, k, q.data_ptr(), k, s.data_ptr(), stream,
                  detail=f"N={n} K={k}")
        return q, s
    if kind == "mxfp8":
        q = torch.empty((n, k), dtype=torch.uint8, device=w.device)
        s = torch.empty((n, k // 32), dtype=torch.uint8, device=w.device)
        _lib.call("ltx_quantize_mxfp8_bf16", w.data_ptr(), k, n, k, q.data_ptr(), k, s.data_ptr(), k // 32,
                  stream, detail=f"N={n} K={k}")
        return q, s
    raise ValueError(f"unknown quantised format {kind!r}")


def make_weight(w: torch.Tensor, bias: torch.Tensor | None = None, kind: str = "bf16") -> LinearWeight:
    """Build a resident weight from a bf16 (N, K) device tensor.

    ``kind="int8"`` / ``"mxfp8"`` quantise on the device with the library's
    encoders (include/ltx_hip.h "weight formats").
    """
    if w.dtype != torch.bfloat16 or w.dim() != 2 or not w.is_cuda:
        raise ValueError("make_weight expects a 2-D bf16 device tensor")
    b = None if bias is None else bias.detach().to(device=w.device, dtype=torch.float32).contiguous()
    if kind == "bf16":
        return LinearWeight("bf16", w.contiguous(), None, b)
    q, s = _quantize(kind, w)
    return LinearWeight(kind, q, s, b, qlinear=kind == "mxfp8")


def dequantize(weight: LinearWeight) -> torch.Tensor:
    """bf16 (N, K) values of a weight, decoded exactly per its format."""
    n, k = weight.w.shape
    if weight.kind == "bf16":
        return weight.w
    out = torch.empty((n, k), dtype=torch.bfloat16, device=weight.w.device)
    stream = _lib.stream_of(out)
    if weight.kind == "int8":
        _lib.call("ltx_dequantize_w8_bf16", weight.w.data_ptr(), k, weight.scale.data_ptr(), n, k,
                  out.data_ptr(), k, stream)
    else:
        _lib.call("ltx_dequantize_mxfp8_bf16", weight.w.data_ptr(), k, weight.scale.data_ptr(), k // 32, n, k,
                  out.data_ptr(), k, stream)
    return out


# Block budget of an automatic split-K launch (128x128 tiles x splits).
SPLITK_MAX_BLOCKS = 80


def auto_splits(m: int, n: int, k: int, kind: str, max_blocks: int | None = None) -> int:
    """Split-K factor for a few-row product: the largest power of two keeping
    at most ``max_blocks`` (default ``SPLITK_MAX_BLOCKS``) blocks of 128x128
    tiles, at least 256 of K per split and K divisible by the split
    granularity; 1 when the product already fills the chip (or has more than
    256 rows)."""
    max_blocks = SPLITK_MAX_BLOCKS if max_blocks is None else max_blocks
    if m > 256 or k < 1024:
        return 1
    tiles = ((m + 127) // 128) * ((n + 127) // 128)
    if tiles >= 160:
        return 1
    unit = 128 if kind == "mxfp8" else 64
    s = 1
    while tiles * s * 2 <= max_blocks and k % (unit * s * 2) == 0 and k // (s * 2) >= 256:
        s *= 2
    return s


# Few-row products (at most ROWS_MAX_M rows: the 68 / 121-token audio stream)
# can run on the one-launch split-K kernel of ltx_gemm_rows_* with about
# ROWS_TARGET_WGS workgroups (LTX_GEMM_ROWS=1).  Off by default: inside the
# 48-block step, where these products run on the audio stream beside the
# video stream's GEMMs, its workgroups (one per CU, held for the whole K
# stream) cost the step 0.9-2.0 ms against the split-K tile kernel (two
# workgroups per CU) in A/B runs on one box, although alone it is up to 15 %
# faster on the larger audio products.
ROWS_KERNEL = os.environ.get("LTX_GEMM_ROWS", "0") == "1"
ROWS_MAX_M = int(os.environ.get("LTX_GEMM_ROWS_MAX_M", "128"))
ROWS_TARGET_WGS = int(os.environ.get("LTX_GEMM_ROWS_WGS", "256"))
_ROWS_COUNTER_WORDS = 1 << 14
_rows_counters: dict[tuple[int, int], torch.Tensor] = {}


def rows_tiles(m: int, n: int) -> int:
    """Output tiles of ltx_gemm_rows_* (its counter words): row tiles of 64, 96
    or 128 rows x column tiles of 128."""
    bm = 64 if m <= 64 else (96 if m <= 96 else 128)
    return -(-m // bm) * -(-n // 128)


def rows_splits(m: int, n: int, k: int, kind: str, target: int | None = None) -> int:
    """Split count of a few-row product: the largest power of two keeping at
    most ``target`` (default ``ROWS_TARGET_WGS``) workgroups, K divisible by
    the split granularity and at least two K stages per split."""
    target = ROWS_TARGET_WGS if target is None else target
    ks = 64 if kind == "bf16" else 128
    tiles = rows_tiles(m, n)
    s = 1
    while s < 64 and tiles * s * 2 <= target and k % (ks * s * 2) == 0 and k // (s * 2) >= 2 * ks:
        s *= 2
    return s


def rows_eligible(m: int, n: int, k: int, kind: str) -> bool:
    ks = 64 if kind == "bf16" else 128
    return ROWS_KERNEL and 0 < m <= ROWS_MAX_M and k % ks == 0 and n % 8 == 0


def _rows_counters_for(device: torch.device, stream: int, words: int) -> torch.Tensor:
    """A zeroed counter array for the calls of one stream (every call leaves
    it zero).  Cached per stream outside graph capture; under capture without
    a cached array, a fresh one whose zero fill is part of the graph."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    buf = _rows_counters.get(key)
    if buf is not None and buf.numel() >= words:
        return buf
    buf = torch.zeros(max(words, _ROWS_COUNTER_WORDS), dtype=torch.int32, device=device)
    if not torch.cuda.is_current_stream_capturing():
        _rows_counters[key] = buf
    return buf


def linear_rows(x: torch.Tensor, weight: LinearWeight, *, epilogue: int = EPI_BIAS,
                out: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                gate: torch.Tensor | None = None, sigmoid_from: int | None = None,
                splits: int | None = None) -> torch.Tensor:
    """:func:`linear` for few-row x on the one-launch split-K kernel
    (ltx_gemm_rows_*): same epilogues, same rounding points."""
    k = weight.in_features
    n = weight.out_features
    if x.dtype != torch.bfloat16:
        raise TypeError(f"linear_rows expects bf16 activations, got {x.dtype}")
    xv, lda = _lib.row_view(x, k)
    m = x.numel() // k
    lead = x.shape[:-1]
    if out is None:
        out = torch.empty((*lead, n), dtype=torch.bfloat16, device=x.device)
    ov, ldc = _lib.row_view(out, n)
    if ov.data_ptr() != out.data_ptr():
        raise ValueError("out must be a row-strided view")
    rptr, ldr, gptr = None, 0, None
    if epilogue in (EPI_RESIDUAL, EPI_RESIDUAL_ROUND):
        if residual is None or gate is None:
            raise ValueError("residual epilogues need residual and gate")
        rv, ldr = _lib.row_view(residual, n)
        if rv.data_ptr() != residual.data_ptr():
            raise ValueError("residual must be a row-strided view")
        rptr = rv.data_ptr()
        gate = gate.reshape(-1).contiguous()
        if gate.dtype != torch.float32 or gate.numel() != n:
            raise ValueError("gate must be fp32 with N elements")
        gptr = gate.data_ptr()
    flags = epilogue
    if weight.qlinear and weight.bias is not None:
        flags |= _lib.GEMM_ROUND_THEN_BIAS
    sig = n if sigmoid_from is None else int(sigmoid_from)
    bptr = None if weight.bias is None else weight.bias.data_ptr()
    if m == 0:
        return out
    s = rows_splits(m, n, k, weight.kind) if splits is None else int(splits)
    stream = _lib.stream_of(x)
    ws = torch.empty(s * m * n, dtype=torch.float32, device=x.device)
    words = rows_tiles(m, n)
    cnt = _rows_counters_for(x.device, stream, words)
    args = (ws.data_ptr(), ws.numel() * 4, cnt.data_ptr(), cnt.numel(), stream)
    detail = f"rows {weight.kind} M={m} N={n} K={k} epi={epilogue} splits={s}"
    hook = LAUNCH_HOOK
    info = (weight.kind, m, n, k, epilogue)
    if hook is not None:
        hook("pre", info)
    if weight.kind == "bf16":
        _lib.call("ltx_gemm_rows_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0), bptr,
                  ov.data_ptr(), ldc, m, n, k, flags, rptr, ldr, gptr, sig, s, *args, detail=detail)
    elif weight.kind == "int8":
        _lib.call("ltx_gemm_rows_w8a16_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0),
                  weight.scale.data_ptr(), bptr, ov.data_ptr(), ldc, m, n, k, flags, rptr, ldr, gptr, sig, s,
                  *args, detail=detail)
    elif weight.kind == "mxfp8":
        _lib.call("ltx_gemm_rows_mxfp8_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0),
                  weight.scale.data_ptr(), weight.scale.stride(0), bptr, ov.data_ptr(), ldc, m, n, k, flags, rptr,
                  ldr, gptr, sig, s, *args, detail=detail)
    else:
        raise ValueError(f"unknown weight format {weight.kind!r}")
    if hook is not None:
        hook("post", info)
    return out


@dataclass
class MxRows:
    """Activation rows in MXFP8: E4M3 codes (M, K) uint8 and E8M0 scales
    (M, K/32) uint8 -- the opt-in MX path's quantised GEMM input."""

    codes: torch.Tensor
    scales: torch.Tensor

    @property
    def shape(self):
        return self.codes.shape


def quantize_rows_mxfp8(x: torch.Tensor, codes: torch.Tensor | None = None,
                        scales: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """MXFP8 of the rows of x (..., K) bf16 with the library's encoder (the
    weights' OCP rule, blocks of 32 along K): E4M3 codes (M, K) uint8 and E8M0
    scales (M, K / 32) uint8."""
    k = x.shape[-1]
    if k % 32:
        raise ValueError(f"K={k} is not a multiple of 32")
    xv, lda = _lib.row_view(x, k)
    m = x.numel() // k
    if codes is None:
        codes = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    if scales is None:
        scales = torch.empty((m, k // 32), dtype=torch.uint8, device=x.device)
    _lib.call("ltx_quantize_mxfp8_bf16", xv.data_ptr(), lda, m, k, codes.data_ptr(), codes.stride(0),
              scales.data_ptr(), scales.stride(0), _lib.stream_of(x), detail=f"activations M={m} K={k}")
    return codes, scales


def linear_mx(codes: torch.Tensor, scales: torch.Tensor, weight: LinearWeight, *, epilogue: int = EPI_BIAS,
              out: torch.Tensor | None = None, residual: torch.Tensor | None = None,
              gate: torch.Tensor | None = None, sigmoid_from: int | None = None) -> torch.Tensor:
    """``epilogue(x @ W.T + b)`` with x given as MXFP8 rows (codes (M, K),
    scales (M, K/32), from :func:`quantize_rows_mxfp8`) and MXFP8 weights, on
    the scaled fp8 MFMA; the weights' quantised-linear rounding is kept.
    Returns (M, N) bf16."""
    if weight.kind != "mxfp8":
        raise ValueError(f"linear_mx needs MXFP8 weights, got {weight.kind!r}")
    m, k = codes.shape
    n = weight.out_features
    if k != weight.in_features or scales.shape != (m, k // 32):
        raise ValueError(f"activation codes {tuple(codes.shape)} / scales {tuple(scales.shape)} do not match "
                         f"K={weight.in_features}")
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=codes.device)
    ov, ldc = _lib.row_view(out, n)
    rptr, ldr, gptr = None, 0, None
    if epilogue in (EPI_RESIDUAL, EPI_RESIDUAL_ROUND):
        if residual is None or gate is None:
            raise ValueError("residual epilogues need residual and gate")
        rv, ldr = _lib.row_view(residual, n)
        rptr = rv.data_ptr()
        gate = gate.reshape(-1).contiguous()
        if gate.dtype != torch.float32 or gate.numel() != n:
            raise ValueError("gate must be fp32 with N elements")
        gptr = gate.data_ptr()
    flags = epilogue
    if weight.qlinear and weight.bias is not None:
        flags |= _lib.GEMM_ROUND_THEN_BIAS
    sig = n if sigmoid_from is None else int(sigmoid_from)
    bptr = None if weight.bias is None else weight.bias.data_ptr()
    _lib.call("ltx_gemm_mx_bf16", codes.data_ptr(), codes.stride(0), scales.data_ptr(), scales.stride(0),
              weight.w.data_ptr(), weight.w.stride(0), weight.scale.data_ptr(), weight.scale.stride(0), bptr,
              ov.data_ptr(), ldc, m, n, k, flags, rptr, ldr, gptr, sig, _lib.stream_of(codes),
              detail=f"mx M={m} N={n} K={k} epi={epilogue}")
    return out


def linear_mx_gelu(x: MxRows, weight: LinearWeight) -> MxRows:
    """The MX path's FF up-projection: ``mxfp8(bf16(gelu_tanh(bf16(x W^T + b))))``
    with the quantisation in the GEMM's epilogue (ltx_gemm_mx_gelu_mxfp8)."""
    if weight.kind != "mxfp8":
        raise ValueError(f"linear_mx_gelu needs MXFP8 weights, got {weight.kind!r}")
    m, k = x.codes.shape
    n = weight.out_features
    if k != weight.in_features or n % 32:
        raise ValueError(f"K={k} / N={n} do not fit the weight {weight.out_features}x{weight.in_features}")
    codes = torch.empty((m, n), dtype=torch.uint8, device=x.codes.device)
    scales = torch.empty((m, n // 32), dtype=torch.uint8, device=x.codes.device)
    flags = _lib.GEMM_ROUND_THEN_BIAS if (weight.qlinear and weight.bias is not None) else 0
    bptr = None if weight.bias is None else weight.bias.data_ptr()
    hook = LAUNCH_HOOK
    info = (weight.kind, m, n, k, EPI_GELU)
    if hook is not None:
        hook("pre", info)
    _lib.call("ltx_gemm_mx_gelu_mxfp8", x.codes.data_ptr(), x.codes.stride(0), x.scales.data_ptr(),
              x.scales.stride(0), weight.w.data_ptr(), weight.w.stride(0), weight.scale.data_ptr(),
              weight.scale.stride(0), bptr, codes.data_ptr(), n, scales.data_ptr(), n // 32, m, n, k, flags,
              _lib.stream_of(x.codes), detail=f"mx gelu M={m} N={n} K={k}")
    if hook is not None:
        hook("post", info)
    return MxRows(codes, scales)


def _mx_eligible(m: int, n: int, k: int, weight: LinearWeight, tile: int) -> bool:
    return (MX_ACTIVATIONS and weight.kind == "mxfp8" and tile in (TILE_AUTO, TILE_G8) and k % 512 == 0
            and ((m + 255) // 256) * ((n + 255) // 256) >= MX_MIN_TILES)


def rowss_eligible(x: torch.Tensor, weight: LinearWeight) -> bool:
    """Whether :func:`linear_rowss` takes this product: bf16 activations,
    weights of one of the three formats, at least 100 tiles of 256x256 (where
    the automatic choice of :func:`linear` is the 8-wave kernel for a
    projection at least as wide as half its depth, so both give the same
    outputs) and the 8-wave kernel's conditions (MXFP8 weights: K a multiple
    of 512), outside the opt-in MX path."""
    if isinstance(x, MxRows) or x.dtype != torch.bfloat16 or weight.kind not in ("bf16", "int8", "mxfp8"):
        return False
    k, n = weight.in_features, weight.out_features
    m = x.numel() // max(k, 1)
    tiles = ((m + 255) // 256) * ((n + 255) // 256)
    if tiles < 100 or (weight.kind == "bf16" and tiles >= 160 and n < k):
        return False
    if weight.kind == "mxfp8" and (k % 512 or _mx_eligible(m, n, k, weight, TILE_AUTO)):
        return False
    return True


def linear_rowss(x: torch.Tensor, weight: LinearWeight, ss_cols: int, *,
                 sigmoid_from: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """:func:`linear` with the bias epilogue on the 8-wave kernel, plus the
    per-row sums of squares of the bf16 outputs of columns [0, ss_cols) in
    fp32 partials of 64 columns: returns (out (M, N) bf16, ss (M, ss_cols/64)
    fp32) (ltx_gemm_rowss_bf16).  ``out`` is bit-identical to :func:`linear`
    on that kernel."""
    k = weight.in_features
    n = weight.out_features
    if not rowss_eligible(x, weight):
        raise ValueError(f"linear_rowss does not take {weight.kind} weights / {x.dtype} activations here")
    xv, lda = _lib.row_view(x, k)
    m = x.numel() // k
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    parts = ss_cols // 64
    ss = torch.empty((m, parts), dtype=torch.float32, device=x.device)
    flags = EPI_BIAS
    if weight.qlinear and weight.bias is not None:
        flags |= _lib.GEMM_ROUND_THEN_BIAS
    sig = n if sigmoid_from is None else int(sigmoid_from)
    bptr = None if weight.bias is None else weight.bias.data_ptr()
    fmt = {"bf16": 0, "int8": 1, "mxfp8": 2}[weight.kind]
    sptr, lds = (None, 0) if weight.kind == "bf16" else (
        weight.scale.data_ptr(), weight.scale.stride(0) if weight.kind == "mxfp8" else 0)
    hook = LAUNCH_HOOK
    info = (weight.kind, m, n, k, EPI_BIAS) if hook is not None else None
    if hook is not None:
        hook("pre", info)
    if m > 0:
        _lib.call("ltx_gemm_rowss_bf16", fmt, xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0), sptr,
                  lds, bptr, out.data_ptr(), n, m, n, k, flags, sig, ss.data_ptr(), parts, ss_cols,
                  _lib.stream_of(x), detail=f"rowss {weight.kind} M={m} N={n} K={k} ss_cols={ss_cols}")
    if hook is not None:
        hook("post", info)
    return out, ss


def linear(x: torch.Tensor, weight: LinearWeight, *, epilogue: int = EPI_BIAS,
           out: torch.Tensor | None = None, residual: torch.Tensor | None = None,
           gate: torch.Tensor | None = None, tile: int = TILE_AUTO,
           sigmoid_from: int | None = None, splits: int | None = None) -> torch.Tensor:
    """``epilogue(x @ W.T + b)`` for x (..., K) bf16; returns (..., N) bf16.

    For the residual epilogues, ``residual`` (..., N) bf16 and ``gate`` fp32
    (N) are required; ``out`` may be ``residual`` itself (in-place update).
    With ``EPI_BIAS``, columns ``n >= sigmoid_from`` get the 2*sigmoid head
    gate instead (fused gate-logit columns of a Q/QKV projection).
    ``splits``: split-K factor (None: ``auto_splits`` for the 128x128 tiles,
    1: single pass); the split form sums fp32 partials from a workspace.
    With ``ROWS_KERNEL`` set, few-row products with ``splits=None`` and the
    automatic tile choice run on :func:`linear_rows`.
    """
    k = weight.in_features
    n = weight.out_features
    if (splits is None and tile == TILE_AUTO and not isinstance(x, MxRows)
            and rows_eligible(x.numel() // max(k, 1), n, k, weight.kind)):
        return linear_rows(x, weight, epilogue=epilogue, out=out, residual=residual, gate=gate,
                           sigmoid_from=sigmoid_from)
    if isinstance(x, MxRows):  # quantised rows of the opt-in MX path
        hook = LAUNCH_HOOK
        info = (weight.kind, x.codes.shape[0], n, k, epilogue)
        if hook is not None:
            hook("pre", info)
        out = linear_mx(x.codes, x.scales, weight, epilogue=epilogue, out=out, residual=residual, gate=gate,
                        sigmoid_from=sigmoid_from)
        if hook is not None:
            hook("post", info)
        return out
    if x.dtype != torch.bfloat16:
        raise TypeError(f"linear expects bf16 activations, got {x.dtype}")
    xv, lda = _lib.row_view(x, k)
    m = x.numel() // k
    lead = x.shape[:-1]
    if out is None:
        out = torch.empty((*lead, n), dtype=torch.bfloat16, device=x.device)
    ov, ldc = _lib.row_view(out, n)
    if ov.data_ptr() != out.data_ptr():
        raise ValueError("out must be a row-strided view")
    rptr, ldr, gptr = None, 0, None
    if epilogue in (EPI_RESIDUAL, EPI_RESIDUAL_ROUND):
        if residual is None or gate is None:
            raise ValueError("residual epilogues need residual and gate")
        rv, ldr = _lib.row_view(residual, n)
        if rv.data_ptr() != residual.data_ptr():
            raise ValueError("residual must be a row-strided view")
        rptr = rv.data_ptr()
        g = gate.reshape(-1)
        if g.dtype != torch.float32 or g.numel() != n:
            raise ValueError("gate must be fp32 with N elements")
        gate = g.contiguous()
        gptr = gate.data_ptr()
    flags = epilogue | (tile << 8)
    if weight.qlinear and weight.bias is not None:
        flags |= _lib.GEMM_ROUND_THEN_BIAS
    sig = n if sigmoid_from is None else int(sigmoid_from)
    bias = weight.bias
    bptr = None if bias is None else bias.data_ptr()
    stream = _lib.stream_of(x)
    detail = f"{weight.kind} M={m} N={n} K={k} epi={epilogue}"
    hook = LAUNCH_HOOK
    info = (weight.kind, m, n, k, epilogue) if hook is not None else None
    if splits is None:
        splits = auto_splits(m, n, k, weight.kind) if tile in (TILE_AUTO, TILE_128) else 1
    if hook is not None:
        hook("pre", info)
    if splits == 1 and _mx_eligible(m, n, k, weight, tile):
        codes, scales = quantize_rows_mxfp8(x)
        linear_mx(codes, scales, weight, epilogue=epilogue, out=ov, residual=residual, gate=gate,
                  sigmoid_from=sigmoid_from)
        if hook is not None:
            hook("post", info)
        return out
    if splits > 1:
        ws_bytes = splits * m * n * 4
        ws = torch.empty(splits * m * n, dtype=torch.float32, device=x.device)
        if weight.kind == "bf16":
            _lib.call("ltx_gemm_splitk_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0), bptr,
                      ov.data_ptr(), ldc, m, n, k, flags, rptr, ldr, gptr, sig, splits, ws.data_ptr(), ws_bytes,
                      stream, detail=detail)
        elif weight.kind == "int8":
            _lib.call("ltx_gemm_splitk_w8a16_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0),
                      weight.scale.data_ptr(), bptr, ov.data_ptr(), ldc, m, n, k, flags, rptr, ldr, gptr, sig,
                      splits, ws.data_ptr(), ws_bytes, stream, detail=detail)
        elif weight.kind == "mxfp8":
            _lib.call("ltx_gemm_splitk_mxfp8_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0),
                      weight.scale.data_ptr(), weight.scale.stride(0), bptr, ov.data_ptr(), ldc, m, n, k, flags,
                      rptr, ldr, gptr, sig, splits, ws.data_ptr(), ws_bytes, stream, detail=detail)
        else:
            raise ValueError(f"unknown weight format {weight.kind!r}")
        if hook is not None:
            hook("post", info)
        return out
    if weight.kind == "bf16":
        _lib.call("ltx_gemm_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0), bptr,
                  ov.data_ptr(), ldc, m, n, k, flags, rptr, ldr, gptr, sig, stream, detail=detail)
    elif weight.kind == "int8":
        _lib.call("ltx_gemm_w8a16_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0),
                  weight.scale.data_ptr(), bptr, ov.data_ptr(), ldc, m, n, k, flags, rptr, ldr, gptr, sig, stream,
                  detail=detail)
    elif weight.kind == "mxfp8":
        _lib.call("ltx_gemm_mxfp8_bf16", xv.data_ptr(), lda, weight.w.data_ptr(), weight.w.stride(0),
                  weight.scale.data_ptr(), weight.scale.stride(0), bptr, ov.data_ptr(), ldc, m, n, k, flags,
                  rptr, ldr, gptr, sig, stream, detail=detail)
    else:
        raise ValueError(f"unknown weight format {weight.kind!r}")
    if hook is not None:
        hook("post", info)
    return out
