"""Oracle for the quantised weight formats and the projection GEMM.

* E4M3 decode table from the bit layout (1-4-3, bias 7, 0x7F/0xFF NaN, no
  infinities), pinned against torch.float8_e4m3fn, which the reference states
  is bit-identical to ``mx.from_fp8`` on every non-NaN code
  (loader/transformer_cache.py:661-663), and against the reference's known
  answer 0x38 -> 1.0 (tests/test_transformer_cache.py:64-95).
* E4M3 encoder: nearest representable value, ties to the even code,
  saturating at +-448.  Pinned by brute force against the decode table.
* MXFP8 (OCP MX v1.0) block quantiser: the reference's encoder is
  ``mx.quantize(W, 32, 8, mode="mxfp8")`` (loader/transformer_cache.py:
  1255-1260), MLX-internal and absent here -- the scale selection rule is
  PARITY UNPINNED against MLX; this restates the OCP rule and the tests pin
  its invariants (scale range, round trip of representable blocks).
* int8 per-channel W8A16: defined by the build (the reference has no int8
  path); closed form, pinned by brute-force minimisation.
* FP8 checkpoint dequantisation (loader/transformer_cache.py:691-705):
  ``from_fp8(w) * weight_scale`` in fp32, rounded once; pinned against torch's
  float8_e4m3fn -> float32 product -> bfloat16 casts and the reference's known
  answer (0x38 with weight_scale 2.0 -> 2.0).
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16r


def e4m3_decode_table() -> np.ndarray:
    """float32 value of every E4M3 code (NaN for 0x7F/0xFF)."""
    codes = np.arange(256)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    e = (codes >> 3) & 0xF
    m = codes & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    val = sign * val
    val[(codes & 0x7F) == 0x7F] = np.nan
    return val.astype(np.float32)


_TABLE = e4m3_decode_table()


def fp8_checkpoint_dequant(codes, scale=None, out: str = "bf16") -> np.ndarray:
    """``out(from_fp8(codes) * scale)``, product in fp32 (exact decode without
    a scale); ``out`` "bf16" (RNE, as float32 values) or "f32"."""
    v = _TABLE[np.asarray(codes, dtype=np.uint8)]
    if scale is not None:
        with np.errstate(over="ignore"):  # IEEE overflow to +-inf is the defined result
            v = (v * np.float32(scale)).astype(np.float32)
    return bf16r(v) if out == "bf16" else v
_POS = _TABLE[:0x7F].astype(np.float64)  # codes 0x00..0x7E, ascending


def e4m3_encode(v) -> np.ndarray:
    """Nearest E4M3 code (ties to even code), saturating to +-448."""
    v = np.asarray(v, dtype=np.float64)
    a = np.minimum(np.abs(v), 448.0)
    hi = np.searchsorted(_POS, a, side="left")  # first code with value >= a
    hi = np.minimum(hi, 0x7E)
    lo = np.maximum(hi - 1, 0)
    dlo = a - _POS[lo]
    dhi = _POS[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(np.signbit(v), code | 0x80, code).astype(np.uint8)
    return np.where(np.isnan(v), np.uint8(0x7F), code).astype(np.uint8)


def mxfp8_quantize(W) -> tuple[np.ndarray, np.ndarray]:
    """OCP MX E4M3 quantisation of W (N, K) float32 (bf16 values) in blocks of
    32 along K -> (codes uint8 (N, K), scales uint8 (N, K/32))."""
    W = np.asarray(W, np.float32)
    n, k = W.shape
    blocks = W.reshape(n, k // 32, 32).astype(np.float64)
    amax = np.abs(blocks).max(-1)
    _, e = np.frexp(amax)
    X = np.where(amax > 0, e - 1 - 8, -127)
    X = np.clip(X, -127, 127)
    scaled = blocks / np.exp2(X)[..., None]
    codes = e4m3_encode(scaled).reshape(n, k)
    return codes, (X + 127).astype(np.uint8)


def mxfp8_dequantize(codes, scales) -> np.ndarray:
    """bf16(e4m3(code) * 2^(scale-127)) as float32 (N, K)."""
    codes = np.asarray(codes, np.uint8)
    n, k = codes.shape
    s = np.asarray(scales, np.int64)
    vals = _TABLE[codes].astype(np.float64).reshape(n, k // 32, 32)
    out = vals * np.exp2(s - 127.0)[..., None]
    return bf16r(out.reshape(n, k).astype(np.float32))


def int8_quantize(W) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-row int8: s = max|w|/127 (fp32), q = clamp(rint(w/s))."""
    W = np.asarray(W, np.float32)
    amax = np.abs(W).max(-1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    safe = np.where(s > 0, s, np.float32(1.0))
    q = np.rint((W / safe[:, None]).astype(np.float32))
    q = np.where(s[:, None] > 0, np.clip(q, -127, 127), 0).astype(np.int8)
    return q, s


def int8_dequantize(q, s) -> np.ndarray:
    """bf16(fp32(q) * s) as float32."""
    prod = (np.asarray(q, np.float32) * np.asarray(s, np.float32)[:, None]).astype(np.float32)
    return bf16r(prod)


def gelu_tanh(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def linear(x, W, b=None, *, epilogue: str = "bias", residual=None, gate=None, exact: bool = False,
           round_then_bias: bool = False):
    """Oracle of the projection GEMM + epilogue (nn.Linear / mx.addmm,
    attention.py:425-437, feed_forward.py:91-112): the product of the bf16
    values accumulated in fp32 (the reference's accumulator; ``exact=True``
    uses float64), then the epilogue's rounding points.

    ``round_then_bias`` is nn.QuantizedLinear's form
    (loader/transformer_cache.py:177-193): ``quantized_matmul`` returns the
    bf16 product and the bias is added to it in bf16, ``bf16(bf16(x W^T) + b)``."""
    import torch

    dt = torch.float64 if exact else torch.float32
    xt = torch.from_numpy(np.asarray(x, np.float32)).to(dt)
    wt = torch.from_numpy(np.asarray(W, np.float32)).to(dt)
    y = (xt @ wt.T).double().numpy()
    if round_then_bias:
        y = bf16r(y.astype(np.float32)).astype(np.float64)
    if b is not None:
        y = y + np.asarray(b, np.float64)
    y = bf16r(y.astype(np.float32)).astype(np.float64)
    if epilogue == "bias":
        return bf16r(y)
    if epilogue == "gelu":
        return bf16r(gelu_tanh(y))
    if epilogue == "sigmoid2":
        return bf16r(2.0 * bf16r(1.0 / (1.0 + np.exp(-y))).astype(np.float64))
    g = np.asarray(gate, np.float64)
    r = np.asarray(residual, np.float64)
    if epilogue == "residual":
        return bf16r(r + g * y)
    if epilogue == "residual_round":
        return bf16r(r + bf16r(g * y).astype(np.float64))
    raise ValueError(epilogue)
