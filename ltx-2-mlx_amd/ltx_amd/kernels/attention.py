"""Flash attention on gfx950 (drop-in for the reference attention core).

``flash_attention`` works on the token-major projection outputs the block
produces; ``maybe_steel_attention`` keeps the reference's interface
(kernels/steel_attention.py:251-280: (B, H, T, D) bf16 views, ``scale``,
``mask``; returns ``None`` when the call is outside the kernel's gate so the
caller uses its stock SDPA).  The kernel covers every sequence length
(the reference's STEEL gate needs T >= 512, :244-245), head dims 64 and 128,
batch 1 and no mask.
"""

from __future__ import annotations

import math

import torch

from .. import _lib


def vt_padded_len(tk: int) -> int:
    return (tk + 63) // 64 * 64


def transpose_v(v: torch.Tensor, heads: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """V (Tk, H*dh) token-major -> Vt (H, dh, Tk_pad) in the kernel's layout."""
    d = v.shape[-1]
    dh = d // heads
    vv, vs = _lib.row_view(v, d)
    tk = v.numel() // d
    tkp = vt_padded_len(tk)
    if out is None:
        out = torch.empty((heads, dh, tkp), dtype=torch.bfloat16, device=v.device)
    elif out.shape != (heads, dh, tkp) or not out.is_contiguous():
        raise ValueError(f"Vt buffer must be contiguous {(heads, dh, tkp)}, got {tuple(out.shape)}")
    _lib.call("ltx_attn_transpose_v_bf16", _lib.ptr(vv), vs, tk, heads, dh, _lib.ptr(out), tkp,
              _lib.stream_of(v), detail=f"Tk={tk} H={heads} dh={dh}")
    return out


# Workgroup counts below which the key range is split over workgroups: a
# full-size tile holds 256 queries, a split tile 128.
_FULL_Q, _SPLIT_Q, _MIN_WG, _TARGET_WG = 256, 128, 128, 512


def kv_splits(tq: int, tk: int, heads: int) -> int:
    """Number of key ranges for split-KV attention (1 = single pass)."""
    if (tq + _FULL_Q - 1) // _FULL_Q * heads >= _MIN_WG:
        return 1
    blocks = (tk + 63) // 64
    base = (tq + _SPLIT_Q - 1) // _SPLIT_Q * heads
    return max(1, min(blocks // 2, _TARGET_WG // base, 64))


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None, heads: int, *,
                    vt: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                    out: torch.Tensor | None = None, scale: float | None = None,
                    splits: int | None = None, qnorm: tuple | None = None) -> torch.Tensor:
    """softmax(q k^T * scale) v per head, optionally times a per-head gate.

    q (Tq, H*dh), k/v (Tk, H*dh) bf16 row views; the kernel reads V in that
    layout (transposing LDS reads).  ``vt`` instead passes V already
    transposed by :func:`transpose_v` (then ``v`` is unused).  gate: bf16
    (Tq, H) or None.  Returns (Tq, H*dh) bf16 (written into ``out`` when
    given).  ``splits`` forces the number of key ranges (default
    :func:`kv_splits`); more than one runs the split-KV kernel pair with a
    workspace from the torch allocator.

    ``qnorm`` = (ss, wq, pe, eps): q holds the raw query projection and the
    kernel applies the query RMS norm (weights wq, fp32 (H*dh)) and split RoPE
    (pe as for :func:`rope_ops.qknorm_rope_`, or None) as it loads Q, with
    the row statistics ss (Tq, parts) fp32 from :func:`gemm.linear_rowss`
    (single pass, token-major V only).
    """
    d = q.shape[-1]
    dh = d // heads
    if scale is None:
        scale = 1.0 / math.sqrt(dh)
    qv, qs = _lib.row_view(q, d)
    kv, ks = _lib.row_view(k, d)
    tq = q.numel() // d
    tk = k.numel() // d
    if vt is None:
        vv, vs = _lib.row_view(v, d)
        if v.numel() // d != tk:
            raise ValueError(f"v has {v.numel() // d} rows, k {tk}")
        vptr, vld, sfx = _lib.ptr(vv), vs, "_v"
    else:
        vptr, vld, sfx = _lib.ptr(vt), vt.shape[-1], ""
    if out is None:
        out = torch.empty((tq, d), dtype=torch.bfloat16, device=q.device)
    ov, os_ = _lib.row_view(out, d)
    if ov.data_ptr() != out.data_ptr():
        raise ValueError("out must be a row-strided view")
    gptr, gs = None, 0
    if gate is not None:
        gv, gs = _lib.row_view(gate, heads)
        if gv.dtype != torch.bfloat16:
            raise TypeError("gate must be bf16")
        gate = gv
        gptr = gv.data_ptr()
    if splits is None:
        splits = kv_splits(tq, tk, heads)
    if qnorm is not None:
        if splits > 1 or vt is not None:
            raise ValueError("the fused query norm runs in the single-pass kernel on token-major V")
        ss, wq, pe, eps = qnorm
        if ss.dtype != torch.float32 or ss.dim() != 2 or ss.shape[0] != tq or ss.stride(1) != 1:
            raise ValueError(f"row statistics must be fp32 ({tq}, parts) rows, got {tuple(ss.shape)}")
        if wq.dtype != torch.float32 or wq.numel() != d:
            raise ValueError("query norm weights must be fp32 with H*dh elements")
        cos = sin = idx = None
        axes, rows = 1, 0
        if pe is not None:
            cos, sin = pe[0], pe[1]
            if cos.dtype != torch.float32 or cos.shape[-1] != d // 2 or sin.shape != cos.shape:
                raise ValueError(f"RoPE tables must be fp32 (R, {d // 2})")
            rows = cos.numel() // (d // 2)
            if len(pe) > 2:
                idx = pe[2].contiguous()
                if idx.dtype != torch.int32 or idx.dim() != 2 or idx.shape[0] < tq:
                    raise ValueError(f"RoPE row index must be int32 (T, axes) covering {tq} rows")
                axes = idx.shape[1]
        _lib.call("ltx_flash_attn_qnorm_v_bf16", _lib.ptr(qv), qs, _lib.ptr(kv), ks, vptr, vld, ov.data_ptr(), os_,
                  gptr, gs, tq, tk, heads, dh, float(scale), ss.data_ptr(), ss.stride(0), ss.shape[1],
                  wq.contiguous().data_ptr(), float(eps), _lib.ptr(cos), _lib.ptr(sin), _lib.ptr(idx), axes, rows,
                  _lib.stream_of(q), detail=f"qnorm Tq={tq} Tk={tk} H={heads} dh={dh}")
        return out
    if splits > 1:
        nbytes = _lib.lib().ltx_attn_splitkv_workspace_bytes(tq, heads, dh, splits)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        _lib.call(f"ltx_flash_attn_splitkv{sfx}_bf16", _lib.ptr(qv), qs, _lib.ptr(kv), ks, vptr, vld,
                  ov.data_ptr(), os_, gptr, gs, tq, tk, heads, dh, float(scale), splits, ws.data_ptr(), nbytes,
                  _lib.stream_of(q), detail=f"Tq={tq} Tk={tk} H={heads} dh={dh} splits={splits}")
        return out
    _lib.call(f"ltx_flash_attn{sfx}_bf16", _lib.ptr(qv), qs, _lib.ptr(kv), ks, vptr, vld, ov.data_ptr(), os_,
              gptr, gs, tq, tk, heads, dh, float(scale), _lib.stream_of(q),
              detail=f"Tq={tq} Tk={tk} H={heads} dh={dh}")
    return out


def _token_major(x: torch.Tensor) -> torch.Tensor:
    """(1, H, T, D) -> (T, H*D) view (copy only if not head-interleaved)."""
    _, h, t, d = x.shape
    tm = x[0].permute(1, 0, 2)  # (T, H, D)
    if tm.stride(2) == 1 and tm.stride(1) == d:
        return tm.as_strided((t, h * d), (tm.stride(0), 1))
    return tm.reshape(t, h * d).contiguous()


def maybe_steel_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                          scale: float | None = None, mask: torch.Tensor | None = None) -> torch.Tensor | None:
    """Reference-compatible entry (kernels/steel_attention.py:251-280)."""
    if mask is not None or q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return None
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        return None
    if q.shape[0] != 1 or k.shape[1] != q.shape[1] or v.shape[1] != q.shape[1]:
        return None
    dh = q.shape[-1]
    if dh not in (64, 128) or k.shape[-1] != dh or v.shape[-1] != dh or k.shape[2] != v.shape[2]:
        return None
    if scale is not None and abs(float(scale) - 1.0 / math.sqrt(dh)) >= 1e-7:
        return None
    heads, tq = q.shape[1], q.shape[2]
    out = flash_attention(_token_major(q), _token_major(k), _token_major(v), heads)
    return out.view(1, tq, heads, dh).transpose(1, 2)
