"""QK-RMSNorm + split RoPE (in place) and the RoPE table layout.

Replaces the ``q_norm``/``k_norm`` + ``apply_rotary_emb`` sequence of
``Attention.__call__`` (model/transformer/attention.py:578-584) with one HIP
launch per attention call.  The kernel reads the cos/sin tables token-major,
(T, D/2) fp32: the reference's (1, H, T, dh/2) tables transposed once when
they are built (rope.py:274-283).
"""

from __future__ import annotations

import torch

from .. import _lib


def qknorm_rope_(q: torch.Tensor, wq: torch.Tensor, pe_q: tuple | None,
                 k: torch.Tensor, wk: torch.Tensor, pe_k: tuple | None,
                 heads: int, eps: float = 1e-6) -> None:
    """In-place ``q = rope(q_norm(q), pe_q)``, ``k = rope(k_norm(k), pe_k)``.

    q: (Tq, D) bf16 rows (any row stride, unit column stride); k: (Tk, D).
    wq/wk: fp32 (D).  pe_*: (cos, sin) fp32 (T, D/2), the factored form
    (cos_f, sin_f, idx) of ``rope.factor_tables_np`` -- stacked per-axis rows
    (R, D/2) and int32 (T, axes) row indices -- or None for no RoPE.
    """
    d = q.shape[-1]
    if k.shape[-1] != d:
        raise ValueError(f"q/k inner dims differ: {d} vs {k.shape[-1]}")
    head_dim = d // heads
    qv, qs = _lib.row_view(q, d)
    kv, ks = _lib.row_view(k, d)
    if qv.data_ptr() != q.data_ptr() or kv.data_ptr() != k.data_ptr():
        raise ValueError("qknorm_rope_ works in place: q/k must be row-strided views")
    tq = q.numel() // d if q.dim() > 1 else 1
    tk = k.numel() // d if k.dim() > 1 else 1
    def table(name, pe, rows):
        if pe is None:
            return None, None, None, 1, 0
        cos, sin = pe[0], pe[1]
        if cos.dtype != torch.float32 or cos.shape[-1] != d // 2 or sin.shape != cos.shape:
            raise ValueError(f"{name} tables must be fp32 (R, {d // 2}), got {tuple(cos.shape)}")
        tab_rows = cos.numel() // (d // 2)
        if len(pe) == 2:
            if tab_rows < rows:
                raise ValueError(f"{name} table covers {tab_rows} of {rows} rows")
            return cos, sin, None, 1, tab_rows
        idx = pe[2]
        if idx.dtype != torch.int32 or idx.dim() != 2 or idx.shape[0] < rows or not 1 <= idx.shape[1] <= 3:
            raise ValueError(f"{name} row index must be int32 (T, axes <= 3) covering {rows} rows")
        return cos, sin, idx.contiguous(), idx.shape[1], tab_rows

    cq, sq, iq, aq, rq = table("pe_q", pe_q, tq)
    ck, sk, ik, ak, rk = table("pe_k", pe_k, tk)
    if iq is None and ik is None:
        _lib.call(
            "ltx_qknorm_rope_bf16",
            _lib.ptr(qv), qs, tq, _lib.ptr(wq), _lib.ptr(cq), _lib.ptr(sq),
            _lib.ptr(kv), ks, tk, _lib.ptr(wk), _lib.ptr(ck), _lib.ptr(sk),
            d, head_dim, float(eps), _lib.stream_of(q),
            detail=f"Tq={tq} Tk={tk} D={d} heads={heads}",
        )
        return
    _lib.call(
        "ltx_qknorm_rope_axes_bf16",
        _lib.ptr(qv), qs, tq, _lib.ptr(wq), _lib.ptr(cq), _lib.ptr(sq), _lib.ptr(iq), aq, rq,
        _lib.ptr(kv), ks, tk, _lib.ptr(wk), _lib.ptr(ck), _lib.ptr(sk), _lib.ptr(ik), ak, rk,
        d, head_dim, float(eps), _lib.stream_of(q),
        detail=f"Tq={tq} Tk={tk} D={d} heads={heads} axes={aq}/{ak}",
    )


def tables_from_reference_layout(cos: torch.Tensor, sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(B=1, H, T, dh/2) reference tables -> token-major (T, H*dh/2) fp32."""
    if cos.dim() != 4 or cos.shape[0] != 1:
        raise ValueError(f"expected (1, H, T, dh/2) tables, got {tuple(cos.shape)}")
    _, h, t, half = cos.shape
    def tm(a):
        return a[0].permute(1, 0, 2).reshape(t, h * half).float().contiguous()
    return tm(cos), tm(sin)
