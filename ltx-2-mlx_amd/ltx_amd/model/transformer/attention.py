"""Gated multi-head attention of the LTX-2.3 block on gfx950 kernels.

Mirrors ``Attention`` (model/transformer/attention.py:361-603): gate logits
-> V, Q, K projections -> QK-RMSNorm over the whole inner dim -> split RoPE ->
attention core -> per-head gate 2*sigmoid -> to_out.  The projections are
fused into as few GEMMs as the data flow allows:

* self-attention: one GEMM against [Wq; Wk; Wv; Wg] (the gate-logit columns
  get the 2*sigmoid epilogue in the same launch);
* cross-attention: [Wq; Wg] on the query input and [Wk; Wv] on the context.

K-norm + RoPE run in place on the fused output.  In the cross-attentions the
query's norm and RoPE are applied by the attention kernel as it loads Q, from
per-row sums of squares that the query projection's epilogue writes
(``FUSED_QNORM``); in the self-attention, and with ``FUSED_QNORM`` off, Q is
normalised in place with K.  The attention kernel reads V where the
projection wrote it, the head gate is applied inside the attention kernel, and
``to_out`` is left to the caller so it can fuse the block's residual update
into its epilogue.
"""

from __future__ import annotations

import os

import torch

from ...kernels import attention as attn_k
from ...kernels import gemm
from ...kernels.rope_ops import qknorm_rope_
from ...utils import signpost as _sp

# The query RMS norm + RoPE inside the attention kernel's Q load (row
# statistics from the Q projection's epilogue) instead of an in-place pass
# over Q; LTX_FUSED_QNORM=0 runs the in-place pass for Q and K together.
# Default for the cross-attentions only: in the 48-block step that measured
# 0.2-0.6 ms faster than the in-place pass (two A/B pairs on one box), while
# the video self-attention's form (three factored table rows per query, 8 us
# more per attention workgroup than it saves) measured 0.1-0.2 ms slower;
# LTX_FUSED_QNORM_SELF=1 adds it.
FUSED_QNORM = os.environ.get("LTX_FUSED_QNORM", "1") == "1"
FUSED_QNORM_SELF = os.environ.get("LTX_FUSED_QNORM_SELF", "0") == "1"


class Attention:
    """Resident weights of one attention module and its core forward."""

    def __init__(self, query_dim: int, context_dim: int | None, heads: int, dim_head: int,
                 proj_q: gemm.LinearWeight, proj_kv: gemm.LinearWeight | None,
                 to_out: gemm.LinearWeight, q_norm: torch.Tensor, k_norm: torch.Tensor,
                 norm_eps: float = 1e-6, gated: bool = True):
        self.query_dim = query_dim
        self.self_attention = context_dim is None
        self.context_dim = query_dim if context_dim is None else context_dim
        self.heads = heads
        self.dim_head = dim_head
        self.inner_dim = heads * dim_head
        self.proj_q = proj_q      # self: [q|k|v|g] (3*inner + heads); cross: [q|g] (inner + heads)
        self.proj_kv = proj_kv    # cross only: [k|v] (2*inner)
        self.to_out = to_out
        self.q_norm = q_norm
        self.k_norm = k_norm
        self.norm_eps = norm_eps
        self.gated = gated

    def weights(self) -> list[gemm.LinearWeight]:
        return [w for w in (self.proj_q, self.proj_kv, self.to_out) if w is not None]

    def context_kv(self, context: torch.Tensor, k_pe: tuple | None = None, passes: int = 1) -> torch.Tensor:
        """Keys and values of a cross-attention context: the [Wk; Wv]
        projection with K normalised (and rotated by ``k_pe``, the table of one
        sequence) in place, returned as the (passes*Tk, 2*inner) buffer that
        ``core(..., kv=...)`` takes.  Lets a caller compute them on another
        stream, ahead of the queries."""
        inner = self.inner_dim
        kvb = gemm.linear(context, self.proj_kv)
        k = kvb[:, :inner]
        tk = k.shape[0] // passes
        for p in range(passes):
            kp = k[p * tk:(p + 1) * tk]
            qknorm_rope_(kp[:0], self.q_norm, None, kp, self.k_norm, k_pe, self.heads, self.norm_eps)
        return kvb

    def core(self, x: torch.Tensor, context: torch.Tensor | None = None,
             pe: tuple | None = None, k_pe: tuple | None = None, passes: int = 1,
             kv: torch.Tensor | None = None, kv_ready=None) -> torch.Tensor:
        """Everything up to (not including) ``to_out``; returns (passes*Tq, inner) bf16.

        x: (passes*Tq, query_dim) bf16 -- ``passes`` independent sequences of
        Tq tokens stacked by rows (the batched passes of a guided step);
        context: (passes*Tk, context_dim) bf16 for cross-attention, sequence
        p's keys in rows [p*Tk, (p+1)*Tk).  pe / k_pe: token-major (cos, sin)
        tables of one sequence (or their factored (cos, sin, idx) form), or
        None.  The projections run once over all
        rows; QK-norm + RoPE and the attention run per sequence.  ``kv``:
        the context's keys and values from :meth:`context_kv` (instead of
        ``context``; its keys are already normalised and rotated);
        ``kv_ready``: an event the current stream waits for before the first
        read of ``kv`` (after the query projection and norm).
        """
        inner, heads = self.inner_dim, self.heads
        gate_cols = heads if self.gated else 0
        tq_all = x.shape[0]
        tk_all = tq_all if self.self_attention else (kv if kv is not None else context).shape[0]
        fused = (FUSED_QNORM and (FUSED_QNORM_SELF or not self.self_attention) and inner % 64 == 0
                 and gemm.rowss_eligible(x, self.proj_q)
                 and attn_k.kv_splits(tq_all // passes, tk_all // passes, heads) == 1)
        ss = None
        _sp.begin("attn_qkv")
        if self.self_attention:
            if fused:
                buf, ss = gemm.linear_rowss(x, self.proj_q, inner, sigmoid_from=3 * inner)
            else:
                buf = gemm.linear(x, self.proj_q, sigmoid_from=3 * inner)
            q, k, v = buf[:, :inner], buf[:, inner:2 * inner], buf[:, 2 * inner:3 * inner]
            g = buf[:, 3 * inner:3 * inner + gate_cols] if self.gated else None
            k_tab = pe
        else:
            if fused:
                qb, ss = gemm.linear_rowss(x, self.proj_q, inner, sigmoid_from=inner)
            else:
                qb = gemm.linear(x, self.proj_q, sigmoid_from=inner)
            kvb = gemm.linear(context, self.proj_kv) if kv is None else kv
            q = qb[:, :inner]
            g = qb[:, inner:inner + gate_cols] if self.gated else None
            k, v = kvb[:, :inner], kvb[:, inner:]
            k_tab = pe if k_pe is None else k_pe
            if pe is None:
                k_tab = None
        k_done = kv is not None  # keys already normalised by context_kv
        if passes == 1:
            if not fused:
                qknorm_rope_(q, self.q_norm, pe, k[:0] if k_done else k, self.k_norm, k_tab, heads, self.norm_eps)
            elif not k_done:
                qknorm_rope_(q[:0], self.q_norm, None, k, self.k_norm, k_tab, heads, self.norm_eps)
            _sp.end("attn_qkv")
            if kv_ready is not None:
                torch.cuda.current_stream().wait_event(kv_ready)
            with _sp.signpost("attn_sdpa"):
                return attn_k.flash_attention(q, k, v, heads, gate=g,
                                              qnorm=(ss, self.q_norm, pe, self.norm_eps) if fused else None)
        _sp.end("attn_qkv")
        tq, tk = q.shape[0] // passes, k.shape[0] // passes
        if tq * passes != q.shape[0] or tk * passes != k.shape[0]:
            raise ValueError(f"{q.shape[0]} query / {k.shape[0]} key rows do not split into {passes} passes")
        out = torch.empty((q.shape[0], inner), dtype=torch.bfloat16, device=q.device)
        if kv_ready is not None:
            torch.cuda.current_stream().wait_event(kv_ready)
        for p in range(passes):
            qp, kp, vp = q[p * tq:(p + 1) * tq], k[p * tk:(p + 1) * tk], v[p * tk:(p + 1) * tk]
            gp = None if g is None else g[p * tq:(p + 1) * tq]
            if not fused:
                qknorm_rope_(qp, self.q_norm, pe, kp[:0] if k_done else kp, self.k_norm, k_tab, heads,
                             self.norm_eps)
            elif not k_done:
                qknorm_rope_(qp[:0], self.q_norm, None, kp, self.k_norm, k_tab, heads, self.norm_eps)
            qn = (ss[p * tq:(p + 1) * tq], self.q_norm, pe, self.norm_eps) if fused else None
            attn_k.flash_attention(qp, kp, vp, heads, gate=gp, out=out[p * tq:(p + 1) * tq], qnorm=qn)
        return out

    def __call__(self, x: torch.Tensor, context: torch.Tensor | None = None, mask=None,
                 pe: tuple | None = None, k_pe: tuple | None = None) -> torch.Tensor:
        """Full module forward (attention.py:528-603) on (B=1, T, D) or (T, D)."""
        if mask is not None:
            raise NotImplementedError("attention masks are not on the T2V hot path")
        squeeze = x.dim() == 3
        x2 = x[0] if squeeze else x
        c2 = None if context is None else (context[0] if context.dim() == 3 else context)
        o = self.core(x2, c2, pe, k_pe)
        out = gemm.linear(o, self.to_out)
        return out[None] if squeeze else out
