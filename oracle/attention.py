"""Oracle for the attention core (model/transformer/attention.py:185-302,
kernels/steel_attention.py:251-280): per-head softmax(q k^T / sqrt(dh)) v
with fp32 scores and softmax (the reference's fp32 path), bf16 output, and
the per-head gate of attention.py:594-598 (bf16(bf16(O) * gate)).  Pinned in
tests/test_oracle_attention.py against a float64 brute-force loop and the
invariants of softmax averaging."""

from __future__ import annotations

import math

import numpy as np

from .bf16 import bf16r


def attention(q, k, v, heads: int, gate=None, scale: float | None = None, exact: bool = False):
    """q (Tq, H*dh), k/v (Tk, H*dh) float32 (bf16 values) -> (Tq, H*dh) bf16."""
    import torch

    dt = torch.float64 if exact else torch.float32
    tq, d = q.shape
    tk = k.shape[0]
    dh = d // heads
    if scale is None:
        scale = 1.0 / math.sqrt(dh)
    qt = torch.from_numpy(np.asarray(q, np.float32)).to(dt).view(tq, heads, dh).transpose(0, 1)
    kt = torch.from_numpy(np.asarray(k, np.float32)).to(dt).view(tk, heads, dh).transpose(0, 1)
    vt = torch.from_numpy(np.asarray(v, np.float32)).to(dt).view(tk, heads, dh).transpose(0, 1)
    s = torch.matmul(qt, kt.transpose(1, 2).contiguous()) * scale
    p = torch.softmax(s, dim=-1)
    o = torch.matmul(p, vt.contiguous()).transpose(0, 1).reshape(tq, d)
    out = bf16r(o.numpy().astype(np.float32))
    if gate is not None:
        g = np.asarray(gate, np.float32)
        out = bf16r((out.reshape(tq, heads, dh) * g[:, :, None]).reshape(tq, d))
    return out
