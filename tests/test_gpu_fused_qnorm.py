"""GPU parity of the query RMS norm + RoPE fused into the attention kernel.

* ``ltx_gemm_rowss_bf16``: the projection output is bit-identical to
  ``ltx_gemm_*`` (the 8-wave kernel, the automatic choice at these shapes),
  and each row statistic equals the float64 sum of squares of those bf16
  outputs over its 64 columns within fp32 summation error.
* ``ltx_flash_attn_qnorm_v_bf16`` on the raw projection against the separate
  in-place pass (``ltx_qknorm_rope_*``, pinned to the oracle in
  test_gpu_fused_ops.py) followed by ``ltx_flash_attn_v_bf16``, for the three
  video-query call shapes of the block: self-attention 3456^2 (factored
  3-axis tables), text cross-attention 3456 x 256 (no RoPE), A2V 3456 x 68 at
  head_dim 64 (time-only tables); and against the oracle's
  ``qknorm_rope`` + ``attention``.  The query values are multiples of 1/8 in
  [-4, 4], so every sum of squares over a row is exact in fp32 whatever the
  summation order: both paths then normalise with the same factor, and only
  the rounding of the rotation's products may differ between the two
  kernels.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import bf16_from_torch, cos_sim, max_rel_err, ulp_diff_bf16
from oracle import attention as oattn
from oracle import rope as orope
from oracle.bf16 import bf16r

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def _bf(rng, shape, scale=1.0):
    return bf16r(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


@pytest.mark.parametrize("kind", ["bf16", "int8", "mxfp8"])
@pytest.mark.parametrize("M,N,ss_cols", [(3456, 12320, 4096), (3456, 4128, 4096), (3456, 2080, 2048),
                                         (2900, 4128, 4096)])
def test_gemm_rowss_output_and_statistics(kind, M, N, ss_cols):
    """QKV + gate, text query + gate and A2V query + gate projections (the
    gate columns past ss_cols take the head-gate epilogue); 2900 rows: the
    automatic row split's second launch writes its rows' statistics at the
    offset rows."""
    from ltx_amd.kernels import gemm

    print(f"rowss {kind} M={M} N={N} ss_cols={ss_cols}", flush=True)
    rng = np.random.default_rng(M + N)
    K = 4096
    x = _t(_bf(rng, (M, K)))
    wt = gemm.make_weight(_t(_bf(rng, (N, K), 0.02)), _t(rng.standard_normal(N).astype(np.float32) * 0.02,
                                                        torch.float32), kind=kind)
    assert gemm.rowss_eligible(x, wt)
    out, ss = gemm.linear_rowss(x, wt, ss_cols, sigmoid_from=ss_cols)
    ref = gemm.linear(x, wt, sigmoid_from=ss_cols)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    want = (out[:, :ss_cols].double() ** 2).view(M, ss_cols // 64, 64).sum(-1)
    assert ss.shape == (M, ss_cols // 64)
    rel = ((ss.double() - want).abs() / want.clamp_min(1e-30)).max().item()
    assert rel <= 64 * 2.0 ** -24, rel


def _grid_q(rng, shape):
    """bf16 multiples of 1/8 in [-4, 4]: every sum of squares of a 4096-wide
    row is a multiple of 1/64 below 2^16, exact in fp32."""
    return (rng.integers(-32, 33, shape).astype(np.float32) / 8.0).astype(np.float32)


def _factored(pos, dim, max_pos):
    from ltx_amd.model.transformer import rope as prope

    full = prope.rope_tables_np(pos, dim, max_pos)
    fac = prope.factor_tables_np(pos, *full)
    return full, tuple(torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in fac)


def _case(tq, tk, d, heads, tables, seed, oracle_tables=None, oracle=False):
    """Fused vs separate pass for one call shape, and against the oracle
    when ``oracle`` (with the oracle's own tables ``oracle_tables``).
    tables: (numpy (cos, sin), the form passed to the kernels) or None."""
    from ltx_amd.kernels import attention as attn_k
    from ltx_amd.kernels.rope_ops import qknorm_rope_

    print(f"qnorm attention Tq={tq} Tk={tk} D={d} heads={heads} rope={tables is not None}", flush=True)
    rng = np.random.default_rng(seed)
    q = _grid_q(rng, (tq, d))
    k = _bf(rng, (tk, d), 1.0)
    v = _bf(rng, (tk, d), 1.0)
    gate = bf16r(rng.uniform(0.0, 2.0, (tq, heads)).astype(np.float32))
    wq = bf16r((1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    qt, kt, vt, gt, wt = _t(q), _t(k), _t(v), _t(gate), _t(wq, torch.float32)
    pe = None if tables is None else tables[1]
    # separate pass: in-place norm + RoPE of Q, then the attention
    qs = qt.clone()
    qknorm_rope_(qs, wt, pe, kt[:0], wt, None, heads)
    ref = attn_k.flash_attention(qs, kt, vt, heads, gate=gt)
    # fused: row statistics as 64-column partials of the raw rows
    ss = (qt.float() ** 2).view(tq, d // 64, 64).sum(-1).contiguous()
    got = attn_k.flash_attention(qt, kt, vt, heads, gate=gt, qnorm=(ss, wt, pe, 1e-6))
    torch.cuda.synchronize()
    g, r = bf16_from_torch(got), bf16_from_torch(ref)
    exact = float((ulp_diff_bf16(g, r) == 0).mean())
    print(f"  bit-identical to the separate pass: {exact:.6f}", flush=True)
    if tables is None:
        np.testing.assert_array_equal(g, r)
    else:
        assert exact >= 0.99
        assert max_rel_err(g, r) <= 1e-2 and cos_sim(g, r) >= 0.99999
    if oracle:
        cos_np, sin_np = (None, None) if oracle_tables is None else oracle_tables
        qn = orope.qknorm_rope(q, wq, cos_np, sin_np, heads)
        ro = oattn.attention(qn, k, v, heads, gate=gate)
        assert max_rel_err(g, ro) <= 1e-2 and cos_sim(g, ro) >= 0.9999


def test_qnorm_attention_video_self():
    pos = orope.video_positions(9, 16, 24, fps=24.0)
    _case(3456, 3456, 4096, 32, _factored(pos, 4096, orope.VIDEO_MAX_POS), seed=1)


def test_qnorm_attention_text_cross():
    _case(3456, 256, 4096, 32, None, seed=2, oracle=True)


def test_qnorm_attention_a2v():
    pos = orope.video_positions(9, 16, 24, fps=24.0)
    _case(3456, 68, 2048, 32, _factored(pos[:, 0:1], 2048, orope.AUDIO_MAX_POS), seed=3,
          oracle_tables=orope.rope_tables(pos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS), oracle=True)


def test_qnorm_attention_per_token_tables_and_ragged():
    """Per-token (unfactored) tables and a query count that leaves the last
    query tile partly empty."""
    pos = orope.video_positions(5, 16, 25, fps=24.0)  # 2000 tokens
    full = orope.rope_tables(pos, 4096, 32, orope.VIDEO_MAX_POS)
    dev = tuple(_t(a, torch.float32) for a in full)
    _case(2000, 2000, 4096, 32, (full, dev), seed=4)


def test_qnorm_attention_rejects():
    from ltx_amd import _lib
    from ltx_amd.kernels import attention as attn_k

    q = torch.zeros((512, 4096), dtype=torch.bfloat16, device=DEV)
    w = torch.ones(4096, dtype=torch.float32, device=DEV)
    ss = torch.ones((512, 64), dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError, match="single-pass"):
        attn_k.flash_attention(q, q, q, 32, qnorm=(ss, w, None, 1e-6), splits=2)
    o = torch.empty_like(q)
    with pytest.raises(_lib.LtxKernelError, match="invalid"):
        _lib.call("ltx_flash_attn_qnorm_v_bf16", q.data_ptr(), 4096, q.data_ptr(), 4096, q.data_ptr(), 4096,
                  o.data_ptr(), 4096, None, 0, 512, 512, 32, 128, 0.088, None, 64, 64, w.data_ptr(), 1e-6,
                  None, None, None, 1, 0, _lib.stream_of(q))


@pytest.mark.parametrize("mode", ["separate", "fused_self_too"])
def test_av_block_query_norm_modes(monkeypatch, mode):
    """The block tests run the default: the query norm fused into the
    cross-attentions (text, A2V), the separate in-place pass for the video
    self-attention.  The same full-width MXFP8 AV block with the separate
    pass everywhere (LTX_FUSED_QNORM=0) and with the fused form in the
    self-attention too (LTX_FUSED_QNORM_SELF=1) meets the same gate against
    the oracle."""
    import test_gpu_block as tb
    from ltx_amd.model.transformer import attention as attn_mod

    if mode == "separate":
        monkeypatch.setattr(attn_mod, "FUSED_QNORM", False)
    else:
        monkeypatch.setattr(attn_mod, "FUSED_QNORM_SELF", True)
    gv, rv, ga, ra = tb._run("mxfp8", (9, 16, 24), 68)
    tb._gate(gv, rv, f"AV block video, query norm {mode}")
    tb._gate(ga, ra, f"AV block audio, query norm {mode}")
