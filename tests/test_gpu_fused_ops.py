"""GPU parity of the bandwidth-bound kernels against the oracle.

Tolerances: each output is one bf16 rounding of an fp32 expression, so the
kernel may differ from the float64 oracle by at most 1 bf16 ulp where the
fp32 evaluation order moves a value across a rounding boundary; the
bf16 tolerance gate (max relative error <= 1e-2, cosine >= 0.9999 as in the
reference's tests/test_fused_ops.py:72) is checked as well.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import bf16_from_torch, cos_sim, max_rel_err, ulp_diff_bf16
from oracle import fused_ops as ofo
from oracle import rope as orope
from oracle.bf16 import bf16r, ulp_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _bf(rng, shape, scale=1.0):
    return bf16r(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


def _t(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def _assert_close_bf16(got, ref, max_ulp=1, min_exact=0.99, atol=4e-6):
    """|got - ref| <= max_ulp bf16 ulps of ref + atol.  The atol covers
    results that cancel to near zero, where the fp32 evaluation error of the
    terms (~2^-24 of their magnitude) exceeds a bf16 ulp of the result."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    bound = max_ulp * ulp_bf16(ref) + atol
    err = np.abs(got.astype(np.float64) - ref)
    worst = int(np.argmax(err - bound))
    assert np.all(err <= bound), (
        f"err {err.flat[worst]:.3g} > bound {bound.flat[worst]:.3g} at {worst} "
        f"(got {got.flat[worst]}, ref {ref.flat[worst]})")
    d = ulp_diff_bf16(got, ref)
    assert (d == 0).mean() >= min_exact, f"exact fraction {(d == 0).mean()}"
    assert max_rel_err(got, ref) <= 1e-2
    assert cos_sim(got, ref) >= 0.9999


@pytest.mark.parametrize("T,C", [(1296, 4096), (1024, 2048), (2900, 2048), (3456, 4096), (14640, 4096)])
def test_adaln_kernel_matches_oracle(T, C):
    from ltx_amd.kernels.fused_ops import adaln_norm_fused, get_dispatch_counts  # noqa: F401

    rng = np.random.default_rng(42 + T)
    x = _bf(rng, (1, T, C))
    table = bf16r(rng.standard_normal((6, C)).astype(np.float32) * np.float32(0.1))
    shift, scale = table[0], table[1]
    out = adaln_norm_fused(_t(x), _t(scale, torch.float32).view(1, 1, C), _t(shift, torch.float32).view(1, 1, C), 1e-6)
    assert out.dtype == torch.bfloat16 and out.shape == (1, T, C)
    ref = ofo.adaln(x[0], scale, shift)
    _assert_close_bf16(bf16_from_torch(out)[0], ref)


@pytest.mark.parametrize("flags", [1, 2])
def test_adaln_kernel_flag_forms(flags):
    from ltx_amd import _lib
    from ltx_amd.kernels.fused_ops import adaln_rows

    rng = np.random.default_rng(7)
    T, C = 300, 4096
    x = _bf(rng, (T, C), 2.0)
    scale = rng.standard_normal(C).astype(np.float32) * 0.1
    shift = rng.standard_normal(C).astype(np.float32) * 0.1
    xt = _t(x)
    out = torch.empty_like(xt)
    adaln_rows(xt, C, _t(scale, torch.float32), _t(shift, torch.float32), out, C, T, C, 1e-6, flags)
    torch.cuda.synchronize()
    ref = ofo.adaln(x, scale, shift, round_norm=bool(flags & _lib.ADALN_ROUND_NORM),
                    no_norm=bool(flags & _lib.ADALN_NO_NORM))
    _assert_close_bf16(bf16_from_torch(out), ref)


@pytest.mark.parametrize("T,C,flags", [(3456, 4096, 1), (68, 2048, 1), (20000, 4096, 0), (300, 4096, 2)])
def test_adaln_two_outputs_equal_two_single_calls(T, C, flags):
    """The two-output AdaLN (A2V and V2A inputs of one stream) equals two
    single-output calls bit for bit (those are checked against the oracle
    above), over the large-workgroup and the grid-stride launch forms."""
    from ltx_amd.kernels.fused_ops import adaln_rows, adaln_rows2

    rng = np.random.default_rng(T + C + flags)
    x = _bf(rng, (T, C), 2.0)
    s1, h1, s2, h2 = (_t(rng.standard_normal(C).astype(np.float32) * 0.1, torch.float32) for _ in range(4))
    xt = _t(x)
    a, b = torch.empty_like(xt), torch.empty_like(xt)
    adaln_rows2(xt, C, s1, h1, a, s2, h2, b, T, C, 1e-6, flags)
    ra, rb = torch.empty_like(xt), torch.empty_like(xt)
    adaln_rows(xt, C, s1, h1, ra, C, T, C, 1e-6, flags)
    adaln_rows(xt, C, s2, h2, rb, C, T, C, 1e-6, flags)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), ra.view(torch.int16))
    assert torch.equal(b.view(torch.int16), rb.view(torch.int16))


def test_adaln_special_cases_exact():
    """scale = -1 makes the output exactly bf16(shift); zero modulation gives
    the plain RMSNorm."""
    from ltx_amd.kernels.fused_ops import adaln_norm_fused

    rng = np.random.default_rng(3)
    T, C = 64, 2048
    x = _bf(rng, (1, T, C))
    shift = rng.standard_normal(C).astype(np.float32)
    out = adaln_norm_fused(_t(x), torch.full((1, 1, C), -1.0, device=DEV), _t(shift, torch.float32).view(1, 1, C), 1e-6)
    np.testing.assert_array_equal(bf16_from_torch(out)[0], np.broadcast_to(bf16r(shift), (T, C)))
    zero = torch.zeros((1, 1, C), device=DEV)
    out = adaln_norm_fused(_t(x), zero, zero, 1e-6)
    rms = np.sqrt(np.mean(bf16_from_torch(out)[0].astype(np.float64) ** 2, axis=-1))
    np.testing.assert_allclose(rms, 1.0, atol=5e-3)


def test_adaln_strided_rows_and_in_place():
    from ltx_amd.kernels.fused_ops import adaln_rows

    rng = np.random.default_rng(11)
    T, C, stride = 100, 2048, 2048 * 3
    big = _bf(rng, (T, stride))
    xt = _t(big)
    scale = _t(rng.standard_normal(C).astype(np.float32) * 0.1, torch.float32)
    shift = _t(rng.standard_normal(C).astype(np.float32) * 0.1, torch.float32)
    view = xt[:, C:2 * C]
    adaln_rows(view, stride, scale, shift, view, stride, T, C, 1e-6, 0)
    got = bf16_from_torch(xt)
    ref = ofo.adaln(big[:, C:2 * C], scale.cpu().numpy(), shift.cpu().numpy())
    _assert_close_bf16(got[:, C:2 * C], ref)
    np.testing.assert_array_equal(got[:, :C], big[:, :C])
    np.testing.assert_array_equal(got[:, 2 * C:], big[:, 2 * C:])


@pytest.mark.parametrize("T,C", [(1296, 4096), (1024, 2048), (14640, 4096)])
def test_gated_add_kernel_matches_oracle(T, C):
    from ltx_amd.kernels.fused_ops import gated_add_fused

    rng = np.random.default_rng(5 + T)
    res = _bf(rng, (1, T, C))
    br = _bf(rng, (1, T, C))
    gate = rng.standard_normal(C).astype(np.float32) * 0.5
    out = gated_add_fused(_t(res), _t(br), _t(gate, torch.float32).view(1, 1, C))
    ref = ofo.gated_add(res[0], br[0], gate)
    _assert_close_bf16(bf16_from_torch(out)[0], ref)


def test_gated_add_special_cases_exact():
    from ltx_amd.kernels.fused_ops import gated_add_fused, gated_add_rows

    rng = np.random.default_rng(9)
    T, C = 77, 4096
    res = _bf(rng, (1, T, C))
    br = _bf(rng, (1, T, C))
    zero = torch.zeros((1, 1, C), device=DEV)
    out = gated_add_fused(_t(res), _t(br), zero)
    np.testing.assert_array_equal(bf16_from_torch(out), res)
    one = torch.ones((1, 1, C), device=DEV)
    out = gated_add_fused(torch.zeros((1, T, C), dtype=torch.bfloat16, device=DEV), _t(br), one)
    np.testing.assert_array_equal(bf16_from_torch(out), br)
    # round-product form, in place on the residual
    gate = rng.standard_normal(C).astype(np.float32) * 0.3
    rt = _t(res[0])
    gated_add_rows(rt, C, _t(br[0]), C, _t(gate, torch.float32), rt, C, T, C, 1)
    ref = ofo.gated_add(res[0], br[0], gate, round_product=True)
    _assert_close_bf16(bf16_from_torch(rt), ref)


def _qk_case(T_q, T_k, D, heads, tables_q, tables_k, stride_mult=1, seed=0):
    from ltx_amd.kernels import rope_ops

    rng = np.random.default_rng(seed)
    q = _bf(rng, (T_q, D * stride_mult), 3.0)
    k = _bf(rng, (T_k, D * stride_mult), 3.0)
    wq = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    wk = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    qt, kt = _t(q), _t(k)
    qv, kv = qt[:, :D], kt[:, :D]
    cq = None if tables_q is None else tuple(_t(a, torch.float32) for a in tables_q)
    ck = None if tables_k is None else tuple(_t(a, torch.float32) for a in tables_k)
    rope_ops.qknorm_rope_(qv, _t(wq, torch.float32), cq, kv, _t(wk, torch.float32), ck, heads)
    torch.cuda.synchronize()
    gq = bf16_from_torch(qt)[:, :D]
    gk = bf16_from_torch(kt)[:, :D]
    rq = orope.qknorm_rope(q[:, :D], wq, *(tables_q or (None, None)), heads)
    rk = orope.qknorm_rope(k[:, :D], wk, *(tables_k or (None, None)), heads)
    # The normalised values are rounded to bf16 before the rotation, so a
    # one-ulp difference there (|x| <= ~4 -> ulp <= 2^-5) can move a rotated
    # output by up to ~0.04 even when the output itself is small.
    _assert_close_bf16(gq, rq, max_ulp=2, min_exact=0.98, atol=0.04)
    _assert_close_bf16(gk, rk, max_ulp=2, min_exact=0.98, atol=0.04)
    if stride_mult > 1:  # untouched tail of each row
        np.testing.assert_array_equal(bf16_from_torch(qt)[:, D:], q[:, D:])


def test_qknorm_rope_video_self():
    pos = orope.video_positions(9, 16, 24, fps=24.0)
    tab = orope.rope_tables(pos, 4096, 32, orope.VIDEO_MAX_POS)
    _qk_case(3456, 3456, 4096, 32, tab, tab, stride_mult=3)


def test_qknorm_rope_audio_self_and_cross():
    apos = orope.audio_positions(68)
    atab = orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS)
    _qk_case(68, 68, 2048, 32, atab, atab, seed=1)
    vpos = orope.video_positions(9, 16, 24, fps=24.0)
    vx = orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS)
    _qk_case(3456, 68, 2048, 32, vx, atab, seed=2)  # A2V: q video cross PE, k audio cross PE
    _qk_case(68, 3456, 2048, 32, atab, vx, seed=3)  # V2A


def test_qknorm_rope_factored_tables_bit_identical():
    """Tables factored over the position axes (stacked per-axis rows + a row
    index per token and axis) give the same bits as the per-token tables:
    video self-attention (3 axes, Q and K in one fused buffer, shared table),
    A2V / V2A (time-only video tables, 1 axis, against per-token audio
    tables), and 768x512x121's 6144 tokens."""
    from ltx_amd.kernels.rope_ops import qknorm_rope_
    from ltx_amd.model.transformer import rope as prope

    def dev(tab):
        return tuple(torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in tab)

    def factored(pos, dim, mp):
        full = prope.rope_tables_np(pos, dim, mp)
        return dev(full), dev(prope.factor_tables_np(pos, *full))

    def run(tq, tk, d, variants, seed):
        rng = np.random.default_rng(seed)
        buf = _t(_bf(rng, (max(tq, tk), 3 * d), 3.0))
        wq = _t(rng.uniform(0.5, 1.5, d).astype(np.float32), torch.float32)
        wk = _t(rng.uniform(0.5, 1.5, d).astype(np.float32), torch.float32)
        outs = []
        for pq, pk in variants:
            b = buf.clone()
            qknorm_rope_(b[:tq, :d], wq, pq, b[:tk, d:2 * d], wk, pk, 32)
            outs.append(b)
        torch.cuda.synchronize()
        assert not torch.equal(outs[0], buf)
        for o in outs[1:]:
            assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))

    for grid in ((9, 16, 24), (16, 16, 24)):
        vpos = orope.video_positions(*grid, fps=24.0)
        t = int(np.prod(grid))
        full, fac = factored(vpos, 4096, orope.VIDEO_MAX_POS)
        assert fac[2].shape == (t, 3)
        run(t, t, 4096, [(full, full), (fac, fac)], seed=grid[0])
        xfull, xfac = factored(vpos[:, 0:1], 2048, orope.AUDIO_MAX_POS)
        assert xfac[2].shape == (t, 1)
        apos = orope.audio_positions(68)
        atab = dev(prope.rope_tables_np(apos, 2048, orope.AUDIO_MAX_POS))
        run(t, 68, 2048, [(xfull, atab), (xfac, atab)], seed=grid[0] + 1)  # A2V
        run(68, t, 2048, [(atab, xfull), (atab, xfac)], seed=grid[0] + 2)  # V2A


def test_qknorm_no_rope_text():
    _qk_case(3456, 256, 4096, 32, None, None, seed=4)
    _qk_case(68, 256, 2048, 32, None, None, seed=5)


def test_qknorm_rope_two_passes_unequal_operands():
    """More rows than one pass of the 16-wave grid holds (4096 tasks), with
    unequal operands: the paired Q / K tasks, then the longer operand's
    remaining rows, each run once (RoPE on Q only, no RoPE on K)."""
    pos = orope.video_positions(10, 20, 25, fps=24.0)
    tab = orope.rope_tables(pos, 2048, 32, orope.VIDEO_MAX_POS)
    _qk_case(5000, 2100, 2048, 32, tab, None, seed=6)
    _qk_case(1900, 5100, 2048, 32, None, None, seed=7)


def test_output_norm_modulate():
    from ltx_amd import _lib

    rng = np.random.default_rng(21)
    T, C = 3456, 4096
    x = _bf(rng, (T, C), 4.0)
    table = rng.standard_normal((2, C)).astype(np.float32) * 0.05
    emb = rng.standard_normal(C).astype(np.float32) * 0.5
    xt, tt, et = _t(x), _t(table, torch.float32), _t(emb, torch.float32)  # keep alive until sync
    out = torch.empty_like(xt)
    _lib.call("ltx_output_norm_modulate_bf16", xt.data_ptr(), C, tt.data_ptr(),
              et.data_ptr(), out.data_ptr(), C, T, C, 1e-6, _lib.stream_of(xt))
    torch.cuda.synchronize()
    ref = ofo.output_norm_modulate(x, table, emb)
    # Three chained bf16 roundings (norm, product, sum): a one-ulp difference
    # of the normalised value (|n| <= ~5 -> ulp <= 2^-5) passes through the
    # product and can exceed an ulp of a small output after the shift.
    _assert_close_bf16(bf16_from_torch(out), ref, max_ulp=2, min_exact=0.98, atol=0.035)


def test_euler_x0_step_bitexact():
    from ltx_amd import _lib

    rng = np.random.default_rng(8)
    n = 3456 * 128 + 5
    lat = _bf(rng, (n,))
    vel = _bf(rng, (n,))
    for s, sn in [(1.0, 0.99375), (0.909375, 0.725), (0.421875, 0.0)]:
        lt, vt = _t(lat), _t(vel)
        out = torch.empty_like(lt)
        _lib.call("ltx_euler_x0_step_bf16", lt.data_ptr(), vt.data_ptr(), float(s), float(np.float32(sn / s)),
                  out.data_ptr(), n, _lib.stream_of(lt))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bf16_from_torch(out), ofo.euler_x0_step(lat, vel, s, sn))


def test_timestep_embedding_and_gemv():
    from ltx_amd import _lib

    vals = np.array([1.0, 0.5, 0.0, 0.421875], np.float32)
    vt = _t(vals, torch.float32)
    out = torch.empty((4, 256), device=DEV)
    _lib.call("ltx_timestep_embedding_f32", vt.data_ptr(), 4, 1000.0, out.data_ptr(), 256, _lib.stream_of(vt))
    torch.cuda.synchronize()
    ref = ofo.timestep_embedding(vals)
    # t*1000 ~ 1e3 has an fp32 ulp of 6e-5; a one-ulp difference of exp()
    # (the reference evaluates it in fp32 on the GPU too) moves sin/cos by that much.
    np.testing.assert_allclose(out.cpu().numpy(), ref, atol=1.5e-4, rtol=0)

    rng = np.random.default_rng(2)
    K, N = 4096, 9 * 4096 + 3
    W = _bf(rng, (N, K), 0.02)
    b = rng.standard_normal(N).astype(np.float32) * 0.02
    x = rng.standard_normal((2, K)).astype(np.float32)
    y = torch.empty((2, N), device=DEV)
    Wt, bt, xt = _t(W), _t(b, torch.float32), _t(x, torch.float32)
    _lib.call("ltx_gemv_f32_bf16w", xt.data_ptr(), 2, K, Wt.data_ptr(), bt.data_ptr(), y.data_ptr(), N,
              _lib.GEMV_SILU_INPUT, _lib.stream_of(xt))
    torch.cuda.synchronize()
    ref = ofo.linear_f32(x, W, b, silu_in=True)
    assert max_rel_err(y.cpu().numpy(), ref) < 1e-4


def test_device_clock_stamp_eager_and_in_graph():
    """Stamps are stream-ordered: eager stamps around a busy kernel advance, and
    a stamp pair captured in a HIP graph brackets the work between them on
    every replay (later replays read later times)."""
    from ltx_amd import _lib

    st = torch.zeros(4, dtype=torch.int64, device=DEV)
    a = torch.randn((2048, 2048), device=DEV)
    c = torch.zeros_like(a)
    s = torch.cuda.current_stream().cuda_stream
    _lib.call("ltx_device_clock_stamp", st.data_ptr(), s)
    for _ in range(20):
        c.add_(a)
    _lib.call("ltx_device_clock_stamp", st.data_ptr() + 8, s)
    torch.cuda.synchronize()
    t = st.tolist()
    assert t[1] > t[0] > 0

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = torch.cuda.current_stream().cuda_stream
        _lib.call("ltx_device_clock_stamp", st.data_ptr() + 16, cs)
        for _ in range(20):
            c.add_(a)
        _lib.call("ltx_device_clock_stamp", st.data_ptr() + 24, cs)
    prev = None
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        t = st.tolist()
        assert t[3] > t[2] > 0
        if prev is not None:
            assert t[2] > prev
        prev = t[3]
    # the stamp pair spans the twenty elementwise kernels: at least a few microseconds on
    # the 100 MHz-class counter, far less than a second
    assert 10 < t[3] - t[2] < 100_000_000
