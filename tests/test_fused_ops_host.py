"""Host-side behaviour of the drop-in fused ops: the reference's shape/dtype
gates and fallbacks (LTX_2_MLX tests/test_fused_ops.py:75-142, :162-217;
tests/test_precision_plumbing.py:162-180), on CPU tensors."""

import atexit

import numpy as np
import torch

from _util import ulp_diff_bf16


def _same_bf16(got, ref):
    """Equal up to the fp32-vs-float64 evaluation of the modulation: at most
    one bf16 ulp, on a vanishing fraction of elements."""
    d = ulp_diff_bf16(got, ref)
    assert d.max() <= 1 and (d == 0).mean() >= 0.999

from ltx_amd.kernels import fused_ops as F
from oracle import fused_ops as ofo

T, C = 64, 4096


def _inputs(seed=42, t=T, c=C):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((1, t, c), generator=g).bfloat16()
    scale = torch.randn((1, 1, c), generator=g) * 0.1
    shift = torch.randn((1, 1, c), generator=g) * 0.1
    gate = torch.randn((1, 1, c), generator=g) * 0.5
    res = torch.randn((1, t, c), generator=g).bfloat16()
    br = torch.randn((1, t, c), generator=g).bfloat16()
    return x, scale, shift, gate, res, br


def test_gate_predicates_accept_production_shapes():
    x, sc, sh, g, r, b = _inputs()
    assert F._adaln_t2v_broadcast_compatible(x, sc, sh)
    assert F._adaln_t2v_broadcast_compatible(x[..., :2048].contiguous(), sc[..., :2048], sh[..., :2048])
    assert F._gated_add_t2v_broadcast_compatible(r, b, g)
    assert F._adaln_t2v_broadcast_compatible(x, sc.reshape(-1), sh.reshape(1, -1))


def test_gate_predicates_reject_like_the_reference():
    x, sc, sh, g, r, b = _inputs()
    assert not F._adaln_t2v_broadcast_compatible(x.float(), sc, sh)            # fp32 x
    assert not F._adaln_t2v_broadcast_compatible(x, sc.expand(1, T, C), sh)    # per-token scale
    assert not F._adaln_t2v_broadcast_compatible(x, sc.bfloat16(), sh)         # bf16 scale
    x3 = torch.zeros((1, 8, 3584), dtype=torch.bfloat16)
    assert not F._adaln_t2v_broadcast_compatible(x3, torch.zeros(3584), torch.zeros(3584))  # C=3584
    assert not F._gated_add_t2v_broadcast_compatible(r, b, g.expand(1, T, C))
    assert not F._gated_add_t2v_broadcast_compatible(r, b[:, :-1], g)
    assert not F._gated_add_t2v_broadcast_compatible(r.float(), b, g)


def test_fallbacks_follow_reference_expressions():
    x, sc, sh, g, r, b = _inputs()
    # fp32 x -> fallback keeps fp32 (reference test_adaln_fallback_on_fp32_x)
    y = F.adaln_norm_fused(x.float(), sc, sh, 1e-6)
    assert y.dtype == torch.float32
    # per-token scale -> fallback equals the inline form (rms_norm bf16, then modulate)
    y = F.adaln_norm_fused(x, sc.expand(1, T, C), sh.expand(1, T, C), 1e-6)
    ref = ofo.adaln(x.float().numpy()[0], sc.numpy().reshape(-1), sh.numpy().reshape(-1), round_norm=True)
    _same_bf16(y.float().numpy()[0], ref)
    # non-default eps forces the fallback (test_precision_plumbing.py:162-180)
    y = F.adaln_norm_fused(x, sc, sh, 1e-5)
    ref = ofo.adaln(x.float().numpy()[0], sc.numpy().reshape(-1), sh.numpy().reshape(-1), 1e-5, round_norm=True)
    _same_bf16(y.float().numpy()[0], ref)
    # gated add fallback
    z = F.gated_add_fused(r, b, g.expand(1, T, C))
    refz = ofo.gated_add(r.float().numpy()[0], b.float().numpy()[0], g.numpy().reshape(-1))
    _same_bf16(z.float().numpy()[0], refz)


def test_kernel_path_refuses_host_tensors():
    """The kernel path never silently falls back: host tensors raise."""
    x, sc, sh, g, r, b = _inputs()
    import pytest

    from ltx_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    with pytest.raises(ValueError):
        F.adaln_norm_fused(x, sc, sh, 1e-6)
    with pytest.raises(ValueError):
        F.gated_add_fused(r, b, g)


def test_dispatch_tally_counts_fallbacks_and_reports(monkeypatch, capsys):
    """``LTX_FUSED_PROBE``: per-operator kernel/fallback tally (reference
    kernels/fused_ops.py:12-69); gate-rejected calls count as fallbacks."""
    monkeypatch.setenv("LTX_FUSED_PROBE", "1")
    tally = F._DispatchTally(("adaln", "gated_add"))
    atexit.unregister(tally.report)  # reported below instead of at exit
    monkeypatch.setattr(F, "_TALLY", tally)
    x, sc, sh, gate, res, br = _inputs()
    F.adaln_norm_fused(x, sc, sh, 1e-5)  # eps != 1e-6 -> fallback
    F.adaln_norm_fused(x.float(), sc, sh, 1e-6)  # fp32 x -> fallback
    F.gated_add_fused(res, br, gate.bfloat16())  # bf16 gate -> fallback
    assert F.get_dispatch_counts() == {"adaln_kernel": 0, "adaln_fallback": 2,
                                       "gated_add_kernel": 0, "gated_add_fallback": 1}
    tally.hit("adaln", "kernel")
    tally.report()
    out = capsys.readouterr().out
    assert "adaln: 1 on the HIP kernel, 2 on the fallback (33.3% kernel)" in out
    assert "gated_add: 0 on the HIP kernel, 1 on the fallback (0.0% kernel)" in out
    monkeypatch.delenv("LTX_FUSED_PROBE")
    quiet = F._DispatchTally(("adaln",))
    quiet.hit("adaln", "kernel")
    assert quiet.counts() == {"adaln_kernel": 0, "adaln_fallback": 0}
