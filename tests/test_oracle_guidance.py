"""Pin the guided-loop oracle (oracle/guidance.py) and the host-side sigma
schedule; CPU only."""

import numpy as np
import pytest
import torch

from oracle import guidance as og
from oracle.bf16 import bf16r


def _lat(rng, shape=(37, 128)):
    return rng.standard_normal(shape).astype(np.float32)


def test_neutral_and_cancelling_guidance(rng):
    c, u, p = _lat(rng), _lat(rng), _lat(rng)
    np.testing.assert_array_equal(og.guide(c, (u,), (0.0,)), c)                     # scale 1 CFG
    np.testing.assert_array_equal(og.guide(c, (c,), (2.0,)), c)                     # uncond == cond
    np.testing.assert_array_equal(og.guide(c, (u, p, u), (0.0, 0.0, 0.0)), c)       # multi-modal neutral
    np.testing.assert_array_equal(og.guide(c, (u,), (2.5,), delta_only=True) * 0, np.zeros_like(c))
    np.testing.assert_array_equal(og.guide(c, (None, None, p), (0.0, 0.0, 0.0)), c)


def test_cfg_star_rescales_onto_cond(rng):
    c = bf16r(_lat(rng))
    u = (2.0 * c).astype(np.float32)
    coef = og.projection_coef(c, u)
    assert abs(float(coef) - 0.5) < 1e-6
    # coef * u is cond up to the coefficient's rounding: the delta vanishes
    d = og.guide(c, (u,), (2.0,), coef=np.float32(0.5), delta_only=True)
    np.testing.assert_array_equal(d, np.zeros_like(c))


def test_projection_coef_closed_form():
    a = np.array([1.0, 2.0, 3.0], np.float32)
    b = np.array([2.0, 0.0, 1.0], np.float32)
    assert og.projection_coef(a, b) == np.float32(np.float32(5.0) / np.float32(5.0 + 1e-8))


def test_std_ratio_halves_a_doubled_prediction(rng):
    c = _lat(rng)
    f = og.std_ratio(c, 2.0 * c, 1.0)
    assert abs(float(f) - 0.5) < 1e-6
    assert og.std_ratio(c, 2.0 * c, 0.0) == np.float32(1.0)  # rescale 0: factor 1


def test_euler_and_ge_special_cases(rng):
    x, d = bf16r(_lat(rng)), _lat(rng)
    np.testing.assert_array_equal(og.euler(x, d, 0.5, 0.0), bf16r(d))   # last step: the denoised latent
    np.testing.assert_array_equal(og.euler(x, x, 0.7, 0.3), x)          # denoised == sample
    d2, cur = og.ge_correct(x, d, None, False, 0.8, 0.5)
    np.testing.assert_array_equal(d2, d)                                # first step: only records
    d3, cur2 = og.ge_correct(x, d, cur, True, 0.8, 1.0)                 # gamma 1: total = cur
    assert np.abs(d3 - d).max() <= 4 * np.abs(d).max() * 2 ** -23 + 4 * np.abs(x).max() * 2 ** -23


@pytest.mark.parametrize("scale", [3.0, 7.0, 1.0])
def test_guide_forms_match_torch_float32(rng, scale):
    """The reference's expressions evaluated by torch in float32 (a python
    float scalar meets a float32 tensor as float32, as in MLX)."""
    c, u, p, m = (torch.from_numpy(_lat(rng)) for _ in range(4))
    cfg = c + (scale - 1) * (c - u)
    np.testing.assert_array_equal(og.guide(c.numpy(), (u.numpy(),), (scale - 1,)), cfg.numpy())
    stg = cfg + 0.7 * (cfg - p)
    np.testing.assert_array_equal(og.guide(cfg.numpy(), (p.numpy(),), (0.7,)), stg.numpy())
    coef = torch.tensor(0.3125)
    star = c + (scale - 1) * (c - coef * u)
    np.testing.assert_array_equal(og.guide(c.numpy(), (u.numpy(),), (scale - 1,), coef=0.3125), star.numpy())
    mm = c + (scale - 1) * (c - u)
    mm = mm + 0.4 * (c - p)
    mm = mm + (2.0 - 1) * (c - m)
    got = og.guide(c.numpy(), (u.numpy(), p.numpy(), m.numpy()), (scale - 1, 0.4, 1.0))
    np.testing.assert_array_equal(got, mm.numpy())
    x = torch.from_numpy(bf16r(_lat(rng)))
    r = torch.tensor(np.float32(0.725 / 0.909375))
    eul = (c + r * (x - c)).bfloat16().float()
    np.testing.assert_array_equal(og.euler(x.numpy(), c.numpy(), 0.909375, 0.725), eul.numpy())


# -- LTX2Scheduler (components/schedulers.py:10-95; invariants of tests/test_scheduler.py) --
@pytest.mark.parametrize("steps", [10, 20, 25, 30, 50])
def test_ltx2_scheduler_invariants(steps):
    from ltx_amd.components.schedulers import LTX2Scheduler

    s = LTX2Scheduler().execute(steps=steps)
    assert s.dtype == np.float32 and s.shape == (steps + 1,)
    assert np.all(s[:-1] >= s[1:])
    assert s[0] == 1.0 and s[-1] == 0.0
    assert abs(float(s[steps - 1]) - 0.1) < 1e-6  # stretched to the terminal value
    assert np.all((s >= 0) & (s <= 1))


def test_ltx2_scheduler_shift_closed_form():
    """At the max-shift anchor (4096 tokens) the shift is max_shift: before the
    stretch, sigma(0.5) = e^2.05 / (e^2.05 + 1)."""
    from ltx_amd.components.schedulers import LTX2Scheduler

    s = LTX2Scheduler().execute(steps=2, stretch=False)
    e = np.float32(np.exp(2.05))
    assert s[1] == np.float32(e / (e + np.float32(1.0)))
    lat = np.zeros((1, 128, 2, 16, 32))  # 1024 tokens: the base-shift anchor
    s2 = LTX2Scheduler().execute(steps=2, latent=lat, stretch=False)
    e2 = np.float32(np.exp(0.95))
    assert s2[1] == np.float32(e2 / (e2 + np.float32(1.0)))


def test_ltx2_scheduler_one_step_stretch_is_nan():
    """One step: the last non-zero sigma is sigma_0 = 1, so the stretch divides
    0 by 0 (components/schedulers.py:74-89); the first sigma is NaN, silently,
    and the shift alone (stretch off) is finite."""
    import warnings

    from ltx_amd.components.schedulers import LTX2Scheduler

    with warnings.catch_warnings():
        warnings.simplefilter("error")
        s = LTX2Scheduler().execute(steps=1)
    assert np.isnan(s[0]) and s[1] == 0.0
    np.testing.assert_array_equal(LTX2Scheduler().execute(steps=1, stretch=False), np.float32([1.0, 0.0]))
