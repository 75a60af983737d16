"""Pin oracle.fused_ops with special cases and invariants (no retyped formulas)."""

import math

import numpy as np

from oracle import fused_ops as ofo
from oracle.bf16 import bf16r


def _x(rng, t=8, c=512, s=1.0):
    return bf16r(rng.standard_normal((t, c)).astype(np.float32) * s)


def test_adaln_scale_minus_one_gives_shift(rng):
    x = _x(rng)
    shift = rng.standard_normal(512).astype(np.float32)
    out = ofo.adaln(x, -np.ones(512, np.float32), shift)
    np.testing.assert_array_equal(out, np.broadcast_to(bf16r(shift), x.shape))


def test_adaln_is_scale_invariant_and_unit_rms(rng):
    x = _x(rng)
    z = np.zeros(512, np.float32)
    a = ofo.adaln(x, z, z)
    np.testing.assert_array_equal(ofo.adaln(x * np.float32(8.0), z, z), a)  # exact power-of-two scaling
    np.testing.assert_allclose(np.sqrt((a.astype(np.float64) ** 2).mean(-1)), 1.0, atol=4e-3)
    # round_norm differs from the fused form only through the extra rounding
    b = ofo.adaln(x, z, z, round_norm=True)
    np.testing.assert_array_equal(a, b)  # with zero modulation both are bf16(rms(x))


def test_adaln_no_norm_is_modulation_only(rng):
    x = _x(rng)
    one = np.ones(512, np.float32)
    np.testing.assert_array_equal(ofo.adaln(x, 0 * one, 0 * one, no_norm=True), x)
    np.testing.assert_array_equal(ofo.adaln(x, one, 0 * one, no_norm=True), bf16r(2 * x))


def test_gated_add_special_cases(rng):
    r, b = _x(rng), _x(rng)
    z, one = np.zeros(512, np.float32), np.ones(512, np.float32)
    np.testing.assert_array_equal(ofo.gated_add(r, b, z), r)
    np.testing.assert_array_equal(ofo.gated_add(np.zeros_like(r), b, one), b)
    np.testing.assert_array_equal(ofo.gated_add(np.zeros_like(r), b, 4 * one, round_product=True), bf16r(4 * b))
    # the double-rounded form differs from the single-rounded one somewhere
    g = rng.standard_normal(512).astype(np.float32)
    assert not np.array_equal(ofo.gated_add(r, b, g), ofo.gated_add(r, b, g, round_product=True))


def test_rms_norm_weighted_linear_in_weight(rng):
    x = _x(rng)
    w = np.ones(512, np.float32)
    a = ofo.rms_norm_weighted(x, w)
    np.testing.assert_array_equal(ofo.rms_norm_weighted(x, 2 * w), bf16r(2 * a))


def test_output_norm_zero_modulation_is_layernorm(rng):
    x = _x(rng, s=3.0) + np.float32(5.0)  # nonzero mean exercises the centring
    z = np.zeros((2, 512), np.float32)
    out = ofo.output_norm_modulate(x, z, np.zeros(512, np.float32))
    ln = ofo.layer_norm_bf16(x)
    np.testing.assert_array_equal(out, ln)
    np.testing.assert_allclose(ln.astype(np.float64).mean(-1), 0.0, atol=2e-2)


def test_euler_edge_cases(rng):
    lat, vel = _x(rng), _x(rng)
    # last distilled step (sigma_next = 0) returns the X0 prediction
    np.testing.assert_array_equal(ofo.euler_x0_step(lat, vel, 0.421875, 0.0),
                                  bf16r((lat - (np.float32(0.421875) * vel).astype(np.float32)).astype(np.float32)))
    # zero velocity keeps the latent
    np.testing.assert_array_equal(ofo.euler_x0_step(lat, np.zeros_like(vel), 1.0, 0.99375), lat)


def test_timestep_embedding_closed_form():
    vals = np.array([0.0, 0.5, 1.0], np.float32)
    emb = ofo.timestep_embedding(vals)
    assert emb.shape == (3, 256)
    np.testing.assert_array_equal(emb[0, :128], 1.0)  # cos(0)
    np.testing.assert_array_equal(emb[0, 128:], 0.0)  # sin(0)
    for j, v in enumerate(vals):
        for i in (0, 1, 64, 127):
            arg = v * 1000.0 * math.exp(-math.log(10000.0) * i / 128)
            assert abs(emb[j, i] - math.cos(arg)) < 2e-4 and abs(emb[j, 128 + i] - math.sin(arg)) < 2e-4


def test_linear_f32_silu_flags(rng):
    x = rng.standard_normal((1, 16)).astype(np.float32)
    W = bf16r(rng.standard_normal((4, 16)).astype(np.float32))
    y = ofo.linear_f32(x, W, None, silu_in=True)
    ref = (x / (1 + np.exp(-x.astype(np.float64)))) @ W.T.astype(np.float64)
    np.testing.assert_allclose(y, ref, rtol=1e-6)
