"""Pin oracle.bf16 against torch's bfloat16 cast (a library routine)."""

import numpy as np
import torch

from oracle.bf16 import bf16r, from_bf16_bits, to_bf16_bits


def _torch_round(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def test_random_values_match_torch(rng):
    a = (rng.standard_normal(200_000) * np.exp(rng.uniform(-30, 30, 200_000))).astype(np.float32)
    np.testing.assert_array_equal(bf16r(a).view(np.uint32), _torch_round(a).view(np.uint32))


def test_ties_round_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1.0078125 -> even (1.0)
    base = np.float32(1.0)
    half = np.float32(2.0 ** -8)
    assert bf16r(base + half) == 1.0
    # 1.0078125 + half is a tie between odd 1.0078125 and even 1.015625 -> 1.015625
    assert bf16r(np.float32(1.0078125) + half) == np.float32(1.015625)
    a = np.array([1.0 + 2.0 ** -8, -(1.0 + 2.0 ** -8), 3.0 * 2.0 ** -9 + 1.0], np.float32)
    np.testing.assert_array_equal(bf16r(a), _torch_round(a))


def test_special_values():
    a = np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-45,
                  np.finfo(np.float32).max], np.float32)
    np.testing.assert_array_equal(bf16r(a).view(np.uint32), _torch_round(a).view(np.uint32))
    assert np.isnan(bf16r(np.array([np.nan], np.float32)))[0]


def test_bits_roundtrip(rng):
    bits = rng.integers(0, 2 ** 16, 10_000, dtype=np.uint16)
    vals = from_bf16_bits(bits)
    finite = np.isfinite(vals)
    np.testing.assert_array_equal(to_bf16_bits(vals[finite]), bits[finite])
