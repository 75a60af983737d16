"""Host logic of the Modality-level forward (no GPU): context-mask handling
and the one-timestep rule.

* ``context_keep_rows``: which context rows a (B, S) mask keeps -- boolean
  masks (True = attend, as model.py:208-250 reads them), additive masks of
  0 / large negative entries; unsupported masks are refused.
* Dropping the masked keys is exactly the masked softmax: checked by brute
  force in float64 and float32 against an attention that adds the
  reference's -3.4e38 mask entries to the scores (pins the equivalence the
  GPU path relies on, including that a mask which drops a key changes the
  result).
* ``_uniform_value``: one timestep where the forward needs one (per sample,
  per audio token); ``token_timestep_groups``: per-token video timesteps as
  (row range, group) segments.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ltx_amd.model.transformer.model import MASK_EXCLUDE, _uniform_value, context_keep_rows


def test_no_mask_keeps_everything():
    assert context_keep_rows(None, 3, 10) == [None, None, None]


def test_boolean_masks():
    m = torch.tensor([[True] * 6 + [False] * 2, [True] * 8])
    keep = context_keep_rows(m, 2, 8)
    assert keep[0].tolist() == list(range(6)) and keep[1] is None
    holes = torch.tensor([True, False, True, True, False, True, False, True])
    assert context_keep_rows(holes, 2, 8)[1].tolist() == [0, 2, 3, 5, 7]  # one row broadcast to the batch
    ints = torch.tensor([[1, 0, 1, 1]])
    assert context_keep_rows(ints, 1, 4)[0].tolist() == [0, 2, 3]


def test_additive_masks():
    m = torch.tensor([[0.0, float("-inf"), 0.0, -3.4e38, MASK_EXCLUDE, 0.0]])
    assert context_keep_rows(m, 1, 6)[0].tolist() == [0, 2, 5]
    assert context_keep_rows(torch.zeros((1, 4), dtype=torch.bfloat16), 1, 4) == [None]


@pytest.mark.parametrize("mask,length", [
    (torch.tensor([[0.0, -5.0, 0.0]]), 3),            # a soft additive bias
    (torch.tensor([[False, False, False]]), 3),        # every key dropped
    (torch.ones((1, 1, 4, 4), dtype=torch.bool), 4),   # (B, 1, S, S) mask
    (torch.ones((1, 5), dtype=torch.bool), 4),         # wrong length
    (torch.ones((3, 4), dtype=torch.bool), 4),         # three masks for two samples
])
def test_unsupported_masks_are_refused(mask, length):
    with pytest.raises(NotImplementedError):
        context_keep_rows(mask, 2, length)


def _masked_attention(q, k, v, add):
    s = q @ k.T + add[None, :]
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    return (p @ v) / p.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-12), (np.float32, 1e-6)])
def test_dropping_masked_keys_is_the_masked_softmax(dtype, tol):
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((n, 16)).astype(dtype) for n in (5, 12, 12))
    q *= dtype(3.0)  # peaked weights
    keep = np.array([0, 1, 4, 5, 6, 9, 11])
    add = np.full(12, -3.4e38, dtype)
    add[keep] = 0
    masked = _masked_attention(q, k, v, add)
    dropped = _masked_attention(q, k[keep], v[keep], np.zeros(len(keep), dtype))
    np.testing.assert_allclose(masked, dropped, rtol=tol, atol=tol)
    # a dropped key contributes nothing: its weight is exactly zero
    s = q @ k.T + add[None, :]
    assert (np.exp(s - s.max(axis=1, keepdims=True))[:, np.setdiff1d(np.arange(12), keep)] == 0).all()
    # and the mask matters here
    assert np.abs(masked - _masked_attention(q, k, v, np.zeros(12, dtype))).max() > 1e-3
    rows = context_keep_rows(torch.from_numpy(add[None].astype(np.float32)), 1, 12)[0]
    assert rows.tolist() == keep.tolist()


def test_one_timestep_per_forward():
    assert _uniform_value(0.5, "t") == 0.5
    assert _uniform_value(torch.full((2, 7), 0.25), "t") == 0.25
    assert _uniform_value(torch.tensor(0.125), "t") == 0.125
    with pytest.raises(NotImplementedError):
        _uniform_value(torch.tensor([0.5, 0.25]), "t")          # per sample
    t = torch.full((1, 6), 0.5)
    t[0, :2] = 0.0                                               # conditioned tokens at t = 0
    with pytest.raises(NotImplementedError):
        _uniform_value(t, "t")


def test_token_timestep_groups():
    from ltx_amd.model.transformer.model import token_timestep_groups

    g = token_timestep_groups(torch.tensor([[0.0, 0.0, 0.6, 0.6, 0.6, 0.0, 0.6]]))
    assert g.values == [0.0, pytest.approx(0.6)]
    assert g.segments == [(0, 2, 0), (2, 5, 1), (5, 6, 0), (6, 7, 1)]
    one = token_timestep_groups(torch.full((5,), 0.25))
    assert one.values == [0.25] and one.segments == [(0, 5, 0)]
    with pytest.raises(ValueError):
        token_timestep_groups(torch.zeros(0))
