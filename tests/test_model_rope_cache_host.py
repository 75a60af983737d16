"""LTXModel.rope: tables are cached per full set of positions.

Two grids with the same token count (landscape 16x24 vs portrait 24x16
latent, 9 frames) share the array shape and their first bytes (the time
bounds of the first frame), yet their spatial RoPE differs; each must get
its own tables.  The cache is bounded.
"""

import numpy as np
import torch

from ltx_amd.model.transformer import model as model_mod
from ltx_amd.model.transformer.model import LTXModel
from ltx_amd.model.transformer.rope import (VIDEO_MAX_POS, audio_positions, expand_tables, rope_tables_np,
                                           video_positions)


def _stub_model(video_dim=256, audio_dim=64):
    m = LTXModel.__new__(LTXModel)  # only the attributes rope() reads
    m.device = torch.device("cpu")
    m.video_dim, m.audio_dim = video_dim, audio_dim
    m.audio_config = object()
    m._rope_cache = {}
    return m


def test_same_shape_same_prefix_positions_get_their_own_tables():
    land, port = video_positions(9, 16, 24, 24.0), video_positions(9, 24, 16, 24.0)
    assert land.shape == port.shape and land.tobytes()[:64] == port.tobytes()[:64]
    assert not np.array_equal(land, port)
    m = _stub_model()
    apos = audio_positions(68)
    pl = m.rope(land, apos)
    pp = m.rope(port, apos)
    assert not torch.equal(expand_tables(pl[0])[0], expand_tables(pp[0])[0])
    for pos, pe in ((land, pl), (port, pp)):
        cos, sin = rope_tables_np(pos, m.video_dim, VIDEO_MAX_POS)
        assert len(pe[0]) == 3  # factored over (frame, row, column)
        c, s = expand_tables(pe[0])
        assert np.array_equal(c.numpy().view(np.uint32), cos.view(np.uint32))
        assert np.array_equal(s.numpy().view(np.uint32), sin.view(np.uint32))
    # a repeated call returns the cached objects
    assert m.rope(land, apos)[0][0] is pl[0][0]


def test_cache_is_bounded_and_evicts_least_recently_used():
    m = _stub_model()
    grids = [video_positions(2, h, 3, 24.0) for h in (1, 2, 3, 4)]
    first = m.rope(grids[0], None)
    for g in grids[1:]:
        m.rope(g, None)
    assert len(m._rope_cache) == model_mod.ROPE_CACHE_ENTRIES
    # grids[0] was evicted: a new call rebuilds equal but distinct tables
    again = m.rope(grids[0], None)
    assert again[0][0] is not first[0][0] and torch.equal(again[0][0], first[0][0])
