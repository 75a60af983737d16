"""Pin the block oracle's residual wiring with invariants on a tiny model."""

import pytest
import torch

from _util import cos_sim, max_rel_err
from oracle import block as ob


def _attn(qd, kd, heads, dh, g):
    inner = heads * dh
    rnd = lambda *s: ob.bf(torch.randn(s, generator=g) * 0.1)  # noqa: E731
    return {"to_q": rnd(inner, qd), "to_q_b": torch.zeros(inner), "to_k": rnd(inner, kd), "to_k_b": torch.zeros(inner),
            "to_v": rnd(inner, kd), "to_v_b": torch.zeros(inner), "to_gate_logits": rnd(heads, qd),
            "to_gate_logits_b": torch.zeros(heads), "to_out": rnd(qd, inner), "to_out_b": torch.zeros(qd),
            "q_norm": torch.ones(inner), "k_norm": torch.ones(inner)}


def _setup(seed=0, tv=6, ta=4, s=3, vd=64, ad=32, heads=4):
    g = torch.Generator().manual_seed(seed)
    W = {"attn1": _attn(vd, vd, heads, vd // heads, g), "attn2": _attn(vd, vd, heads, vd // heads, g),
         "audio_attn1": _attn(ad, ad, heads, ad // heads, g), "audio_attn2": _attn(ad, ad, heads, ad // heads, g),
         "audio_to_video_attn": _attn(vd, ad, heads, ad // heads, g),
         "video_to_audio_attn": _attn(ad, vd, heads, ad // heads, g),
         "ff": {"w1": ob.bf(torch.randn(4 * vd, vd, generator=g) * 0.1), "b1": torch.zeros(4 * vd),
                "w2": ob.bf(torch.randn(vd, 4 * vd, generator=g) * 0.1), "b2": torch.zeros(vd)},
         "audio_ff": {"w1": ob.bf(torch.randn(4 * ad, ad, generator=g) * 0.1), "b1": torch.zeros(4 * ad),
                      "w2": ob.bf(torch.randn(ad, 4 * ad, generator=g) * 0.1), "b2": torch.zeros(ad)}}
    vx, ax = ob.bf(torch.randn(tv, vd, generator=g)), ob.bf(torch.randn(ta, ad, generator=g))
    vctx, actx = ob.bf(torch.randn(s, vd, generator=g)), ob.bf(torch.randn(s, ad, generator=g))
    vada, aada = torch.randn(16, vd, generator=g) * 0.1, torch.randn(16, ad, generator=g) * 0.1
    return W, vx, ax, vctx, actx, vada, aada


def _run(W, vx, ax, vctx, actx, vada, aada):
    # RoPE off in the wiring tests (pe=None everywhere); heads fixed to 32 in
    # the oracle, so use 32-head-compatible dims via a wrapper
    return ob.block(W, vx, ax, vada, aada, vctx, actx, None, None, None, None)


GATES = (2, 5, 8, 15)


def test_zero_gates_make_the_block_the_identity(monkeypatch):
    W, vx, ax, vctx, actx, vada, aada = _setup()
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    for r in GATES:
        vada[r] = 0.0
        aada[r] = 0.0
    vo, ao = _run(W, vx, ax, vctx, actx, vada, aada)
    assert torch.equal(vo, vx) and torch.equal(ao, ax)


def test_each_gate_drives_its_sub_layer(monkeypatch):
    W, vx, ax, vctx, actx, vada, aada = _setup(1)
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    for r in GATES:
        vada[r] = 0.0
        aada[r] = 0.0
    for r in GATES:
        v2 = vada.clone()
        v2[r] = 1.0
        vo, ao = _run(W, vx, ax, vctx, actx, v2, aada)
        assert not torch.equal(vo, vx), r
        assert torch.equal(ao, ax), r  # a video gate never changes audio


def test_zero_a2v_gate_decouples_video_from_audio(monkeypatch):
    W, vx, ax, vctx, actx, vada, aada = _setup(2)
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    vada[15] = 0.0
    v1, _ = _run(W, vx, ax, vctx, actx, vada, aada)
    v2, a2 = _run(W, vx, ob.bf(ax * 3.0 + 1.0), vctx, actx, vada, aada)
    assert torch.equal(v1, v2)
    assert not torch.equal(a2, ax)


def test_ff_path_is_per_token(monkeypatch):
    W, vx, ax, vctx, actx, vada, aada = _setup(3)
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    for r in (2, 8, 15):   # only the FF sub-layer stays active on video
        vada[r] = 0.0
    perm = torch.tensor([3, 0, 5, 1, 4, 2])
    v1, _ = _run(W, vx, None, vctx, None, vada, None)
    v2, _ = _run(W, vx[perm], None, vctx, None, vada, None)
    assert torch.equal(v1[perm], v2)


def _small_heads(fn):
    def wrapped(w, x, context=None, pe=None, k_pe=None, heads=32, eps=ob.EPS):
        return fn(w, x, context, pe, k_pe, heads=4, eps=eps)
    return wrapped


# ---- modulation-row pins ----------------------------------------------------
# With scale row = -1 and shift row = c, the modulated input of a sub-layer is
# bf(norm * 0 + c) = bf(c) for every token, whatever the stream holds; the
# sub-layer's output is then one row u shared by all tokens, and with gate 1
# the stream becomes bf(x + u).  Running once on a zero stream gives u itself
# (each output row equals u), so the check needs no restatement of the
# sub-layer: out(x) == bf(x + out(0)).  A wiring that reads any other row as
# the scale leaves the input dependent on x and fails.  When the pinned input
# is the keys/values side (identical keys and values: every query averages
# the same value row), the per-head output gate 2*sigmoid(x Wg) still varies
# with the query, so that module's gate logits are zeroed (gate 1).
#
# (table, gate row, scale row, shift row, stream updated, streams zeroed in the
#  baseline run, module whose head gate is neutralised) -- rows of the (16, D) layout [sst(9) | prompt(2) | av(5)]:
#  sst 0 shift_msa 1 scale_msa 2 gate_msa 3 shift_mlp 4 scale_mlp 5 gate_mlp
#  6 shift_q 7 scale_q 8 gate_q (transformer.py:450-452, :632-634, :360-362),
#  prompt 9 shift_kv 10 scale_kv (:363-369), av 11 scale_a2v 12 shift_a2v
#  13 scale_v2a 14 shift_v2a 15 gate (scale before shift, :311-342, :539-564).
ROW_CASES = [
    ("v", 2, 1, 0, "v", "v", None),                         # video self-attention input
    ("v", 8, 7, 6, "v", "v", None),                         # video text cross-attention query
    ("v", 8, 10, 9, "v", "v", "attn2"),                     # video text cross-attention context
    ("v", 5, 4, 3, "v", "v", None),                         # video FF input
    ("a", 2, 1, 0, "a", "a", None),                         # audio self-attention input
    ("a", 8, 7, 6, "a", "a", None),                         # audio text cross-attention query
    ("a", 8, 10, 9, "a", "a", "audio_attn2"),               # audio text cross-attention context
    ("a", 5, 4, 3, "a", "a", None),                         # audio FF input
    ("v", 15, 11, 12, "v", "v", None),                      # A2V: video queries
    ("a", 15, 11, 12, "v", "va", "audio_to_video_attn"),    # A2V: audio keys/values
    ("a", 15, 13, 14, "a", "a", None),                      # V2A: audio queries
    ("v", 15, 13, 14, "a", "va", "video_to_audio_attn"),    # V2A: video keys/values
]


def _isolate(vada, aada, table, gate):
    """Zero every gate but ``gate`` of ``table``'s sub-layer (set to 1)."""
    for r in GATES:
        vada[r] = 0.0
        aada[r] = 0.0
    # the AV gate row sits in the table of the stream it updates
    (vada if table == "v" else aada)[gate] = 1.0


def _row_case(seed, table, gate, scale, shift, updated, zeroed, ungated, swap=False):
    W, vx, ax, vctx, actx, vada, aada = _setup(seed)
    if ungated is not None:
        W[ungated] = dict(W[ungated], to_gate_logits=torch.zeros_like(W[ungated]["to_gate_logits"]))
    _isolate(vada, aada, updated, gate)
    mod = vada if table == "v" else aada
    c = ob.bf(torch.randn(mod.shape[1], generator=torch.Generator().manual_seed(seed + 100)))
    s_row, h_row = (shift, scale) if swap else (scale, shift)
    mod[s_row] = -1.0
    mod[h_row] = c
    v0 = torch.zeros_like(vx) if "v" in zeroed else vx
    a0 = torch.zeros_like(ax) if "a" in zeroed else ax
    out0 = _run(W, v0, a0, vctx, actx, vada, aada)
    out = _run(W, vx, ax, vctx, actx, vada, aada)
    i = 0 if updated == "v" else 1
    x = (vx, ax)[i]
    u = out0[i]
    uniform = bool((u == u[0:1]).all())
    return uniform and torch.equal(out[i], ob.bf(x + u[0:1]))


@pytest.mark.parametrize("case", ROW_CASES, ids=lambda c: f"{c[0]}{c[2]}-{c[3]}->{c[4]}")
def test_modulation_rows_feed_the_right_sub_layer_input(monkeypatch, case):
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    assert _row_case(11, *case)
    # the same check with scale and shift rows exchanged fails: it can tell the
    # reference's row order from its mirror image
    assert not _row_case(11, *case, swap=True)


def test_v2a_reads_the_norm_taken_before_a2v(monkeypatch):
    """V2A's video keys come from rms_norm(vx) computed before A2V updates vx
    (transformer.py:535-536, used at :613): the A2V projections cannot reach
    the audio output of the block."""
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    W, vx, ax, vctx, actx, vada, aada = _setup(12)
    vada[15], aada[15] = 1.5, 1.5  # A2V and V2A both active, everything else too
    v1, a1 = _run(W, vx, ax, vctx, actx, vada, aada)
    g = torch.Generator().manual_seed(99)
    W2 = dict(W)
    W2["audio_to_video_attn"] = {k: (ob.bf(t + torch.randn(t.shape, generator=g) * 0.3) if t.dim() == 2 else t)
                                 for k, t in W["audio_to_video_attn"].items()}
    v2, a2 = _run(W2, vx, ax, vctx, actx, vada, aada)
    assert not torch.equal(v1, v2)  # the change does reach video
    assert torch.equal(a1, a2)


def _rot90_rows(w: torch.Tensor, heads: int) -> torch.Tensor:
    """Rows of a projection whose output is the split-RoPE rotation by 90
    degrees of the original's: per head [x1, x2] -> [-x2, x1]."""
    n, k = w.shape
    wh = w.view(heads, 2, n // heads // 2, k)
    return torch.cat([-wh[:, 1:2], wh[:, 0:1]], 1).reshape(n, k)


def _cross_pe_block(W, vx, ax, vctx, actx, vada, aada, vx_rot, ax_rot):
    t_v, t_a, half = vx.shape[0], ax.shape[0], ax.shape[1] // 2

    def table(t, rot):  # (cos, sin): 90 degrees or identity on every token
        return (torch.zeros(t, half), torch.ones(t, half)) if rot else (torch.ones(t, half), torch.zeros(t, half))

    return ob.block(W, vx, ax, vada, aada, vctx, actx, None, table(t_v, vx_rot), None, table(t_a, ax_rot))


@pytest.mark.parametrize("rotated", ["video", "audio"])
def test_cross_pe_tables_rotate_their_own_side_in_each_direction(monkeypatch, rotated):
    """Cross-modal RoPE (transformer.py:584-589, :617-623): in A2V the video
    cross table rotates the queries and the audio table the keys; in V2A the
    audio table rotates the queries and the video table the keys.  A table of
    90-degree rotations equals rotating the projection rows that produce the
    rotated side, so the block with one side's table at 90 degrees must match
    the block with identity tables and those rows rotated: A2V to_q and V2A
    to_k for the video table, A2V to_k and V2A to_q for the audio table.
    Video and audio have the same token count here, so a wiring that swaps
    the tables within a direction runs and is caught."""
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    W, vx, ax, vctx, actx, vada, aada = _setup(13, tv=4, ta=4)
    vada[15], aada[15] = 1.0, 1.0
    for r in (2, 5, 8):  # only the AV cross-attentions act
        vada[r] = aada[r] = 0.0
    heads = 4
    got = _cross_pe_block(W, vx, ax, vctx, actx, vada, aada, rotated == "video", rotated == "audio")

    def rotate(Wm, a2v_name, v2a_name):
        W2 = dict(Wm)
        W2["audio_to_video_attn"] = dict(Wm["audio_to_video_attn"])
        W2["video_to_audio_attn"] = dict(Wm["video_to_audio_attn"])
        W2["audio_to_video_attn"][a2v_name] = _rot90_rows(Wm["audio_to_video_attn"][a2v_name], heads)
        W2["video_to_audio_attn"][v2a_name] = _rot90_rows(Wm["video_to_audio_attn"][v2a_name], heads)
        return W2

    right = ("to_q", "to_k") if rotated == "video" else ("to_k", "to_q")
    want = _cross_pe_block(rotate(W, *right), vx, ax, vctx, actx, vada, aada, False, False)
    wrong = _cross_pe_block(rotate(W, *right[::-1]), vx, ax, vctx, actx, vada, aada, False, False)
    for g, w, x in zip(got, want, wrong):
        assert cos_sim(g, w) >= 0.99999 and max_rel_err(g, w) <= 1e-2
        assert max_rel_err(g, x) > 5e-2  # the other assignment is far away


def test_text_cross_attention_rounds_twice_self_attention_once(monkeypatch):
    """The text cross-attention output is rounded after the gate and again
    after the residual add, bf(x + bf(o * gate)) (transformer.py:387, :484);
    the self-attention residual rounds once, bf(x + o * gate)
    (transformer.py:46-50, :469).  With the sub-layer input pinned to a
    constant (scale -1 / shift c), o is the zero-stream output at gate 1."""
    monkeypatch.setattr(ob, "attention", _small_heads(ob.attention))
    for gate_row, scale, shift, double in ((8, 7, 6, True), (2, 1, 0, False)):
        W, vx, ax, vctx, actx, vada, aada = _setup(14, tv=64)
        _isolate(vada, aada, "v", gate_row)
        vada[scale], vada[shift] = -1.0, ob.bf(torch.full((vada.shape[1],), 0.7))
        o = _run(W, torch.zeros_like(vx), ax, vctx, actx, vada, aada)[0][0:1]
        vx = ob.bf(vx * 4.0)  # residual magnitudes where the two forms part
        gate = torch.full((vada.shape[1],), 0.3071)
        vada[gate_row] = gate
        out = _run(W, vx, ax, vctx, actx, vada, aada)[0]
        twice, once = ob.bf(vx + ob.bf(o * gate)), ob.bf(vx + o * gate)
        assert not torch.equal(twice, once)  # the two forms differ on these inputs
        assert torch.equal(out, twice if double else once)


def _mlp(d_out, g, zero_embedding=True):
    w = {"w1": ob.bf(torch.randn(16, 256, generator=g) * 0.1), "b1": torch.zeros(16),
         "w2": torch.zeros(8, 16), "b2": torch.zeros(8),
         "w": ob.bf(torch.randn(d_out, 8, generator=g) * 0.1), "b": ob.bf(torch.randn(d_out, generator=g) * 0.1)}
    if not zero_embedding:
        w["w2"] = ob.bf(torch.randn(8, 16, generator=g) * 0.1)
    return w


@pytest.mark.parametrize("swap", [False, True])
def test_output_head_reads_shift_row_0_and_scale_row_1(swap):
    """Output head (model.py:1312-1326): ``shift, scale = sst_out + emb``
    rows 0 and 1.  With the embedded timestep zero (its second MLP layer
    zeroed), scale row -1 and shift row c give ``proj_out(c)`` on every token
    whatever the latent; the mirrored assignment does not."""
    g = torch.Generator().manual_seed(21)
    vd, ad = 8, 8
    lin = lambda n, k: (ob.bf(torch.randn(n, k, generator=g) * 0.1), ob.bf(torch.randn(n, generator=g) * 0.1))  # noqa: E731
    c = ob.bf(torch.randn(vd, generator=g))
    table = torch.stack([c, -torch.ones(vd)]) if not swap else torch.stack([-torch.ones(vd), c])
    MW = {"patchify": lin(vd, 128), "audio_patchify": lin(ad, 128),
          "mlps_v": [_mlp(9 * vd, g), _mlp(2 * vd, g), _mlp(4 * vd, g), _mlp(vd, g)],
          "mlps_a": [_mlp(9 * ad, g), _mlp(2 * ad, g), _mlp(4 * ad, g), _mlp(ad, g)],
          "tables_v": None, "tables_a": None, "blocks": [],
          "sst_out_v": table, "proj_out_v": lin(128, vd), "sst_out_a": table, "proj_out_a": lin(128, ad)}
    lat = ob.bf(torch.randn(5, 128, generator=g))
    vv, av = ob.model_velocity(MW, lat, lat[:3], None, None, 0.5, (None,) * 4)
    want_v, want_a = (ob.linear(c[None, :], *MW[k]) for k in ("proj_out_v", "proj_out_a"))
    hit = torch.equal(vv, want_v.expand_as(vv)) and torch.equal(av, want_a.expand_as(av))
    assert hit != swap
