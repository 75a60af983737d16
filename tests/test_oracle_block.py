"""Pin the block oracle's residual wiring with invariants on a tiny model."""

import torch

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
