"""GPU tests of the Modality-level forward (``LTXModel.__call__``,
model/transformer/model.py:1344-1486) and ``X0Model`` (:1489-1542).

A 2-block full-width AV model on a small grid (48 video tokens, 12 audio
tokens, 16 text tokens):

* B = 2 samples (own latents and contexts, one timestep) as one stacked
  forward: each sample's velocity equals its own B = 1 forward to fp32
  summation order (the stacked rows change the GEMM tiling), and sample 1
  matches the oracle's ``model_velocity``;
* (B, S) context masks: a boolean padding mask and an additive 0 / -inf mask
  with holes give the same bits as the forward on the kept context rows
  (a dropped key's softmax weight is exactly 0), alone and for samples with
  different kept lengths (then run one after another);
* X0Model: ``latent - sigma * velocity`` in fp32, bit for bit, with and
  without the audio modality; the audio velocity of a video-only call is an
  empty (B, 0, 128) tensor;
* per-token video timesteps (an image-conditioned denoise mask: conditioned
  tokens at 0) run as row groups and match the oracle's per-token forward
  (cosine >= 0.999, normwise error <= 2e-2), in two and three row segments;
  one value on every token is the uniform forward bit for bit;
* the conditioned distilled loop (``condition_video`` + ``denoise_conditioned``)
  follows the oracle's loop per step and keeps the conditioned rows clean.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import bf16_from_torch, cos_sim, max_rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(seed=11):
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.pipeline import DenoiseState

    model = LTXModel(num_layers=2, weight_format="mxfp8", seed=seed)
    states = [DenoiseState(model, height=128, width=192, frames=9, text_tokens=16, audio_frames=12, seed=s)
              for s in (5, 6)]
    return model, states


def _mod(st, latent=None, context=None, mask=None, audio=False, sigma=0.6):
    from ltx_amd.model.transformer.model import Modality

    if audio:
        return Modality(latent=st.audio_latent[None] if latent is None else latent,
                        context=st.audio_context[None] if context is None else context, context_mask=mask,
                        timesteps=torch.full((1,), sigma), positions=st.audio_positions)
    return Modality(latent=st.video_latent[None] if latent is None else latent,
                    context=st.video_context[None] if context is None else context, context_mask=mask,
                    timesteps=torch.full((1,), sigma), positions=st.video_positions)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu()


def test_two_samples_stacked_match_single_sample_forwards_and_oracle():
    from test_gpu_model import _model_weights

    from oracle import block as ob
    from oracle import rope as orope

    model, (s0, s1) = _setup()
    print("modality: B=2 stacked vs B=1 forwards", flush=True)
    v = torch.stack([s0.video_latent, s1.video_latent])
    a = torch.stack([s0.audio_latent, s1.audio_latent])
    vc = torch.stack([s0.video_context, s1.video_context])
    ac = torch.stack([s0.audio_context, s1.audio_context])
    vv, av = model(_mod(s0, v, vc), _mod(s0, a, ac, audio=True))
    torch.cuda.synchronize()
    assert vv.shape == (2, s0.video_tokens, 128) and av.shape == (2, s0.audio_tokens, 128)
    for i, st in enumerate((s0, s1)):
        v1, a1 = model(_mod(st), _mod(st, audio=True))
        torch.cuda.synchronize()
        for got, ref in ((vv[i], v1[0]), (av[i], a1[0])):
            g, r = bf16_from_torch(got), bf16_from_torch(ref)
            assert max_rel_err(g, r) <= 1e-2 and cos_sim(g, r) >= 0.9999
    MW = _model_weights(model)
    vpos, apos = s0.video_positions, s0.audio_positions
    pes = tuple(tuple(torch.from_numpy(x) for x in p) for p in (
        orope.rope_tables(vpos, 4096, 32, orope.VIDEO_MAX_POS),
        orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS)))
    ov, oa = ob.model_velocity(MW, s1.video_latent.float().cpu(), s1.audio_latent.float().cpu(),
                               s1.video_context.float().cpu(), s1.audio_context.float().cpu(),
                               float(np.float32(0.6)), pes)
    assert cos_sim(bf16_from_torch(vv[1]), ov.numpy()) >= 0.999
    assert cos_sim(bf16_from_torch(av[1]), oa.numpy()) >= 0.999


def test_context_masks_equal_the_kept_rows():
    model, (s0, s1) = _setup()
    n = s0.video_context.shape[0]
    print("modality: boolean padding mask and additive mask with holes", flush=True)
    # boolean padding mask on the video context: the last 4 tokens are padding
    pad = torch.ones((1, n), dtype=torch.bool)
    pad[0, n - 4:] = False
    got, _ = model(_mod(s0, mask=pad))
    ref, _ = model(_mod(s0, context=s0.video_context[None, : n - 4]))
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(ref))
    # additive mask with holes on both contexts
    keep = np.array([0, 2, 3, 5, 8, 9, 10, 13, 15])
    add = torch.full((1, n), float("-inf"))
    add[0, keep] = 0.0
    kv = torch.from_numpy(keep).to(DEV)
    gv, ga = model(_mod(s0, mask=add), _mod(s0, mask=add.clone(), audio=True))
    rv, ra = model(_mod(s0, context=s0.video_context.index_select(0, kv)[None]),
                   _mod(s0, context=s0.audio_context.index_select(0, kv)[None], audio=True))
    torch.cuda.synchronize()
    assert torch.equal(_bits(gv), _bits(rv)) and torch.equal(_bits(ga), _bits(ra))
    # the mask changes the result (the dropped keys mattered)
    full, _ = model(_mod(s0))
    torch.cuda.synchronize()
    assert not torch.equal(_bits(full), _bits(gv))


def test_samples_with_unequal_kept_contexts_run_one_after_another():
    model, (s0, s1) = _setup()
    n = s0.video_context.shape[0]
    print("modality: B=2 with kept lengths 16 and 11", flush=True)
    mask = torch.ones((2, n), dtype=torch.bool)
    mask[1, 11:] = False
    v = torch.stack([s0.video_latent, s1.video_latent])
    vc = torch.stack([s0.video_context, s1.video_context])
    got, aud = model(_mod(s0, v, vc, mask=mask))
    r0, _ = model(_mod(s0))
    r1, _ = model(_mod(s1, context=s1.video_context[None, :11]))
    torch.cuda.synchronize()
    assert aud.shape == (2, 0, 128)
    assert torch.equal(_bits(got[0]), _bits(r0[0])) and torch.equal(_bits(got[1]), _bits(r1[0]))


def test_x0_model_is_latent_minus_sigma_velocity():
    from ltx_amd.model.transformer.model import X0Model

    model, (s0, _) = _setup()
    print("modality: X0Model", flush=True)
    sigma = float(np.float32(0.6))
    dv, da = X0Model(model)(_mod(s0), _mod(s0, audio=True))
    vv, av = model(_mod(s0), _mod(s0, audio=True))
    torch.cuda.synchronize()
    for d, lat, vel in ((dv, s0.video_latent, vv[0]), (da, s0.audio_latent, av[0])):
        ref = lat.float() - torch.tensor(sigma, device=DEV) * vel.float()
        assert d.dtype == torch.float32 and torch.equal(d[0], ref)
    # video-only inference on the AV model (no A2V / V2A): the video alone
    only = X0Model(model)(_mod(s0))
    vo, ao = model(_mod(s0))
    torch.cuda.synchronize()
    assert ao.shape == (1, 0, 128)
    assert torch.equal(only[0], s0.video_latent.float() - torch.tensor(sigma, device=DEV) * vo[0].float())


def _oracle_pes(st):
    from oracle import rope as orope

    vpos, apos = st.video_positions, st.audio_positions
    return tuple(tuple(torch.from_numpy(x) for x in p) for p in (
        orope.rope_tables(vpos, 4096, 32, orope.VIDEO_MAX_POS),
        orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS)))


@pytest.mark.parametrize("pattern", ["first_frame", "middle_run"])
def test_per_token_video_timesteps_match_the_oracle(pattern):
    """Image-conditioned denoise mask: the conditioned video tokens at t = 0,
    the rest at the sample sigma 0.6 (given as ``sigma``): the block's AdaLN
    inputs, gated residual adds and the output head run per row group (two
    or three segments) and match the oracle's per-token forward."""
    from test_gpu_model import _model_weights

    from ltx_amd.model.transformer.model import Modality, X0Model
    from oracle import block as ob

    model, (s0, _) = _setup()
    t = s0.video_tokens
    tok = torch.full((1, t), float(np.float32(0.6)))
    if pattern == "first_frame":
        tok[0, : t // 2] = 0.0          # latent frame 0 of 2
    else:
        tok[0, 8:16] = 0.0              # a run inside the first frame: three segments
    print(f"modality: per-token timesteps ({pattern})", flush=True)
    vmod = Modality(latent=s0.video_latent[None], context=s0.video_context[None], context_mask=None, timesteps=tok,
                    positions=s0.video_positions, sigma=torch.full((1,), 0.6))
    v, a = model(vmod, _mod(s0, audio=True))
    uv, _ = model(_mod(s0), _mod(s0, audio=True))
    torch.cuda.synchronize()
    assert not torch.equal(_bits(v), _bits(uv))
    ov, oa = ob.model_velocity(_model_weights(model), s0.video_latent.float().cpu(), s0.audio_latent.float().cpu(),
                               s0.video_context.float().cpu(), s0.audio_context.float().cpu(),
                               float(np.float32(0.6)), _oracle_pes(s0), video_token_sigmas=tok[0])
    gv, ga = bf16_from_torch(v[0]), bf16_from_torch(a[0])
    assert cos_sim(gv, ov.numpy()) >= 0.999 and cos_sim(ga, oa.numpy()) >= 0.999
    assert max_rel_err(gv, ov.numpy()) <= 2e-2
    # X0: latent - t_token * velocity per token
    dv, _ = X0Model(model)(vmod, _mod(s0, audio=True))
    torch.cuda.synchronize()
    ref = s0.video_latent.float() - tok[0].to(DEV)[:, None] * v[0].float()
    assert torch.equal(dv[0], ref)


def test_per_token_timesteps_all_equal_are_the_uniform_forward():
    from ltx_amd.model.transformer.model import Modality

    model, (s0, _) = _setup()
    print("modality: per-token timesteps, one value", flush=True)
    vmod = Modality(latent=s0.video_latent[None], context=s0.video_context[None], context_mask=None,
                    timesteps=torch.full((1, s0.video_tokens), 0.6), positions=s0.video_positions)
    v, a = model(vmod, _mod(s0, audio=True))
    uv, ua = model(_mod(s0), _mod(s0, audio=True))
    torch.cuda.synchronize()
    assert torch.equal(_bits(v), _bits(uv)) and torch.equal(_bits(a), _bits(ua))


def test_conditioned_loop_matches_the_oracle_and_keeps_the_clean_rows():
    """``condition_video`` + ``denoise_conditioned``: the first latent frame
    held clean (mask 0), eight distilled steps; per step the latents match the
    oracle's loop (per-token timesteps sigma * mask, X0 per token, clean rows
    blended in, Euler) at cosine >= 0.999, and the conditioned rows stay the
    clean rows bit for bit."""
    from test_gpu_model import _model_weights

    from ltx_amd.pipeline import condition_video, denoise_conditioned
    from oracle import block as ob

    model, (s0, _) = _setup()
    t = s0.video_tokens
    mask = torch.ones(t)
    mask[: t // 2] = 0.0
    g = torch.Generator().manual_seed(3)
    clean = torch.randn((t, 128), generator=g).to(torch.bfloat16)
    condition_video(s0, mask, clean)
    print("modality: conditioned 8-step loop vs oracle", flush=True)
    MW = _model_weights(model)
    pes = _oracle_pes(s0)
    vlat, alat = s0.video_latent.float().cpu(), s0.audio_latent.float().cpu()
    vctx, actx = s0.video_context.float().cpu(), s0.audio_context.float().cpu()
    got = []
    denoise_conditioned(model, s0, callback=lambda step, st: got.append(
        (st.video_latent.float().cpu().clone(), st.audio_latent.float().cpu().clone())))
    cleanf = clean.float()
    keep = mask == 0
    for step in range(len(s0.sigmas) - 1):
        sigma, sigma_next = s0.sigmas[step], s0.sigmas[step + 1]
        tok = mask * torch.tensor(sigma, dtype=torch.float32)
        vv, av = ob.model_velocity(MW, vlat, alat, vctx, actx, sigma, pes, video_token_sigmas=tok)
        x0 = vlat - tok[:, None] * vv
        x0[keep] = cleanf[keep]
        ratio = torch.tensor(sigma_next / sigma, dtype=torch.float32)
        vlat = ob.bf(x0 + ratio * (vlat - x0))
        alat = ob.euler_x0(alat, av, sigma, sigma_next)
        cv, ca = cos_sim(got[step][0].numpy(), vlat.numpy()), cos_sim(got[step][1].numpy(), alat.numpy())
        print(f"conditioned step {step}: video cos {cv:.6f} audio cos {ca:.6f}", flush=True)
        assert cv >= 0.999 and ca >= 0.999
        assert torch.equal(got[step][0][keep], cleanf[keep])
