"""Guided loops on the GPU: the guidance kernels against the oracle (bit-exact
for the elementwise forms, tolerance for the two global reductions), and the
CFG/STG (av_pipeline.py:625-757) and multi-modal (two_stage.py:306-388)
loops of a 2-block full-width model against the oracle's passes, guidance
and Euler steps."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import cos_sim
from _weights import block_weights, mlp_weights
from oracle import block as ob
from oracle import guidance as og
from oracle import rope as orope
from oracle.bf16 import bf16r

pytestmark = pytest.mark.gpu
DEV = "cuda"
SIZES = [1, 7, 8, 9, 4096 + 5, 3456 * 128]


def _f32(rng, n):
    return rng.standard_normal(n).astype(np.float32)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("n", SIZES)
def test_x0_and_euler_bit_exact(n):
    from ltx_amd.components.diffusion_steps import EulerDiffusionStep, to_denoised

    print(f"x0/euler n={n}", flush=True)
    rng = np.random.default_rng(n)
    x, v = bf16r(_f32(rng, n)), bf16r(_f32(rng, n))
    xd, vd = _dev(x).bfloat16(), _dev(v).bfloat16()
    d = to_denoised(xd, vd, 0.909375)
    np.testing.assert_array_equal(d.cpu().numpy(), og.x0(x, v, np.float32(0.909375)))
    out = EulerDiffusionStep().step(xd, d, None, 0, sigma=float(np.float32(0.909375)),
                                    sigma_next=float(np.float32(0.725)))
    ref = og.euler(x, d.cpu().numpy(), float(np.float32(0.909375)), float(np.float32(0.725)))
    np.testing.assert_array_equal(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("n", SIZES)
def test_guidance_forms_bit_exact(n):
    from ltx_amd.components import guiders as G

    print(f"guidance forms n={n}", flush=True)
    rng = np.random.default_rng(n + 1)
    c, u, p, m = (_f32(rng, n) for _ in range(4))
    C, U, P, M = (_dev(a) for a in (c, u, p, m))
    for scale in (3.0, 7.0, 1.0):
        g = G.CFGGuider(scale)
        np.testing.assert_array_equal(g.guide(C, U).cpu().numpy(), og.guide(c, (u,), (scale - 1,)))
        np.testing.assert_array_equal(g.delta(C, U).cpu().numpy(), og.guide(c, (u,), (scale - 1,), delta_only=True))
    s = G.STGGuider(1.5)
    np.testing.assert_array_equal(s.guide(C, P).cpu().numpy(), og.guide(c, (p,), (1.5,)))
    mm = G.MultiModalGuider(G.MultiModalGuiderParams(cfg_scale=3.0, stg_scale=0.5, modality_scale=3.0))
    np.testing.assert_array_equal(mm.calculate(C, U, P, M).cpu().numpy(),
                                  og.guide(c, (u, p, m), (2.0, 0.5, 2.0)))
    np.testing.assert_array_equal(mm.calculate(C, U, 0.0, M).cpu().numpy(),
                                  og.guide(c, (u, None, m), (2.0, 0.0, 2.0)))


@pytest.mark.parametrize("n", [9, 4096 + 5, 3456 * 128])
def test_guidance_reductions(n):
    """CFG-star projection coefficient and the std rescale: the statistic to
    1e-6 relative, the guided latent then bit-exact given the kernel's own
    statistic and within one fp32 ulp-scale difference of the oracle's."""
    from ltx_amd.components import guiders as G

    print(f"guidance reductions n={n}", flush=True)
    rng = np.random.default_rng(n + 2)
    c, u = _f32(rng, n), (0.8 * _f32(rng, n) + 0.3).astype(np.float32)
    C, U = _dev(c), _dev(u)
    coef = G.projection_coef(C, U)
    ref_coef = og.projection_coef(c, u)
    assert abs(float(coef) - float(ref_coef)) <= 1e-6 * abs(float(ref_coef))
    star = G.CFGStarRescalingGuider(3.0)
    got = star.guide(C, U).cpu().numpy()
    np.testing.assert_array_equal(got, og.guide(c, (u,), (2.0,), coef=float(coef)))
    mm = G.MultiModalGuider(G.MultiModalGuiderParams(cfg_scale=3.0, rescale_scale=0.7))
    pred = og.guide(c, (u,), (2.0,))
    fac = og.std_ratio(c, pred, 0.7)
    got = mm.calculate(C, U, 0.0, 0.0).cpu().numpy()
    ref = og.guide(pred, (), (), factor=fac)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6)


def test_ge_correct_bit_exact():
    from ltx_amd import _lib

    rng = np.random.default_rng(4)
    n = 3456 * 128 + 3
    x, d = bf16r(_f32(rng, n)), _f32(rng, n)
    X, D = _dev(x).bfloat16(), _dev(d)
    prev = torch.empty_like(D)
    _lib.call("ltx_ge_correct_f32", X.data_ptr(), D.data_ptr(), prev.data_ptr(), 0, 0.725, 0.5, n,
              _lib.stream_of(D))
    d1, cur = og.ge_correct(x, d, None, False, 0.725, 0.5)
    np.testing.assert_array_equal(D.cpu().numpy(), d1)
    np.testing.assert_array_equal(prev.cpu().numpy(), cur)
    d_next = _f32(rng, n)
    D2 = _dev(d_next)
    _lib.call("ltx_ge_correct_f32", X.data_ptr(), D2.data_ptr(), prev.data_ptr(), 1, 0.421875, 0.5, n,
              _lib.stream_of(D2))
    d2, cur2 = og.ge_correct(x, d_next, cur, True, 0.421875, 0.5)
    np.testing.assert_array_equal(D2.cpu().numpy(), d2)
    np.testing.assert_array_equal(prev.cpu().numpy(), cur2)


# -- loops ------------------------------------------------------------------------
def _model_weights(m):
    from ltx_amd.kernels import gemm

    def lw(w):
        return gemm.dequantize(w).float().cpu(), w.bias.float().cpu()

    return {
        "patchify": lw(m.patchify_proj), "audio_patchify": lw(m.audio_patchify_proj),
        "mlps_v": [mlp_weights(x) for x in (m.adaln_single, m.prompt_adaln_single,
                                            m.av_ca_video_scale_shift_adaln_single, m.av_ca_a2v_gate_adaln_single)],
        "mlps_a": [mlp_weights(x) for x in (m.audio_adaln_single, m.audio_prompt_adaln_single,
                                            m.av_ca_audio_scale_shift_adaln_single, m.av_ca_v2a_gate_adaln_single)],
        "tables_v": m.video_tables.float().cpu(), "tables_a": m.audio_tables.float().cpu(),
        "blocks": [block_weights(b) for b in m.transformer_blocks],
        "sst_out_v": m.scale_shift_table.float().cpu(), "proj_out_v": lw(m.proj_out),
        "sst_out_a": m.audio_scale_shift_table.float().cpu(), "proj_out_a": lw(m.audio_proj_out),
    }


def _setup(steps):
    from ltx_amd.components.schedulers import LTX2Scheduler
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.pipeline import DenoiseState

    model = LTXModel(num_layers=2, weight_format="bf16", seed=21)
    sig = LTX2Scheduler().execute(steps=steps)
    state = DenoiseState(model, height=128, width=192, frames=9, text_tokens=16, audio_frames=12, seed=8,
                         sigmas=sig)
    vpos, apos = state.video_positions, state.audio_positions
    pes = tuple(tuple(torch.from_numpy(a) for a in p) for p in (
        orope.rope_tables(vpos, 4096, 32, orope.VIDEO_MAX_POS),
        orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS)))
    cpu = {k: getattr(state, k).float().cpu() for k in ("video_latent", "audio_latent", "video_context",
                                                         "audio_context", "negative_video_context",
                                                         "negative_audio_context")}
    return model, state, pes, cpu


def test_cfg_stg_ge_loop_matches_oracle():
    """CFG-star (video 3, audio 7) + STG (scale 1, block 1, cutoff 0.75) + GE
    (gamma 0.5) over 4 shifted-schedule steps, every step's latents against
    the oracle fed the oracle's own previous latents."""
    from ltx_amd.components.guiders import CFGStarRescalingGuider, STGGuider
    from ltx_amd.components.perturbations import create_batched_stg_config
    from ltx_amd.pipeline import denoise_cfg_av

    print("cfg/stg/ge loop", flush=True)
    steps = 4
    model, state, pes, cpu = _setup(steps)
    MW = _model_weights(model)
    got = []
    denoise_cfg_av(model, state, video_guider=CFGStarRescalingGuider(3.0), audio_guider=CFGStarRescalingGuider(7.0),
                   stg_guider=STGGuider(1.0), stg_perturbations=create_batched_stg_config(1, blocks=[1]),
                   stg_cutoff=0.75, ge_gamma=0.5,
                   callback=lambda s, st: got.append((st.video_latent.float().cpu().clone(),
                                                      st.audio_latent.float().cpu().clone())))
    sig = state.sigmas
    vl, al = cpu["video_latent"], cpu["audio_latent"]
    prev = None
    for step in range(steps):
        s = sig[step]

        def den(ctx_v, ctx_a, skips=None):
            vv, av = ob.model_velocity(MW, vl, al, ctx_v, ctx_a, s, pes, skips=skips)
            return og.x0(vl.numpy(), vv.numpy(), s), og.x0(al.numpy(), av.numpy(), s)

        pv, pa = den(cpu["video_context"], cpu["audio_context"])
        nv, na = den(cpu["negative_video_context"], cpu["negative_audio_context"])
        vd = og.guide(pv, (nv,), (2.0,), coef=og.projection_coef(pv, nv))
        ad = og.guide(pa, (na,), (6.0,), coef=og.projection_coef(pa, na))
        if (step + 1) / steps <= 0.75:
            tv, _ = den(cpu["video_context"], cpu["audio_context"],
                        skips=lambda i: {"skip_video_self_attn"} if i == 1 else set())
            vd = og.guide(vd, (tv,), (1.0,))
        vd, cur = og.ge_correct(vl.numpy(), vd, prev, prev is not None, s, 0.5)
        prev = cur
        vl = torch.from_numpy(og.euler(vl.numpy(), vd, s, sig[step + 1]))
        al = torch.from_numpy(og.euler(al.numpy(), ad, s, sig[step + 1]))
        cv, ca = cos_sim(got[step][0].numpy(), vl.numpy()), cos_sim(got[step][1].numpy(), al.numpy())
        print(f"step {step}: video cos {cv:.6f} audio cos {ca:.6f}", flush=True)
        assert cv >= 0.999 and ca >= 0.999
        vl, al = got[step]  # continue from the product's latents (per-step comparison)


def test_multimodal_loop_matches_oracle():
    """MultiModalGuider: CFG 3 / audio 7, modality 3, rescale 0.7 (video) over
    3 steps; the modality-isolated pass skips A2V and V2A in every block."""
    from ltx_amd.components.guiders import MultiModalGuider, MultiModalGuiderParams
    from ltx_amd.pipeline import denoise_multimodal_av

    print("multimodal loop", flush=True)
    steps = 3
    model, state, pes, cpu = _setup(steps)
    MW = _model_weights(model)
    vg = MultiModalGuider(MultiModalGuiderParams(cfg_scale=3.0, modality_scale=3.0, rescale_scale=0.7))
    ag = MultiModalGuider(MultiModalGuiderParams(cfg_scale=7.0, modality_scale=3.0))
    got = []
    denoise_multimodal_av(model, state, video_guider=vg, audio_guider=ag,
                          callback=lambda s, st: got.append((st.video_latent.float().cpu().clone(),
                                                             st.audio_latent.float().cpu().clone())))
    sig = state.sigmas
    vl, al = cpu["video_latent"], cpu["audio_latent"]
    iso = lambda i: {"skip_a2v_cross_attn", "skip_v2a_cross_attn"}  # noqa: E731
    for step in range(steps):
        s = sig[step]

        def den(ctx_v, ctx_a, skips=None):
            vv, av = ob.model_velocity(MW, vl, al, ctx_v, ctx_a, s, pes, skips=skips)
            return og.x0(vl.numpy(), vv.numpy(), s), og.x0(al.numpy(), av.numpy(), s)

        cv_, ca_ = den(cpu["video_context"], cpu["audio_context"])
        uv, ua = den(cpu["negative_video_context"], cpu["negative_audio_context"])
        mv, ma = den(cpu["video_context"], cpu["audio_context"], skips=iso)
        pred = og.guide(cv_, (uv, None, mv), (2.0, 0.0, 2.0))
        vd = og.guide(pred, (), (), factor=og.std_ratio(cv_, pred, 0.7))
        ad = og.guide(ca_, (ua, None, ma), (6.0, 0.0, 2.0))
        vl = torch.from_numpy(og.euler(vl.numpy(), vd, s, sig[step + 1]))
        al = torch.from_numpy(og.euler(al.numpy(), ad, s, sig[step + 1]))
        cv, ca = cos_sim(got[step][0].numpy(), vl.numpy()), cos_sim(got[step][1].numpy(), al.numpy())
        print(f"step {step}: video cos {cv:.6f} audio cos {ca:.6f}", flush=True)
        assert cv >= 0.999 and ca >= 0.999
        vl, al = got[step]


@pytest.mark.parametrize("loop", ["cfg_stg", "multimodal"])
def test_batched_passes_match_sequential_passes(loop):
    """The passes of a guided step stacked into one forward (M = passes * T
    in every projection, attention per pass, perturbed sub-layers skipped for
    their pass only) against the same passes run one after another, over a
    3-step trajectory: the latents agree as closely as the loop agrees with the
    oracle (the projections' kernel / split-K choice changes with M, guidance
    scales up to 7 amplify the fp32 summation-order differences, and the two
    trajectories drift apart step by step).  Pass
    isolation itself is checked bit-exactly by
    test_stacked_pass_velocities_match_single_passes."""
    from ltx_amd.components.guiders import (CFGStarRescalingGuider, MultiModalGuider, MultiModalGuiderParams,
                                            STGGuider)
    from ltx_amd.components.perturbations import create_batched_stg_config
    from ltx_amd.pipeline import denoise_cfg_av, denoise_multimodal_av

    print(f"batched vs sequential passes: {loop}", flush=True)
    steps = 3
    runs = {}
    for batched in (True, False):
        model, state, _, _ = _setup(steps)
        got = []
        cb = lambda s, st: got.append((st.video_latent.float().cpu().clone(), st.audio_latent.float().cpu().clone()))
        if loop == "cfg_stg":
            denoise_cfg_av(model, state, video_guider=CFGStarRescalingGuider(3.0),
                           audio_guider=CFGStarRescalingGuider(7.0), stg_guider=STGGuider(1.0),
                           stg_perturbations=create_batched_stg_config(1, blocks=[1]), stg_cutoff=0.75,
                           callback=cb, batch_passes=batched)
        else:
            denoise_multimodal_av(model, state,
                                  video_guider=MultiModalGuider(MultiModalGuiderParams(cfg_scale=3.0,
                                                                                       modality_scale=3.0)),
                                  audio_guider=MultiModalGuider(MultiModalGuiderParams(cfg_scale=7.0,
                                                                                       modality_scale=3.0)),
                                  callback=cb, batch_passes=batched)
        torch.cuda.synchronize()
        runs[batched] = got
    for step in range(steps):
        (bv, ba), (sv, sa) = runs[True][step], runs[False][step]
        cv, ca = cos_sim(bv.numpy(), sv.numpy()), cos_sim(ba.numpy(), sa.numpy())
        rv = (bv - sv).abs().max().item() / sv.abs().max().item()
        print(f"step {step}: video cos {cv:.7f} rel {rv:.2e} audio cos {ca:.7f}", flush=True)
        assert cv >= 0.999 and ca >= 0.999


def test_stacked_pass_velocities_match_single_passes():
    """model.velocity over three stacked passes -- positive context, negative
    context, positive context with block 1's video self-attention skipped.
    Against stacks of the same shape (same M in every projection, so the same
    kernels) holding other passes: each pass's velocities are bit-identical --
    no pass sees another's rows.  Against single-pass forwards (M three times
    smaller: other kernel / split-K choices): equal to fp32 summation order."""
    from ltx_amd.components.perturbations import (BatchedPerturbationConfig, PerturbationConfig,
                                                  create_stg_perturbation)

    print("stacked pass velocities", flush=True)
    model, state, _, _ = _setup(2)
    pes = model.rope(state.video_positions, state.audio_positions)
    sig = state.sigmas_dev[0:1]
    stg = create_stg_perturbation(blocks=[1])
    none = PerturbationConfig.empty()
    pos = (state.video_context, state.audio_context, none)
    neg = (state.negative_video_context, state.negative_audio_context, none)
    ptb = (state.video_context, state.audio_context, stg)

    def stacked(passes):
        v, a = model.velocity(state.video_latent, torch.stack([p[0] for p in passes]), sig, pes,
                              state.audio_latent, torch.stack([p[1] for p in passes]),
                              perturbations=BatchedPerturbationConfig([p[2] for p in passes]), passes=len(passes))
        return v.float().cpu(), a.float().cpu()

    mixed = stacked([pos, neg, ptb])
    # stacks of the same shape (the third pass perturbed, so every projection
    # has the same M as in the mixed stack): the positive / negative copies
    # agree with each other and with the mixed stack's pass
    ref_pos = stacked([pos, pos, ptb])
    ref_neg = stacked([neg, neg, ptb])
    for m in (0, 1):
        assert torch.equal(ref_pos[m][0], ref_pos[m][1]) and torch.equal(ref_neg[m][0], ref_neg[m][1])
        assert torch.equal(mixed[m][0], ref_pos[m][0]), f"{'video audio'.split()[m]} positive pass"
        assert torch.equal(mixed[m][1], ref_neg[m][0]), f"{'video audio'.split()[m]} negative pass"
        assert torch.equal(mixed[m][2], ref_pos[m][2]) and torch.equal(mixed[m][2], ref_neg[m][2]), \
            f"{'video audio'.split()[m]} perturbed pass"
    for i, p in enumerate((pos, neg, ptb)):
        v1, a1 = model.velocity(state.video_latent, p[0], sig, pes, state.audio_latent, p[1],
                                perturbations=BatchedPerturbationConfig([p[2]]))
        for name, got, ref in (("video", mixed[0][i], v1.float().cpu()), ("audio", mixed[1][i], a1.float().cpu())):
            c = cos_sim(got.numpy(), ref.numpy())
            print(f"pass {i} {name} stacked vs single: cos {c:.7f}", flush=True)
            assert c >= 0.9999
    # the perturbed and negative passes are different forwards than the positive one
    assert cos_sim(mixed[0][2].numpy(), mixed[0][0].numpy()) < 0.99999
    assert cos_sim(mixed[0][1].numpy(), mixed[0][0].numpy()) < 0.99999


def test_captured_guided_loop_is_bit_identical_to_eager():
    """The CFG-star + STG + GE loop (stacked passes) captured as one HIP graph
    per step: replaying the graphs gives the eager loop's latents bit for bit
    at every step; a second generation (the initial noise written back in
    place, eager work in between) replays to the same latents again."""
    from ltx_amd.components.guiders import CFGStarRescalingGuider, STGGuider
    from ltx_amd.components.perturbations import create_batched_stg_config
    from ltx_amd.pipeline import CfgAvLoop

    print("captured guided loop", flush=True)
    steps = 3
    kw = dict(video_guider=CFGStarRescalingGuider(3.0), audio_guider=CFGStarRescalingGuider(7.0),
              stg_guider=STGGuider(1.0), stg_perturbations=create_batched_stg_config(1, blocks=[1]),
              stg_cutoff=0.75, ge_gamma=0.5)
    model, state, _, _ = _setup(steps)
    noise = (state.video_latent.clone(), state.audio_latent.clone())
    eager = []
    CfgAvLoop(model, state, **kw).run(lambda i, st: eager.append((st.video_latent.clone(), st.audio_latent.clone())))
    state.video_latent.copy_(noise[0])
    state.audio_latent.copy_(noise[1])
    loop = CfgAvLoop(model, state, **kw).capture()
    for gen in range(2):
        state.video_latent.copy_(noise[0])
        state.audio_latent.copy_(noise[1])
        torch.randn(1 << 20, device="cuda").sum().item()  # unrelated eager work between generations
        got = []
        loop.run(lambda i, st: got.append((st.video_latent.clone(), st.audio_latent.clone())))
        torch.cuda.synchronize()
        for i in range(steps):
            assert torch.equal(got[i][0], eager[i][0]), f"generation {gen} step {i} video"
            assert torch.equal(got[i][1], eager[i][1]), f"generation {gen} step {i} audio"
