"""Whole-model GPU parity: the 8-step distilled AV denoise vs the oracle.

A 2-block model at the full widths (video 4096 / audio 2048, 32 heads) on a
small latent grid (2x4x6 video tokens, 12 audio tokens, 16 text tokens) so
the CPU oracle finishes in seconds.  Gate: per-step latent
cosine >= 0.999 over all 8 steps, for video and audio.  The full-size run
(48 blocks, 3456 + 68 tokens) is exercised by bench.py and smoke().
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import cos_sim
from _weights import block_weights, mlp_weights
from oracle import block as ob
from oracle import rope as orope

pytestmark = pytest.mark.gpu
DEV = "cuda"


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


@pytest.mark.parametrize("fmt", ["bf16", "mxfp8"])
def test_eight_step_denoise_cosine(fmt):
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.pipeline import DenoiseState, denoise

    model = LTXModel(num_layers=2, weight_format=fmt, seed=11)
    state = DenoiseState(model, height=128, width=192, frames=9, text_tokens=16, audio_frames=12, seed=5)
    assert state.video_tokens == 2 * 4 * 6
    MW = _model_weights(model)
    vlat = state.video_latent.float().cpu()
    alat = state.audio_latent.float().cpu()
    vctx, actx = state.video_context.float().cpu(), state.audio_context.float().cpu()
    vpos, apos = state.video_positions, state.audio_positions
    pes_np = (orope.rope_tables(vpos, 4096, 32, orope.VIDEO_MAX_POS),
              orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS),
              orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS),
              orope.rope_tables(apos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS))
    pes = tuple(tuple(torch.from_numpy(a) for a in p) for p in pes_np)
    # product tables equal the oracle's bit for bit
    from ltx_amd.model.transformer.rope import expand_tables

    gpes = model.rope(vpos, apos)
    for g, o in zip(gpes, pes):  # factored forms expanded to per-token rows
        for gt, ot in zip(expand_tables(g), o):
            assert torch.equal(gt.view(torch.int32), ot.view(torch.int32))
    got = []
    denoise(model, state, callback=lambda step, st: got.append(
        (st.video_latent.float().cpu().clone(), st.audio_latent.float().cpu().clone())))
    sig = state.sigmas
    for step in range(8):
        vlat, alat = ob.model_step(MW, vlat, alat, vctx, actx, sig[step], sig[step + 1], pes)
        cv, ca = cos_sim(got[step][0].numpy(), vlat.numpy()), cos_sim(got[step][1].numpy(), alat.numpy())
        print(f"{fmt} step {step}: video cos {cv:.6f} audio cos {ca:.6f}", flush=True)
        assert cv >= 0.999 and ca >= 0.999
    assert torch.isfinite(got[-1][0]).all() and torch.isfinite(got[-1][1]).all()


def test_concurrent_audio_stream_is_bit_identical_and_graph_safe():
    """The audio stream on its own HIP stream gives the serial result bit for
    bit (same kernels, same inputs; only the launch streams differ), eagerly
    and as a captured graph replayed several times with eager work and
    synchronisation in between.  Larger video grid so both streams overlap."""
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.pipeline import DenoiseState, denoise_step

    model = LTXModel(num_layers=2, weight_format="bf16", seed=3)
    state = DenoiseState(model, height=256, width=256, frames=17, text_tokens=32, audio_frames=20, seed=9)
    pes = model.rope(state.video_positions, state.audio_positions)
    v0, a0 = state.video_latent.clone(), state.audio_latent.clone()

    def run(concurrent, step=1):
        model.concurrent_audio = concurrent
        state.video_latent.copy_(v0)
        state.audio_latent.copy_(a0)
        denoise_step(model, state, step, pes)
        torch.cuda.synchronize()
        return state.video_latent.clone(), state.audio_latent.clone()

    sv, sa = run(False)
    cv, ca = run(True)
    assert torch.equal(sv, cv) and torch.equal(sa, ca)

    model.concurrent_audio = True
    state.video_latent.copy_(v0)
    state.audio_latent.copy_(a0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        denoise_step(model, state, 1, pes)
    torch.cuda.synchronize()
    for rep in range(3):
        state.video_latent.copy_(v0)
        state.audio_latent.copy_(a0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(state.video_latent, sv), f"replay {rep} video"
        assert torch.equal(state.audio_latent, sa), f"replay {rep} audio"
        run(False, step=2)  # eager work between replays
