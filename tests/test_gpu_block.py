"""Block-level GPU parity: BasicAVTransformerBlock on HIP kernels vs the oracle.

Configs: the video block at 3456 tokens with 256 text tokens, and the joint
AV block (3456 video + 68 audio tokens), random-init bf16 weights
~N(0, 0.02), AdaLN rows from a sigma-0.5 timestep-like draw.  Gate: the
north-star bf16 tolerance -- normwise max relative error <= 1e-2 against the
fp32 oracle -- plus cosine >= 0.999 on each stream.  Also the int8 and MXFP8
weight formats (oracle fed the decoded weights) and the block's contract
(inputs untouched, disabled modality passed through, perturbation skip).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import cos_sim, max_rel_err
from _weights import block_weights
from oracle import block as ob
from oracle import rope as orope

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cfgs(audio: bool):
    from ltx_amd.model.transformer.transformer import TransformerConfig

    v = TransformerConfig(4096, 32, 128, 4096, True, True)
    a = TransformerConfig(2048, 32, 64, 2048, True, True) if audio else None
    return v, a


def _inputs(tv, ta, s=256, seed=0):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    def rn(shape, std=1.0):
        return (torch.randn(shape, generator=g, device=DEV) * std).to(torch.bfloat16)
    vx, vctx = rn((tv, 4096)), rn((s, 4096))
    ax, actx = (rn((ta, 2048)), rn((s, 2048))) if ta else (None, None)
    # timestep rows as the AdaLN MLP would produce (fp32, modest magnitude)
    vt = torch.randn((16, 4096), generator=g, device=DEV) * 0.1
    at = torch.randn((16, 2048), generator=g, device=DEV) * 0.1
    return vx, vctx, ax, actx, vt, at


def _pes(tv_grid, ta):
    vpos = orope.video_positions(*tv_grid, fps=24.0)
    vpe = orope.rope_tables(vpos, 4096, 32, orope.VIDEO_MAX_POS)
    if not ta:
        return vpe, None, None, None
    apos = orope.audio_positions(ta)
    ape = orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS)
    vxpe = orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS)
    axpe = orope.rope_tables(apos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS)
    return vpe, vxpe, ape, axpe


def _to_dev(pe):
    return None if pe is None else tuple(torch.from_numpy(a).to(DEV) for a in pe)


def _to_cpu(pe):
    return None if pe is None else tuple(torch.from_numpy(a) for a in pe)


def _run(weight_format, grid, ta, seed=1):
    from ltx_amd.model.transformer.transformer import BasicAVTransformerBlock, TransformerArgs

    vcfg, acfg = _cfgs(ta > 0)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    blk = BasicAVTransformerBlock(0, vcfg, acfg, weight_format=weight_format, generator=gen)
    tv = grid[0] * grid[1] * grid[2]
    vx, vctx, ax, actx, vt, at = _inputs(tv, ta, seed=seed)
    vpe, vxpe, ape, axpe = _pes(grid, ta)
    video = TransformerArgs(x=vx[None], context=vctx[None], timesteps=vt[:9].reshape(1, 1, 9, -1),
                            positional_embeddings=_to_dev(vpe), cross_positional_embeddings=_to_dev(vxpe),
                            prompt_timestep=vt[9:11].reshape(1, 1, 2, -1),
                            cross_scale_shift_timestep=vt[11:15].reshape(1, 1, 4, -1),
                            cross_gate_timestep=vt[15:16].reshape(1, 1, 1, -1))
    audio = None
    if ta:
        audio = TransformerArgs(x=ax[None], context=actx[None], timesteps=at[:9].reshape(1, 1, 9, -1),
                                positional_embeddings=_to_dev(ape), cross_positional_embeddings=_to_dev(axpe),
                                prompt_timestep=at[9:11].reshape(1, 1, 2, -1),
                                cross_scale_shift_timestep=at[11:15].reshape(1, 1, 4, -1),
                                cross_gate_timestep=at[15:16].reshape(1, 1, 1, -1))
    vx_before = vx.clone()
    vo, ao = blk(video, audio)
    torch.cuda.synchronize()
    assert torch.equal(vx, vx_before), "block modified its input"
    W = block_weights(blk)
    v_ada = (blk.video_tables + vt).float().cpu()
    a_ada = (blk.audio_tables + at).float().cpu() if ta else None
    rv, ra = ob.block(W, vx.float().cpu(), ax.float().cpu() if ta else None, v_ada, a_ada,
                      vctx.float().cpu(), actx.float().cpu() if ta else None,
                      _to_cpu(vpe), _to_cpu(vxpe), _to_cpu(ape), _to_cpu(axpe))
    return vo.x[0].float().cpu().numpy(), rv.numpy(), (None if not ta else ao.x[0].float().cpu().numpy()), \
        (None if not ta else ra.numpy())


def _gate(got, ref, label):
    rel, cs = max_rel_err(got, ref), cos_sim(got, ref)
    print(f"{label}: max_rel_err={rel:.3e} cos={cs:.6f}", flush=True)
    assert rel <= 1e-2 and cs >= 0.999, label


def test_video_block_3456_tokens():
    gv, rv, _, _ = _run("bf16", (9, 16, 24), 0)
    _gate(gv, rv, "video block")


def test_av_block_3456_plus_68():
    gv, rv, ga, ra = _run("bf16", (9, 16, 24), 68)
    _gate(gv, rv, "AV block video")
    _gate(ga, ra, "AV block audio")


@pytest.mark.parametrize("fmt", ["int8", "mxfp8"])
def test_av_block_quantised_weights(fmt):
    gv, rv, ga, ra = _run(fmt, (3, 8, 12), 20, seed=3)
    _gate(gv, rv, f"{fmt} video")
    _gate(ga, ra, f"{fmt} audio")


def test_block_contract_passthrough_and_skip():
    from ltx_amd.components.perturbations import create_batched_stg_config
    from ltx_amd.model.transformer.transformer import BasicAVTransformerBlock, TransformerArgs

    vcfg, acfg = _cfgs(True)
    blk = BasicAVTransformerBlock(5, vcfg, acfg)
    vx, vctx, ax, actx, vt, at = _inputs(96, 16, s=32, seed=9)
    vpe, vxpe, ape, axpe = _pes((1, 8, 12), 16)
    mk = lambda x, c, t, pe, xpe, en=True: TransformerArgs(  # noqa: E731
        x=x[None], context=c[None], timesteps=t[:9].reshape(1, 1, 9, -1), positional_embeddings=_to_dev(pe),
        cross_positional_embeddings=_to_dev(xpe), prompt_timestep=t[9:11].reshape(1, 1, 2, -1),
        cross_scale_shift_timestep=t[11:15].reshape(1, 1, 4, -1), cross_gate_timestep=t[15:].reshape(1, 1, 1, -1),
        enabled=en)
    video, audio = mk(vx, vctx, vt, vpe, vxpe), mk(ax, actx, at, ape, axpe, en=False)
    vo, ao = blk(video, audio)
    assert ao is audio  # disabled modality passes through untouched
    # skipping every sub-layer that can be skipped leaves text CA + FF: the
    # output must differ from the input but equal a run with skips on both
    pert = create_batched_stg_config(1, skip_video_self_attn=True, blocks=[5])
    vo2, _ = blk(video, None, perturbations=pert)
    vo3, _ = blk(video, None, perturbations=create_batched_stg_config(1, blocks=[4]))
    torch.cuda.synchronize()
    assert not torch.equal(vo2.x, vo3.x)
