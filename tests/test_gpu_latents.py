"""Latent layouts and latent sidecars on the GPU: the patchifiers
(components/patchifiers.py:52-124, :327-374) bit-exact against numpy's
reshape/transpose restatement of them, state round trips through the VAE
layouts and a sidecar, and a denoise continued from loaded latents."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np_video_patchify(x):  # (B, C, F, H, W) -> (B, F*H*W, C), patch size 1
    b, c, f, h, w = x.shape
    return x.reshape(b, c, f, 1, h, 1, w, 1).transpose(0, 2, 4, 6, 1, 3, 5, 7).reshape(b, f * h * w, c)


def _np_audio_patchify(x):  # (B, C, T, M) -> (B, T, C*M)
    b, c, t, m = x.shape
    return x.transpose(0, 2, 1, 3).reshape(b, t, c * m)


@pytest.mark.parametrize("grid", [(1, 1, 1), (3, 4, 6), (9, 16, 24), (2, 7, 5)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_video_patchify_bit_exact(grid, dtype):
    from ltx_amd.components.patchifiers import VideoLatentPatchifier

    print(f"video patchify grid={grid} {dtype}", flush=True)
    x = torch.randn(1, 128, *grid).to(dtype)
    p = VideoLatentPatchifier(1)
    tok = p.patchify(x.to(DEV))
    ref = _np_video_patchify(x.float().numpy())
    np.testing.assert_array_equal(tok.float().cpu().numpy(), ref)
    back = p.unpatchify(tok, (128, *grid))
    assert torch.equal(back.cpu(), x)


@pytest.mark.parametrize("t", [1, 68, 127])
def test_audio_patchify_bit_exact(t):
    from ltx_amd.components.patchifiers import AudioPatchifier

    x = torch.randn(1, 8, t, 16).bfloat16()
    p = AudioPatchifier(1)
    tok = p.patchify(x.to(DEV))
    np.testing.assert_array_equal(tok.float().cpu().numpy(), _np_audio_patchify(x.float().numpy()))
    assert torch.equal(p.unpatchify(tok, (8, t, 16)).cpu(), x)


def test_state_latents_round_trip_and_continue(tmp_path):
    """Latents saved as a sidecar, loaded into a fresh state, denoised further:
    identical to denoising the original state (same kernels, same inputs)."""
    from ltx_amd import pipeline as pl
    from ltx_amd.model.transformer.model import LTXModel

    model = LTXModel(num_layers=1, weight_format="bf16", seed=2)
    st = pl.DenoiseState(model, height=128, width=192, frames=9, text_tokens=16, audio_frames=12, seed=3)
    pes = model.rope(st.video_positions, st.audio_positions)
    pl.denoise_step(model, st, 0, pes)
    v, a = pl.get_latents(st)
    assert v.shape == (1, 128, 2, 4, 6) and a.shape == (1, 8, 12, 16)
    path = pl.save_distilled_two_stage_latents(str(tmp_path / "run"), v, v, a, a)
    v1, a1, _ = pl.load_stage1_latents(path, device=DEV)
    st2 = pl.DenoiseState(model, height=128, width=192, frames=9, text_tokens=16, audio_frames=12, seed=3)
    pl.set_latents(st2, v1, a1)
    assert torch.equal(st2.video_latent, st.video_latent) and torch.equal(st2.audio_latent, st.audio_latent)
    pl.denoise_step(model, st, 1, pes)
    pl.denoise_step(model, st2, 1, pes)
    torch.cuda.synchronize()
    assert torch.equal(st2.video_latent, st.video_latent) and torch.equal(st2.audio_latent, st.audio_latent)
    with pytest.raises(ValueError, match="does not fit the grid"):
        pl.set_latents(st2, torch.zeros(1, 128, 2, 4, 7, device=DEV))
