"""Distilled audio+video denoise loop on the resident transformer.

Restates ``AVPipeline._denoise_loop_simple_av`` (pipelines/av_pipeline.py:
899-1146) for the text-to-video+audio path: uniform denoise masks (scalar
timestep), no CFG, eight Euler steps over ``DISTILLED_SIGMA_VALUES``.  The
sigma schedule lives on the device for the whole loop, RoPE tables are built
once per stage, and a step enqueues its kernels without host synchronisation
(the reference's one per-step barrier, av_pipeline.py:1113, is left to the
caller).
"""

from __future__ import annotations

import numpy as np
import torch

from .components.diffusion_steps import EulerDiffusionStep
from .components.patchifiers import audio_latent_frames, video_latent_grid
from .components.schedulers import DISTILLED_SIGMA_VALUES
from .model.transformer.model import LTXModel
from .model.transformer.rope import audio_positions, video_positions


class DenoiseState:
    """Latents, contexts and positions of one generation."""

    def __init__(self, model: LTXModel, height: int, width: int, frames: int, fps: float = 24.0,
                 text_tokens: int = 256, audio_frames: int | None = None, seed: int = 0,
                 sigmas=DISTILLED_SIGMA_VALUES):
        dev = model.device
        f, h, w = video_latent_grid(height, width, frames)
        self.video_tokens = f * h * w
        self.audio_tokens = audio_latent_frames(frames, fps) if audio_frames is None else audio_frames
        if model.audio_config is None:
            self.audio_tokens = 0
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        # Gaussian noise at sigma 1 on a zero latent (noisers.py:62-75)
        self.video_latent = torch.randn((self.video_tokens, 128), generator=gen, device=dev).to(torch.bfloat16)
        self.audio_latent = torch.randn((self.audio_tokens, 128), generator=gen, device=dev).to(torch.bfloat16)
        self.video_context = torch.randn((text_tokens, model.video_dim), generator=gen, device=dev).to(torch.bfloat16)
        self.audio_context = torch.randn((text_tokens, model.audio_dim), generator=gen, device=dev).to(torch.bfloat16)
        self.video_positions = video_positions(f, h, w, fps)
        self.audio_positions = audio_positions(self.audio_tokens) if self.audio_tokens else None
        self.sigmas = [float(s) for s in sigmas]
        self.sigmas_dev = torch.tensor(self.sigmas, dtype=torch.float32, device=dev)


def denoise_step(model: LTXModel, state: DenoiseState, step: int, pes=None,
                 stepper: EulerDiffusionStep | None = None, profile_events: list | None = None) -> None:
    """Advance ``state`` by one Euler step in place."""
    stepper = stepper or EulerDiffusionStep()
    if pes is None:
        pes = model.rope(state.video_positions, state.audio_positions)
    sigma, sigma_next = state.sigmas[step], state.sigmas[step + 1]
    sig = state.sigmas_dev[step:step + 1]
    v_vel, a_vel = model.velocity(state.video_latent, state.video_context, sig, pes,
                                  state.audio_latent if state.audio_tokens else None,
                                  state.audio_context if state.audio_tokens else None,
                                  profile_events=profile_events)
    stepper.step_from_velocity(state.video_latent, v_vel, sigma, sigma_next, out=state.video_latent)
    if a_vel is not None:
        stepper.step_from_velocity(state.audio_latent, a_vel, sigma, sigma_next, out=state.audio_latent)


def denoise(model: LTXModel, state: DenoiseState, callback=None) -> DenoiseState:
    pes = model.rope(state.video_positions, state.audio_positions)
    stepper = EulerDiffusionStep()
    for step in range(len(state.sigmas) - 1):
        denoise_step(model, state, step, pes, stepper)
        if callback is not None:
            callback(step, state)
    return state
