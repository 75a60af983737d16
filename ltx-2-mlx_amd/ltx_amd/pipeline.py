"""Audio+video denoise loops on the resident transformer.

* ``denoise`` / ``denoise_step`` restate ``AVPipeline._denoise_loop_simple_av``
  (pipelines/av_pipeline.py:899-1146) for the text-to-video+audio path:
  uniform denoise masks (scalar timestep), no CFG, eight Euler steps over
  ``DISTILLED_SIGMA_VALUES``.
* ``denoise_cfg_av`` restates ``_denoise_loop_cfg_av`` (av_pipeline.py:
  625-757): per step the positive pass, the negative-prompt pass when either
  modality's CFG guider is enabled, and the STG pass (perturbed video
  self-attention) while the step is within the STG cutoff; video and audio
  guided separately, optional GE velocity correction, Euler.
* ``denoise_multimodal_av`` restates the multi-modal guided loop of
  pipelines/two_stage.py:306-388: conditioned, unconditioned and
  modality-isolated passes combined by ``MultiModalGuider``.

``set_latents`` / ``get_latents`` convert between the VAE latent layouts and
the token rows (the patchifiers); ``save_final_latents``,
``save_distilled_two_stage_latents`` and ``load_stage1_latents`` read and
write the reference's latent sidecars; ``load_text_conditioning`` /
``set_contexts`` bring real text contexts (a conditioning sidecar or the
connector's output) into a state.

The sigma schedule lives on the device for the whole loop, RoPE tables are
built once per stage, and a step enqueues its kernels without host
synchronisation (the reference's one per-step barrier, av_pipeline.py:1113,
is left to the caller).  The uniform denoise mask makes the reference's
``maybe_post_process_latent`` the identity (pipelines/common.py:299-318).
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib
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
        self.grid = (f, h, w)
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
        self.sigmas = [float(np.float32(s)) for s in sigmas]
        self.sigmas_dev = torch.tensor(self.sigmas, dtype=torch.float32, device=dev)
        # negative-prompt contexts of the guided loops (synthetic, own stream of draws)
        neg = torch.Generator(device=dev)
        neg.manual_seed(seed + 0x5EED)
        self.negative_video_context = torch.randn((text_tokens, model.video_dim), generator=neg,
                                                  device=dev).to(torch.bfloat16)
        self.negative_audio_context = torch.randn((text_tokens, model.audio_dim), generator=neg,
                                                  device=dev).to(torch.bfloat16)


def set_latents(state: DenoiseState, video_latent: torch.Tensor, audio_latent: torch.Tensor | None = None) -> None:
    """Start ``state`` from given latents in the VAE layouts -- video (1, 128,
    F, H, W), audio (1, 8, T, 16) -- patchified into the token rows (e.g. a
    stage-1 result read with ``load_stage1_latents``)."""
    from .components.patchifiers import AudioPatchifier, VideoLatentPatchifier

    f, h, w = state.grid
    if tuple(video_latent.shape[2:]) != (f, h, w) or video_latent.shape[1] != 128:
        raise ValueError(f"video latent {tuple(video_latent.shape)} does not fit the grid {(f, h, w)}")
    v = VideoLatentPatchifier(1).patchify(video_latent.to(state.video_latent.device, torch.bfloat16))
    state.video_latent.copy_(v[0])
    if audio_latent is not None:
        if state.audio_tokens != audio_latent.shape[2]:
            raise ValueError(f"audio latent {tuple(audio_latent.shape)} has {audio_latent.shape[2]} frames, "
                             f"the state {state.audio_tokens}")
        a = AudioPatchifier(1).patchify(audio_latent.to(state.audio_latent.device, torch.bfloat16))
        state.audio_latent.copy_(a[0])


def get_latents(state: DenoiseState) -> tuple[torch.Tensor, torch.Tensor | None]:
    """The state's latents unpatchified: video (1, 128, F, H, W), audio
    (1, 8, T, 16) or None."""
    from .components.patchifiers import (AUDIO_LATENT_CHANNELS, AUDIO_MEL_BINS, AudioPatchifier,
                                         VideoLatentPatchifier)

    f, h, w = state.grid
    video = VideoLatentPatchifier(1).unpatchify(state.video_latent[None], (128, f, h, w))
    audio = None
    if state.audio_tokens:
        audio = AudioPatchifier(1).unpatchify(state.audio_latent[None],
                                              (AUDIO_LATENT_CHANNELS, state.audio_tokens, AUDIO_MEL_BINS))
    return video, audio


def save_final_latents(path: str, video_latent: torch.Tensor, audio_latent: torch.Tensor | None = None) -> str:
    """``final_video_latent`` / ``final_audio_latent`` sidecar
    (av_pipeline.py:233-253); returns the path written."""
    from .sidecars import save_sidecar

    arrays = {"final_video_latent": video_latent}
    if audio_latent is not None:
        arrays["final_audio_latent"] = audio_latent
    return save_sidecar(path, arrays)


def save_distilled_two_stage_latents(path: str, stage_1_video_latent: torch.Tensor,
                                     stage_2_video_latent: torch.Tensor,
                                     stage_1_audio_latent: torch.Tensor | None = None,
                                     stage_2_audio_latent: torch.Tensor | None = None) -> str:
    """Both distilled stages plus the final-latent keys (av_pipeline.py:255-290)."""
    from .sidecars import save_sidecar

    arrays = {"stage_1_video_latent": stage_1_video_latent, "stage_2_video_latent": stage_2_video_latent,
              "final_video_latent": stage_2_video_latent}
    if stage_1_audio_latent is not None:
        arrays["stage_1_audio_latent"] = stage_1_audio_latent
    if stage_2_audio_latent is not None:
        arrays["stage_2_audio_latent"] = stage_2_audio_latent
        arrays["final_audio_latent"] = stage_2_audio_latent
    return save_sidecar(path, arrays, metadata={"pipeline": "distilled_two_stage"})


def load_stage1_latents(path: str, device: str | torch.device = "cpu"):
    """``(video, audio or None, metadata)`` of a two-stage sidecar
    (scripts/stage2_harness.py:56-74)."""
    from .sidecars import load_sidecar

    arrays, file_metadata = load_sidecar(path, device=device)
    if "stage_1_video_latent" not in arrays:
        raise ValueError(f"{path} does not contain stage_1_video_latent. "
                         "Use a distilled two-stage latent sidecar saved with --save-latents.")
    video = arrays["stage_1_video_latent"]
    audio = arrays.get("stage_1_audio_latent")
    metadata = {"pipeline": file_metadata.get("pipeline"), "video_shape": tuple(video.shape),
                "audio_shape": tuple(audio.shape) if audio is not None else None}
    return video, audio, metadata


def infer_dimensions_from_stage1(video_latent: torch.Tensor) -> tuple[int, int, int]:
    """(height, width, frames) of the full-resolution output of a stage-1
    latent (half resolution, scripts/stage2_harness.py:77-85)."""
    if video_latent.dim() != 5:
        raise ValueError(f"stage_1_video_latent must be 5D (B,C,F,H,W), got shape {tuple(video_latent.shape)}")
    frames = (video_latent.shape[2] - 1) * 8 + 1
    return video_latent.shape[3] * 64, video_latent.shape[4] * 64, frames


def load_text_conditioning(path: str, device: str | torch.device = "cpu") -> dict:
    """The text-conditioning sidecar of a run (generate.py:1531-1560): the
    ``positive_video_encoding`` / ``negative_*`` / ``*_audio_encoding`` and
    attention masks, or a legacy ``embedding`` + ``attention_mask`` file."""
    from .sidecars import load_sidecar

    arrays, _ = load_sidecar(path, device=device)
    if "positive_video_encoding" not in arrays:
        return {"format": "legacy", "positive_video_encoding": arrays["embedding"],
                "positive_attention_mask": arrays["attention_mask"], "negative_video_encoding": None,
                "negative_attention_mask": None, "positive_audio_encoding": None, "negative_audio_encoding": None}
    keys = ("positive_video_encoding", "positive_attention_mask", "negative_video_encoding", "negative_attention_mask",
            "positive_audio_encoding", "negative_audio_encoding")
    out = {"format": "text_conditioning"}
    out.update({k: arrays.get(k) for k in keys})
    return out


def set_contexts(state: DenoiseState, video_context: torch.Tensor, audio_context: torch.Tensor | None = None,
                 negative_video_context: torch.Tensor | None = None,
                 negative_audio_context: torch.Tensor | None = None) -> None:
    """Replace the state's text contexts ((1, S, D) or (S, D), any S) -- e.g.
    the connector's output or a loaded text-conditioning sidecar."""
    dev = state.video_latent.device

    def two_d(t):
        t = t[0] if t.dim() == 3 else t
        return t.to(device=dev, dtype=torch.bfloat16).contiguous()

    state.video_context = two_d(video_context)
    if audio_context is not None:
        state.audio_context = two_d(audio_context)
    if negative_video_context is not None:
        state.negative_video_context = two_d(negative_video_context)
    if negative_audio_context is not None:
        state.negative_audio_context = two_d(negative_audio_context)


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


def condition_video(state: DenoiseState, denoise_mask, clean_latent: torch.Tensor) -> None:
    """Image / keyframe conditioning of the video tokens: a 0 / 1 denoise
    mask (T,) -- 0 on conditioned tokens -- and the clean latent rows (T, 128)
    they hold.  The conditioned rows of the state's latent become the clean
    rows (noisers.py:40-80 with a hard mask: ``clean + mask * (noise -
    clean)``); ``denoise_conditioned`` then keeps them there."""
    from .model.transformer.model import token_timestep_groups

    mask = torch.as_tensor(denoise_mask).detach().float().reshape(-1).cpu()
    if mask.numel() != state.video_tokens or not bool(((mask == 0) | (mask == 1)).all()):
        raise ValueError(f"a 0 / 1 denoise mask over the {state.video_tokens} video tokens is expected")
    clean = clean_latent.to(device=state.video_latent.device, dtype=torch.bfloat16).reshape(state.video_tokens, -1)
    state.video_denoise_mask = mask
    state.video_clean_latent = clean.contiguous()
    for r0, r1, g in token_timestep_groups(mask).segments:
        if float(mask[r0]) == 0.0:
            state.video_latent[r0:r1].copy_(state.video_clean_latent[r0:r1])


def denoise_conditioned(model: LTXModel, state: DenoiseState, callback=None) -> DenoiseState:
    """The distilled loop (av_pipeline.py:899-1146) with the non-uniform video
    denoise mask of ``condition_video``: per step the video timesteps are
    ``sigma * mask`` (common.py:194-204) -- per-token, as row groups -- the X0
    prediction ``latent - t * velocity`` per row group (model.py:1519-1525),
    blended with the clean latent where the mask is 0 (common.py:169-191,
    :299-318), then the Euler step (diffusion_steps.py:19-69); the audio
    stream's mask is uniform."""
    from .components.diffusion_steps import to_denoised
    from .model.transformer.model import TokenTimesteps, token_timestep_groups

    mask = state.video_denoise_mask
    base = token_timestep_groups(mask)
    pes = model.rope(state.video_positions, state.audio_positions)
    stepper = EulerDiffusionStep()
    dev = state.video_latent.device
    audio = state.audio_tokens > 0
    for step in range(len(state.sigmas) - 1):
        sigma, sigma_next = state.sigmas[step], state.sigmas[step + 1]
        values = [float(np.float32(np.float32(v) * np.float32(sigma))) for v in base.values]
        groups = TokenTimesteps(values, base.segments)
        sig = state.sigmas_dev[step:step + 1]
        t0 = torch.tensor(values[:1], dtype=torch.float32, device=dev)
        v_vel, a_vel = model.velocity(state.video_latent, state.video_context, sig, pes,
                                      state.audio_latent if audio else None, state.audio_context if audio else None,
                                      sigmas=(t0, sig, sig, sig),
                                      video_token_timesteps=groups if len(values) > 1 else None)
        denoised = torch.empty(state.video_latent.shape, dtype=torch.float32, device=dev)
        for r0, r1, g in groups.segments:
            if float(mask[r0]) == 0.0:
                denoised[r0:r1] = state.video_clean_latent[r0:r1].float()  # the clean rows (mask 0)
            else:
                denoised[r0:r1] = to_denoised(state.video_latent[r0:r1], v_vel[r0:r1], values[g])
        stepper.step(state.video_latent, denoised, state.sigmas, step, out=state.video_latent)
        if a_vel is not None:
            stepper.step_from_velocity(state.audio_latent, a_vel, sigma, sigma_next, out=state.audio_latent)
        if callback is not None:
            callback(step, state)
    return state


def _velocities(model: LTXModel, state: DenoiseState, sig, pes, video_context, audio_context, perturbations=None):
    audio = state.audio_tokens > 0
    return model.velocity(state.video_latent, video_context, sig, pes,
                          state.audio_latent if audio else None, audio_context if audio else None,
                          perturbations=perturbations)


def _stacked_passes(model: LTXModel, state: DenoiseState, sig, pes, contexts: list, perturbations: list):
    """The passes of one guided step as one forward with their tokens
    stacked by rows: ``contexts`` holds (video, audio) context pairs, one per
    pass; ``perturbations`` one ``PerturbationConfig`` (or None) per pass.
    Returns per-pass (video velocity, audio velocity) pairs."""
    from .components.perturbations import BatchedPerturbationConfig, PerturbationConfig

    n = len(contexts)
    audio = state.audio_tokens > 0
    vctx = torch.stack([c[0] for c in contexts])
    actx = torch.stack([c[1] for c in contexts]) if audio else None
    pert = None
    if any(p is not None for p in perturbations):
        pert = BatchedPerturbationConfig([p if p is not None else PerturbationConfig.empty() for p in perturbations])
    v, a = model.velocity(state.video_latent, vctx, sig, pes, state.audio_latent if audio else None, actx,
                          perturbations=pert, passes=n)
    return [(v[i], a[i] if audio else None) for i in range(n)]


class CfgAvLoop:
    """The guided joint denoising loop with separate guidance per modality
    (av_pipeline.py:625-757) as a step function over a ``DenoiseState``:
    ``step(i)`` enqueues step i (its transformer passes, guidance, optional
    GE velocity correction and the Euler update, in place on the state's
    latents) without host synchronisation.

    With ``batch_passes`` (default) the positive, negative-prompt and STG
    passes of a step run as one forward over their stacked tokens (the
    reference runs them one after another, av_pipeline.py:688-717); each
    pass's tokens see exactly the arithmetic of a pass of its own.  The
    contexts of the stacked passes must have equal lengths; otherwise, or with
    ``batch_passes=False``, the passes run one after another.

    ``capture()`` records every step as a HIP graph (one per step: the step's
    sigmas and flags are launch arguments); ``replay(i)`` then runs step i
    from its graph, on the same state buffers -- a new generation of the same
    shape and schedule writes its noise into ``state.video_latent`` /
    ``state.audio_latent`` in place and replays."""

    def __init__(self, model: LTXModel, state: DenoiseState, *, video_guider, audio_guider, stg_guider=None,
                 stg_perturbations=None, stg_cutoff: float = 1.0, ge_gamma: float = 0.0,
                 batch_passes: bool = True):
        self.model, self.state = model, state
        self.video_guider, self.audio_guider, self.stg_guider = video_guider, audio_guider, stg_guider
        self.stg_perturbations, self.stg_cutoff, self.ge_gamma = stg_perturbations, stg_cutoff, ge_gamma
        self.batch_passes = batch_passes
        self.pes = model.rope(state.video_positions, state.audio_positions)
        self.stepper = EulerDiffusionStep()
        self.num_steps = len(state.sigmas) - 1
        self.need_cfg = video_guider.enabled() or audio_guider.enabled()
        self.audio = state.audio_tokens > 0
        self.stg_one = None
        if stg_perturbations is not None:
            if len(stg_perturbations.perturbations) != 1:
                raise ValueError("the STG pass takes one perturbation config")
            self.stg_one = stg_perturbations.perturbations[0]
        # GE correction: the previous step's velocity (fixed buffer, so every
        # step's graph reads and writes the same memory) and whether it holds one
        self.prev_velocity = (torch.empty(state.video_latent.shape, dtype=torch.float32, device=model.device)
                              if ge_gamma > 0 else None)
        self.prev_valid = False
        self.graphs: list | None = None

    def step(self, step: int) -> None:
        from .components.diffusion_steps import to_denoised

        model, state, pes, audio = self.model, self.state, self.pes, self.audio
        sigma = state.sigmas[step]
        sig = state.sigmas_dev[step:step + 1]
        stg_active = (self.stg_guider is not None and self.stg_guider.enabled() and self.stg_perturbations is not None
                      and (step + 1) / self.num_steps <= self.stg_cutoff)
        pos_ctx = (state.video_context, state.audio_context)
        neg_ctx = (state.negative_video_context, state.negative_audio_context)
        contexts, perts = [pos_ctx], [None]
        if self.need_cfg:
            contexts.append(neg_ctx)
            perts.append(None)
        if stg_active:
            contexts.append(pos_ctx)
            perts.append(self.stg_one)
        same_len = all(c[0].shape == pos_ctx[0].shape and (not audio or c[1].shape == pos_ctx[1].shape)
                       for c in contexts)
        if self.batch_passes and len(contexts) > 1 and same_len:
            vel = _stacked_passes(model, state, sig, pes, contexts, perts)
        else:
            vel = [_velocities(model, state, sig, pes, c[0], c[1],
                               perturbations=None if p is None else self.stg_perturbations)
                   for c, p in zip(contexts, perts)]
        v_pos, a_pos = vel[0]
        video_d = to_denoised(state.video_latent, v_pos, sigma)
        audio_d = to_denoised(state.audio_latent, a_pos, sigma) if audio else None
        if self.need_cfg:
            v_neg, a_neg = vel[1]
            video_d = self.video_guider.guide(video_d, to_denoised(state.video_latent, v_neg, sigma))
            if audio:
                audio_d = self.audio_guider.guide(audio_d, to_denoised(state.audio_latent, a_neg, sigma))
        if stg_active:
            v_ptb, _ = vel[-1]
            video_d = self.stg_guider.guide(video_d, to_denoised(state.video_latent, v_ptb, sigma))
        if self.ge_gamma > 0 and sigma > 0:
            _lib.call("ltx_ge_correct_f32", _lib.ptr(state.video_latent), _lib.ptr(video_d),
                      _lib.ptr(self.prev_velocity), int(self.prev_valid), float(sigma), float(self.ge_gamma),
                      video_d.numel(), _lib.stream_of(video_d))
            self.prev_valid = True
        self.stepper.step(state.video_latent, video_d, state.sigmas, step, out=state.video_latent)
        if audio:
            self.stepper.step(state.audio_latent, audio_d, state.sigmas, step, out=state.audio_latent)

    def run(self, callback=None) -> DenoiseState:
        """Every step in order (from the graphs when captured)."""
        for i in range(self.num_steps):
            if self.graphs is not None:
                self.graphs[i].replay()
            else:
                self.step(i)
            if callback is not None:
                callback(i, self.state)
        return self.state

    def capture(self, pool=None) -> "CfgAvLoop":
        """Record every step as a HIP graph (nothing runs).  The first step's
        work is run once eagerly first -- on a copy of the latents, restored
        after -- so every lazily built table and workspace exists before
        capture."""
        st = self.state
        saved = (st.video_latent.clone(), st.audio_latent.clone(), self.prev_valid)
        self.step(0)
        torch.cuda.synchronize()
        st.video_latent.copy_(saved[0])
        st.audio_latent.copy_(saved[1])
        self.prev_valid = saved[2]
        pool = torch.cuda.graph_pool_handle() if pool is None else pool
        graphs = []
        for i in range(self.num_steps):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self.step(i)
            graphs.append(g)
        torch.cuda.synchronize()
        self.graphs = graphs
        self.prev_valid = saved[2]
        return self


def denoise_cfg_av(model: LTXModel, state: DenoiseState, *, video_guider, audio_guider, stg_guider=None,
                   stg_perturbations=None, stg_cutoff: float = 1.0, ge_gamma: float = 0.0,
                   callback=None, batch_passes: bool = True) -> DenoiseState:
    """Guided joint denoising with separate guidance per modality
    (av_pipeline.py:625-757), in place on ``state``'s latents; the loop of
    ``CfgAvLoop`` run eagerly."""
    loop = CfgAvLoop(model, state, video_guider=video_guider, audio_guider=audio_guider, stg_guider=stg_guider,
                     stg_perturbations=stg_perturbations, stg_cutoff=stg_cutoff, ge_gamma=ge_gamma,
                     batch_passes=batch_passes)
    return loop.run(callback)


def denoise_multimodal_av(model: LTXModel, state: DenoiseState, *, video_guider, audio_guider,
                          callback=None, batch_passes: bool = True) -> DenoiseState:
    """Multi-modal guided joint denoising (pipelines/two_stage.py:306-388):
    conditioned pass, unconditioned pass when either guider runs CFG,
    modality-isolated pass (A2V and V2A skipped in every block) when either
    runs modality guidance; ``MultiModalGuider.calculate`` per modality.
    ``batch_passes`` stacks the passes of a step into one forward, as in
    ``denoise_cfg_av``."""
    from .components.diffusion_steps import to_denoised
    from .components.perturbations import modality_isolation_config

    pes = model.rope(state.video_positions, state.audio_positions)
    stepper = EulerDiffusionStep()
    audio = state.audio_tokens > 0
    iso = modality_isolation_config()
    for step in range(len(state.sigmas) - 1):
        sigma = state.sigmas[step]
        sig = state.sigmas_dev[step:step + 1]
        x_v, x_a = state.video_latent, state.audio_latent

        def den(v, a):
            return to_denoised(x_v, v, sigma), (to_denoised(x_a, a, sigma) if audio else None)

        pos_ctx = (state.video_context, state.audio_context)
        contexts, perts = [pos_ctx], [None]
        do_uncond = video_guider.do_unconditional_generation() or audio_guider.do_unconditional_generation()
        do_iso = video_guider.do_isolated_modality_generation() or audio_guider.do_isolated_modality_generation()
        if do_uncond:
            contexts.append((state.negative_video_context, state.negative_audio_context))
            perts.append(None)
        if do_iso:
            contexts.append(pos_ctx)
            perts.append(iso.perturbations[0])
        same_len = all(c[0].shape == pos_ctx[0].shape and (not audio or c[1].shape == pos_ctx[1].shape)
                       for c in contexts)
        if batch_passes and len(contexts) > 1 and same_len:
            vel = _stacked_passes(model, state, sig, pes, contexts, perts)
        else:
            vel = [_velocities(model, state, sig, pes, c[0], c[1], perturbations=None if p is None else iso)
                   for c, p in zip(contexts, perts)]
        cond_v, cond_a = den(*vel[0])
        uncond_v = uncond_a = 0.0
        if do_uncond:
            uncond_v, uncond_a = den(*vel[1])
        mod_v = mod_a = 0.0
        if do_iso:
            mod_v, mod_a = den(*vel[-1])
        video_d = video_guider.calculate(cond_v, uncond_v, 0.0, mod_v)
        stepper.step(x_v, video_d, state.sigmas, step, out=x_v)
        if audio:
            audio_d = audio_guider.calculate(cond_a, uncond_a, 0.0, mod_a)
            stepper.step(x_a, audio_d, state.sigmas, step, out=x_a)
        if callback is not None:
            callback(step, state)
    return state
