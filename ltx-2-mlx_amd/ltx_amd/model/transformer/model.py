"""LTX-2.3 audio+video transformer with all blocks resident in HBM.

Mirrors ``LTXModel`` / ``X0Model`` (model/transformer/model.py:497-1546) for
the distilled text-to-video+audio path:

* preprocess (:285-497): patchify projection, the four AdaLN MLPs per
  modality (timestep, prompt, cross scale/shift, cross gate), RoPE tables;
* block scheduler (:1044-1310): the reference streams or compiles groups of
  blocks and materialises every N blocks; here all blocks' weights stay
  resident (about 37 GB bf16 or 19 GB MXFP8 of the 288 GB HBM) and the loop
  only enqueues kernels on one stream -- no host synchronisation inside a
  step.  The modulation rows of every block are computed in one launch
  (table + timestep embedding) before the loop;
* output head (:1312-1342) and the X0 conversion (:1489-1542), the latter
  fused with the Euler step in ``components.diffusion_steps``.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np
import torch

from ... import _lib
from ...kernels import gemm
from ...loader.weights import build_block, linear_weight
from .rope import AUDIO_MAX_POS, VIDEO_MAX_POS, rope_tables
from .timestep_embedding import SINUSOID_DIM, AdaLayerNormSingle
from .transformer import ADA_ROWS, BasicAVTransformerBlock, TransformerArgs, TransformerConfig

AUDIO_HEADS = 32
AUDIO_HEAD_DIM = 64
AUDIO_IN_CHANNELS = 128
AUDIO_CROSS_PE_MAX_POS = 20
# distinct position sets whose RoPE tables an LTXModel keeps (one 6144-token
# video set is ~100 MB of fp32 tables)
ROPE_CACHE_ENTRIES = 2


def _positions_digest(positions: np.ndarray) -> tuple:
    arr = np.ascontiguousarray(positions)
    return arr.shape, arr.dtype.str, hashlib.blake2b(arr.tobytes(), digest_size=16).hexdigest()


@dataclass
class Modality:
    """Input modality (model.py:103-118): patchified latent (B, T, 128),
    text context (B, S, D), context mask (B, S) -- boolean (True = attend)
    or additive -- or None, timesteps (B,) / (B, T) / a scalar, positions
    (B, n_dims, T, 2), and the prompt-AdaLN sigma (B,) or None (then the
    timesteps)."""

    latent: torch.Tensor
    context: torch.Tensor
    context_mask: torch.Tensor | None
    timesteps: torch.Tensor | float
    positions: np.ndarray
    enabled: bool = True
    sigma: torch.Tensor | float | None = None


# An additive context-mask value at or below this excludes its key: the
# softmax weight exp(s - m + v) of such a key underflows to exactly 0 in fp32
# for any score range the attention sees, as for the reference's boolean
# masks, which become -3.4e38 (model.py:208-250).
MASK_EXCLUDE = -1.0e4


def _uniform_value(t, what: str) -> float:
    """The one value of a scalar / (B,) / (B, T) timestep tensor; distinct
    values per sample or per token are not supported (the modulation rows of
    a forward are shared by all of its tokens)."""
    if isinstance(t, (int, float)):
        return float(t)
    v = torch.as_tensor(t).detach().float().reshape(-1).cpu()
    if v.numel() == 0:
        raise ValueError(f"empty {what}")
    if not bool((v == v[0]).all()):
        raise NotImplementedError(f"{what} differ across samples or tokens: one timestep per forward is "
                                  "supported (the text-to-video path's uniform denoise mask)")
    return float(v[0])


@dataclass
class TokenTimesteps:
    """Per-token timesteps of one sample as row groups: ``values`` the
    distinct timesteps (first-occurrence order), ``segments`` the maximal
    runs of rows [r0, r1) sharing group g, in row order."""

    values: list
    segments: list


def token_timestep_groups(t) -> TokenTimesteps:
    """Row groups of a (T,) per-token timestep vector (the image-conditioned
    denoise masks: timesteps = sigma * mask, model.py:160-187)."""
    v = torch.as_tensor(t).detach().float().reshape(-1).cpu().numpy()
    if v.size == 0:
        raise ValueError("empty per-token timesteps")
    values, index, segments = [], {}, []
    r0 = 0
    for r in range(1, v.size + 1):
        if r == v.size or v[r] != v[r0]:
            key = float(v[r0])
            if key not in index:
                index[key] = len(values)
                values.append(key)
            segments.append((r0, r, index[key]))
            r0 = r
    return TokenTimesteps(values, segments)


def context_keep_rows(mask: torch.Tensor | None, batch: int, length: int) -> list[torch.Tensor | None]:
    """Per sample, the context rows a (B, S) mask keeps (None: all of them).

    Boolean masks keep their True entries; additive float masks keep 0 and
    drop values <= MASK_EXCLUDE -- a dropped key's softmax weight is exactly 0,
    so attending over the kept rows only gives the masked attention's result
    (model.py:208-250 turns a boolean mask into -3.4e38 additive entries).
    Other additive values, masks that drop every key of a sample (the
    reference then spreads the weights uniformly) and (B, 1, S, S) masks are
    not supported."""
    if mask is None:
        return [None] * batch
    m = torch.as_tensor(mask)
    if m.dim() == 1:
        m = m[None]
    if m.dim() != 2 or m.shape[-1] != length or m.shape[0] not in (1, batch):
        raise NotImplementedError(f"context mask of shape {tuple(m.shape)}: (B, S) masks over the {length} "
                                  "context tokens are supported")
    m = m.detach().cpu()
    if m.dtype == torch.bool:
        keep = m
    elif m.is_floating_point():
        mf = m.float()
        if not bool(((mf == 0) | (mf <= MASK_EXCLUDE)).all()):
            raise NotImplementedError("additive context-mask values other than 0 and <= -1e4")
        keep = mf == 0
    else:
        keep = m != 0
    out = []
    for b in range(batch):
        row = keep[b if keep.shape[0] == batch else 0]
        n = int(row.sum())
        if n == 0:
            raise NotImplementedError(f"context mask of sample {b} excludes every key")
        out.append(None if n == length else torch.nonzero(row).reshape(-1))
    return out


class LTXModel:
    """LTX-2.3 AV transformer (model.py:497-1486): random-init weights, or
    ``init="empty"`` storage filled by ``loader.load_transformer_cache`` /
    ``loader.load_transformer_weights``."""

    def __init__(self, num_layers: int = 48, *, num_attention_heads: int = 32, attention_head_dim: int = 128,
                 in_channels: int = 128, out_channels: int = 128, cross_attention_dim: int = 4096,
                 norm_eps: float = 1e-6, timestep_scale_multiplier: float = 1000.0,
                 av_ca_timestep_scale_multiplier: float = 1000.0, weight_format: str = "bf16",
                 device: str | torch.device = "cuda", seed: int = 0, audio: bool = True, init: str = "random",
                 audio_attention_heads: int = AUDIO_HEADS, audio_attention_head_dim: int = AUDIO_HEAD_DIM):
        self.device = torch.device(device)
        self.num_layers = num_layers
        self.norm_eps = norm_eps
        self.timestep_scale_multiplier = timestep_scale_multiplier
        self.av_ca_timestep_scale_multiplier = av_ca_timestep_scale_multiplier
        self.weight_format = weight_format
        # audio stream work on its own HIP stream, overlapping the video stream
        self.concurrent_audio = True
        self._audio_stream: torch.cuda.Stream | None = None
        self.video_dim = num_attention_heads * attention_head_dim
        self.audio_dim = audio_attention_heads * audio_attention_head_dim
        self.video_config = TransformerConfig(self.video_dim, num_attention_heads, attention_head_dim,
                                              cross_attention_dim, True, True)
        self.audio_config = (TransformerConfig(self.audio_dim, audio_attention_heads, audio_attention_head_dim,
                                               self.audio_dim, True, True)
                             if audio else None)
        if init not in ("random", "empty"):
            raise ValueError(f"init must be 'random' or 'empty', got {init!r}")
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        dev = self.device
        vd, ad = self.video_dim, self.audio_dim
        lin = dict(gen=gen, device=dev, weight_format="bf16", init=init)
        mlp = dict(device=dev, generator=gen, init=init)

        def table(d):
            if init == "empty":
                return torch.zeros((2, d), device=dev)
            return (torch.randn((2, d), generator=gen, device=dev) * 0.02).contiguous()

        # preprocess / output heads (bf16 weights; small, kept unquantised)
        self.patchify_proj = linear_weight(vd, in_channels, **lin)
        self.adaln_single = AdaLayerNormSingle(vd, 9, **mlp)
        self.prompt_adaln_single = AdaLayerNormSingle(vd, 2, **mlp)
        self.av_ca_video_scale_shift_adaln_single = AdaLayerNormSingle(vd, 4, **mlp)
        self.av_ca_a2v_gate_adaln_single = AdaLayerNormSingle(vd, 1, **mlp)
        self.scale_shift_table = table(vd)
        self.proj_out = linear_weight(out_channels, vd, **lin)
        if audio:
            self.audio_patchify_proj = linear_weight(ad, AUDIO_IN_CHANNELS, **lin)
            self.audio_adaln_single = AdaLayerNormSingle(ad, 9, **mlp)
            self.audio_prompt_adaln_single = AdaLayerNormSingle(ad, 2, **mlp)
            self.av_ca_audio_scale_shift_adaln_single = AdaLayerNormSingle(ad, 4, **mlp)
            self.av_ca_v2a_gate_adaln_single = AdaLayerNormSingle(ad, 1, **mlp)
            self.audio_scale_shift_table = table(ad)
            self.audio_proj_out = linear_weight(out_channels, ad, **lin)

        # all blocks' modulation tables packed for the one-launch row update
        self.video_tables = torch.empty((num_layers, ADA_ROWS, vd), dtype=torch.float32, device=dev)
        self.audio_tables = (torch.empty((num_layers, ADA_ROWS, ad), dtype=torch.float32, device=dev)
                             if audio else None)
        self.transformer_blocks: list[BasicAVTransformerBlock] = []
        for i in range(num_layers):
            w = build_block(self.video_config, self.audio_config, device=dev, weight_format=weight_format,
                            generator=gen, norm_eps=norm_eps, video_tables=self.video_tables[i],
                            audio_tables=None if self.audio_tables is None else self.audio_tables[i], init=init)
            self.transformer_blocks.append(BasicAVTransformerBlock(i, self.video_config, self.audio_config,
                                                                   norm_eps=norm_eps, weights=w))
        # per-step buffers
        self._temb_v = torch.empty((ADA_ROWS, vd), device=dev)
        self._emb_v = torch.empty(vd, device=dev)
        self._ada_v = torch.empty_like(self.video_tables)
        if audio:
            self._temb_a = torch.empty((ADA_ROWS, ad), device=dev)
            self._emb_a = torch.empty(ad, device=dev)
            self._ada_a = torch.empty_like(self.audio_tables)
        self._rope_cache: dict = {}

    # ------------------------------------------------------------------------
    def weight_bytes(self) -> int:
        n = sum(b.nbytes() for b in self.transformer_blocks)
        mlps = [self.adaln_single, self.prompt_adaln_single, self.av_ca_video_scale_shift_adaln_single,
                self.av_ca_a2v_gate_adaln_single]
        if self.audio_config is not None:
            mlps += [self.audio_adaln_single, self.audio_prompt_adaln_single,
                     self.av_ca_audio_scale_shift_adaln_single, self.av_ca_v2a_gate_adaln_single]
        return n + sum(m.nbytes() for m in mlps)

    def rope(self, video_positions: np.ndarray, audio_positions: np.ndarray | None):
        """RoPE tables for a stage: (video self, video cross, audio self, audio
        cross), each token-major (cos, sin) or its factored (cos, sin, idx)
        form (``rope.factor_tables_np``; ``rope.expand_tables`` restores it).

        Tables are built once per distinct set of positions and reused across
        the steps of a stage.  The cache key is a digest of the full position
        arrays (shape, dtype and every byte), so two grids with the same token
        count but different layouts (landscape vs portrait) get their own
        tables; at most ``ROPE_CACHE_ENTRIES`` sets are kept, least recently
        used first out.  A caller that captured a graph over the returned
        tensors keeps them alive by holding the returned tuple.
        """
        key = (_positions_digest(video_positions), None if audio_positions is None
               else _positions_digest(audio_positions))
        hit = self._rope_cache.pop(key, None)
        if hit is None:
            dev = self.device
            # factored over the position axes where that is smaller (video:
            # a few rows per frame / row / column instead of one per token)
            vpe = rope_tables(video_positions, self.video_dim, VIDEO_MAX_POS, dev, factored=True)
            vxpe = ape = axpe = None
            if audio_positions is not None and self.audio_config is not None:
                # cross PE: temporal axis only, dim = audio inner dim (model.py:392-416)
                vxpe = rope_tables(video_positions[:, 0:1], self.audio_dim, (AUDIO_CROSS_PE_MAX_POS,), dev,
                                   factored=True)
                ape = rope_tables(audio_positions, self.audio_dim, AUDIO_MAX_POS, dev, factored=True)
                axpe = rope_tables(audio_positions[:, 0:1], self.audio_dim, (AUDIO_CROSS_PE_MAX_POS,), dev,
                                   factored=True)
            hit = (vpe, vxpe, ape, axpe)
        self._rope_cache[key] = hit  # re-inserted: most recently used last
        while len(self._rope_cache) > ROPE_CACHE_ENTRIES:
            self._rope_cache.pop(next(iter(self._rope_cache)))
        return hit

    def _mlps(self, video: bool) -> tuple:
        if video:
            return (self.adaln_single, self.prompt_adaln_single, self.av_ca_video_scale_shift_adaln_single,
                    self.av_ca_a2v_gate_adaln_single)
        return (self.audio_adaln_single, self.audio_prompt_adaln_single,
                self.av_ca_audio_scale_shift_adaln_single, self.av_ca_v2a_gate_adaln_single)

    def _timestep_rows(self, sigma_dev: torch.Tensor, cross_sigma_dev: torch.Tensor, video: bool,
                       prompt_sigma_dev: torch.Tensor | None = None) -> None:
        """Fill the (16, D) timestep rows of one modality (model.py:160-187,
        :305-314, :418-497) and its embedded timestep: the AdaLN rows 0-8 and
        the cross scale / shift rows 11-14 from the modality's timestep, the
        prompt rows 9-10 from its sigma (``prompt_sigma_dev``, default the
        timestep), the cross gate row 15 from the other modality's sigma."""
        d = self.video_dim if video else self.audio_dim
        temb = self._temb_v if video else self._temb_a
        emb = self._emb_v if video else self._emb_a
        ts = self.timestep_scale_multiplier
        mlps = self._mlps(video)
        flat = temb.view(-1)
        mlps[0](sigma_dev, ts, flat[: 9 * d], embedded=emb)
        mlps[1](sigma_dev if prompt_sigma_dev is None else prompt_sigma_dev, ts, flat[9 * d: 11 * d])
        if self.audio_config is not None:
            mlps[2](sigma_dev, ts, flat[11 * d: 15 * d])
            mlps[3](cross_sigma_dev, self.av_ca_timestep_scale_multiplier, flat[15 * d: 16 * d])
        else:
            flat[11 * d:].zero_()

    def _token_group_rows(self, groups: TokenTimesteps) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-token video timesteps as row groups: for each distinct value
        the (L, 16, D) modulation rows of every block and the embedded
        timestep, from the rows of the sample (``_temb_v``): rows 0-8 and
        11-14 and the embedded timestep follow the group's value, the prompt
        and cross gate rows stay the sample's (model.py:418-497)."""
        d, dev = self.video_dim, self.device
        mlps, ts = self._mlps(True), self.timestep_scale_multiplier
        g_n = len(groups.values)
        vals = torch.tensor(groups.values, dtype=torch.float32, device=dev)
        temb = self._temb_v.unsqueeze(0).repeat(g_n, 1, 1)
        emb = torch.empty((g_n, d), device=dev)
        ada = torch.empty((g_n,) + tuple(self._ada_v.shape), device=dev)
        stream = _lib.stream_of(ada)
        for g in range(g_n):
            flat = temb[g].view(-1)
            mlps[0](vals[g:g + 1], ts, flat[: 9 * d], embedded=emb[g])
            if self.audio_config is not None:
                mlps[2](vals[g:g + 1], ts, flat[11 * d: 15 * d])
            _lib.call("ltx_broadcast_add_f32", self.video_tables.data_ptr(), temb[g].data_ptr(), ada[g].data_ptr(),
                      self.num_layers, ADA_ROWS * d, stream)
        return ada, emb

    def velocity(self, video_latent: torch.Tensor, video_context: torch.Tensor, sigma_dev: torch.Tensor,
                 pes: tuple, audio_latent: torch.Tensor | None = None,
                 audio_context: torch.Tensor | None = None,
                 profile_events: list | None = None,
                 perturbations=None, passes: int = 1, sigmas: tuple | None = None,
                 video_token_timesteps: TokenTimesteps | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
        """One transformer forward -> (video velocity (T, 128), audio velocity).

        Latents are 2-D (T, 128) bf16; contexts (S, D) bf16; ``sigma_dev`` is
        the fp32 device scalar of this step's sigma.  ``perturbations`` (a
        ``BatchedPerturbationConfig``) skips attention sub-layers per block, the
        STG / modality-isolated passes (model.py:1044-1310 hands it to every
        block).

        ``passes`` > 1 runs that many passes of the same latents and timestep
        as one forward, their tokens stacked by rows (M = passes * T in every
        projection): contexts are then (passes, S, D) -- one per pass -- or a
        shared (S, D), ``perturbations`` holds one config per pass, and the
        velocities come back as (passes, T, 128).  The batched passes of a
        guided step (av_pipeline.py:688-717 runs them one after another).
        Latents of shape (B, T, 128) are B samples at one timestep, run the
        same way (passes = B), each on its own latents.

        ``sigmas`` = (video timestep, video sigma, audio timestep, audio
        sigma) fp32 device scalars when they differ (default: ``sigma_dev``
        for all): each modality's AdaLN and cross scale / shift rows follow
        its timestep, its prompt rows its sigma, its cross gate the other
        modality's sigma (model.py:418-497).  ``video_token_timesteps`` gives
        the video tokens per-token timesteps as row groups (one sample, no
        perturbations): the block's AdaLN inputs, gated residual adds and the
        output head then use each row group's modulation.
        """
        vpe, vxpe, ape, axpe = pes
        if video_latent.dim() == 3 and video_latent.shape[0] == 1:  # one sample: the 2-D form
            video_latent = video_latent[0]
            audio_latent = audio_latent[0] if audio_latent is not None and audio_latent.dim() == 3 else audio_latent
        if video_latent.dim() == 3:
            if passes not in (1, video_latent.shape[0]):
                raise ValueError(f"{video_latent.shape[0]} latent samples for {passes} passes")
            passes = video_latent.shape[0]
        run_audio = self.audio_config is not None and audio_latent is not None and audio_latent.shape[-2] > 0

        def stacked(x):  # (T, C) -> (passes, T, C)
            return x if passes == 1 else x.unsqueeze(0).expand(passes, *x.shape).contiguous()

        def project(latent, proj):  # (T, 128) shared by the passes, or (passes, T, 128)
            if latent.dim() == 3:
                return gemm.linear(latent.reshape(-1, latent.shape[-1]).contiguous(),
                                   proj).view(passes, latent.shape[1], -1)
            return stacked(gemm.linear(latent, proj))

        groups = video_token_timesteps
        if groups is not None and len(groups.values) < 2:
            sigmas = sigmas or (sigma_dev,) * 4
            val = torch.tensor(groups.values[:1], dtype=torch.float32, device=self.device)
            sigmas = (val,) + tuple(sigmas[1:])
            groups = None
        if groups is not None:
            if passes != 1 or video_latent.dim() != 2:
                raise NotImplementedError("per-token timesteps: one sample, unstacked")
            if groups.segments[-1][1] != video_latent.shape[0]:
                raise ValueError(f"per-token timesteps cover {groups.segments[-1][1]} rows, the latent has "
                                 f"{video_latent.shape[0]}")
        vt, vs, at, as_ = sigmas if sigmas is not None else (sigma_dev,) * 4

        # preprocess
        vx = project(video_latent, self.patchify_proj)
        self._timestep_rows(vt, as_, video=True, prompt_sigma_dev=vs)
        stream = _lib.stream_of(vx)
        _lib.call("ltx_broadcast_add_f32", self.video_tables.data_ptr(), self._temb_v.data_ptr(),
                  self._ada_v.data_ptr(), self.num_layers, ADA_ROWS * self.video_dim, stream)
        video = TransformerArgs(x=vx, context=video_context, timesteps=self._temb_v[:9], positional_embeddings=vpe,
                                cross_positional_embeddings=vxpe)
        audio = None
        if run_audio:
            ax = project(audio_latent, self.audio_patchify_proj)
            self._timestep_rows(at, vs, video=False, prompt_sigma_dev=as_)
            _lib.call("ltx_broadcast_add_f32", self.audio_tables.data_ptr(), self._temb_a.data_ptr(),
                      self._ada_a.data_ptr(), self.num_layers, ADA_ROWS * self.audio_dim, stream)
            audio = TransformerArgs(x=ax, context=audio_context, timesteps=self._temb_a[:9],
                                    positional_embeddings=ape, cross_positional_embeddings=axpe)
        # blocks; the audio stream's work overlaps the video stream's on a
        # second HIP stream (forked once here, joined before the heads)
        side = None
        if run_audio and self.concurrent_audio:
            if self._audio_stream is None:
                self._audio_stream = torch.cuda.Stream(device=vx.device)  # default priority
            side = self._audio_stream
        blocks = self.transformer_blocks
        ada_g = emb_g = None
        if groups is not None:
            ada_g, emb_g = self._token_group_rows(groups)
        for i, block in enumerate(blocks):
            block.ada_rows_video = self._ada_v[i] if groups is None else [ada_g[g, i] for g in range(len(groups.values))]
            block.segments_video = None if groups is None else groups.segments
            block.ada_rows_audio = self._ada_a[i] if run_audio else None
            block.audio_stream = side
            block.audio_fork = i == 0
            block.next_block = blocks[i + 1] if side is not None and i + 1 < len(blocks) else None
            block._prefetched_kv = None
        for block in blocks:
            video, audio = block(video, audio, perturbations=perturbations, profile_events=profile_events)
        if side is not None:
            torch.cuda.current_stream().wait_stream(side)
            audio.x.record_stream(torch.cuda.current_stream())
        # output heads
        def rows(x):
            return x.reshape(-1, x.shape[-1])

        def unstack(y):
            return y if passes == 1 else y.view(passes, -1, y.shape[-1])

        if groups is None:
            v_out = unstack(self._output(rows(video.x), self.scale_shift_table, self._emb_v, self.proj_out))
        else:
            vxr = rows(video.x)
            v_out = torch.empty((vxr.shape[0], self.proj_out.w.shape[0]), dtype=torch.bfloat16, device=vxr.device)
            for r0, r1, g in groups.segments:
                self._output(vxr[r0:r1], self.scale_shift_table, emb_g[g], self.proj_out, out=v_out[r0:r1])
        a_out = None
        if run_audio:
            a_out = unstack(self._output(rows(audio.x), self.audio_scale_shift_table, self._emb_a,
                                         self.audio_proj_out))
        return v_out, a_out

    def __call__(self, video: Modality | None = None, audio: Modality | None = None,
                 perturbations=None) -> tuple[torch.Tensor, torch.Tensor]:
        """The reference's forward on ``Modality`` inputs (model.py:1344-1486):
        (video velocity (B, T, 128), audio velocity (B, Ta, 128)); without an
        audio modality (or with ``enabled=False`` / no tokens) the audio
        velocity is an empty (B, 0, 128) tensor, as there.

        Covered: B >= 1 samples sharing their timesteps (each modality's
        timestep and sigma may differ, model.py:418-497), positions shared by
        the samples, and (B, S) context masks -- the masked keys are dropped
        from the context (``context_keep_rows``), which gives the masked
        softmax exactly.  The samples run as one forward (tokens stacked by
        rows) when their kept contexts have equal lengths, else one after
        another; ``perturbations`` holds one config per sample.  Per-token
        video timesteps (the image-conditioned denoise masks, (1, T)) run as
        row groups for one sample without perturbations; per-sample
        timesteps and per-token audio timesteps raise NotImplementedError.
        """
        if video is None:
            raise ValueError("Video modality required for video-enabled model")
        dev = self.device

        def as3(t, dtype=torch.bfloat16):
            t = torch.as_tensor(t)
            return (t[None] if t.dim() == 2 else t).to(device=dev, dtype=dtype)

        vlat, vctx = as3(video.latent), as3(video.context)
        batch = vlat.shape[0]
        if vctx.shape[0] not in (1, batch):
            raise ValueError(f"{vctx.shape[0]} video contexts for {batch} samples")
        use_audio = (audio is not None and audio.enabled and self.audio_config is not None
                     and torch.as_tensor(audio.latent).shape[-2] > 0)

        def sample_sigma(mod, what):
            # the prompt / cross-gate sigma: given, or the first token's
            # timestep (model.py:305-314, :459-461)
            if mod.sigma is not None:
                return _uniform_value(mod.sigma, f"{what} sigma")
            t = mod.timesteps
            if isinstance(t, (int, float)):
                return float(t)
            t = torch.as_tensor(t).detach().float().cpu()
            return _uniform_value(t.reshape(t.shape[0], -1)[:, 0] if t.dim() >= 2 else t, f"{what} sigma")

        groups = None
        tv_raw = video.timesteps
        if not isinstance(tv_raw, (int, float)) and torch.as_tensor(tv_raw).dim() == 2 and \
                torch.as_tensor(tv_raw).shape[1] == vlat.shape[1] and torch.as_tensor(tv_raw).shape[1] > 1:
            if batch == 1 and torch.as_tensor(tv_raw).shape[0] == 1:
                groups = token_timestep_groups(tv_raw)
                if len(groups.values) == 1:
                    groups = None
                elif perturbations is not None:
                    raise NotImplementedError("per-token timesteps with perturbations")
        vt = groups.values[0] if groups is not None else _uniform_value(tv_raw, "video timesteps")
        vs = sample_sigma(video, "video")
        alat = actx = None
        at, as_ = vt, vs
        if use_audio:
            alat, actx = as3(audio.latent), as3(audio.context)
            if alat.shape[0] != batch or actx.shape[0] not in (1, batch):
                raise ValueError("audio latents / contexts do not match the video samples")
            at = _uniform_value(audio.timesteps, "audio timesteps")
            as_ = sample_sigma(audio, "audio")
        sig4 = tuple(torch.tensor([x], dtype=torch.float32, device=dev) for x in (vt, vs, at, as_))
        sigma_dev = sig4[0]

        def shared_positions(pos, what):
            if pos is None:
                return None
            pos = pos.detach().cpu().numpy() if torch.is_tensor(pos) else np.asarray(pos)
            if pos.ndim >= 1 and pos.shape[0] > 1 and not all(np.array_equal(pos[0], p) for p in pos[1:]):
                raise NotImplementedError(f"{what} positions differ across samples")
            return pos[0:1] if pos.ndim >= 1 and pos.shape[0] > 1 else pos

        pes = self.rope(shared_positions(video.positions, "video"),
                        shared_positions(audio.positions, "audio") if use_audio else None)
        vkeep = context_keep_rows(video.context_mask, batch, vctx.shape[1])
        akeep = context_keep_rows(audio.context_mask, batch, actx.shape[1]) if use_audio else [None] * batch

        def ctx_of(ctx, keep, b):
            c = ctx[b if ctx.shape[0] == batch else 0]
            return c if keep[b] is None else c.index_select(0, keep[b].to(dev)).contiguous()

        vctxs = [ctx_of(vctx, vkeep, b) for b in range(batch)]
        actxs = [ctx_of(actx, akeep, b) for b in range(batch)] if use_audio else None
        same = len({c.shape[0] for c in vctxs}) == 1 and (not use_audio or len({c.shape[0] for c in actxs}) == 1)
        if batch == 1 or same:
            v, a = self.velocity(vlat if batch > 1 else vlat[0],
                                 torch.stack(vctxs) if batch > 1 else vctxs[0], sigma_dev, pes,
                                 (alat if batch > 1 else alat[0]) if use_audio else None,
                                 (torch.stack(actxs) if batch > 1 else actxs[0]) if use_audio else None,
                                 perturbations=perturbations, passes=batch, sigmas=sig4,
                                 video_token_timesteps=groups)
            v = v if batch > 1 else v[None]
            a = (a if batch > 1 else a[None]) if use_audio else None
        else:
            from ...components.perturbations import BatchedPerturbationConfig

            v_outs, a_outs = [], []
            for b in range(batch):
                pert = None
                if perturbations is not None:
                    pert = BatchedPerturbationConfig([perturbations.perturbations[b]])
                vb, ab = self.velocity(vlat[b], vctxs[b], sigma_dev, pes, alat[b] if use_audio else None,
                                       actxs[b] if use_audio else None, perturbations=pert, sigmas=sig4)
                v_outs.append(vb)
                a_outs.append(ab)
            v = torch.stack(v_outs)
            a = torch.stack(a_outs) if use_audio else None
        if a is None:
            a = torch.zeros((batch, 0, AUDIO_IN_CHANNELS), dtype=torch.bfloat16, device=dev)
        return v, a

    def _output(self, x: torch.Tensor, table: torch.Tensor, emb: torch.Tensor, proj: gemm.LinearWeight,
                out: torch.Tensor | None = None) -> torch.Tensor:
        t, d = x.shape
        h = torch.empty_like(x)
        _lib.call("ltx_output_norm_modulate_bf16", x.data_ptr(), d, table.data_ptr(), emb.data_ptr(), h.data_ptr(),
                  d, t, d, float(self.norm_eps), _lib.stream_of(x))
        return gemm.linear(h, proj, out=out)


class X0Model:
    """Denoised outputs instead of velocities (model.py:1489-1542):
    ``latent - timestep * velocity`` per modality in fp32, on the device
    (``ltx_x0_from_velocity_f32``); the video-only case returns the video
    prediction alone, as there."""

    def __init__(self, velocity_model: LTXModel):
        self.velocity_model = velocity_model

    def __call__(self, video: Modality | None = None, audio: Modality | None = None, perturbations=None):
        from ...components.diffusion_steps import to_denoised

        v, a = self.velocity_model(video, audio, perturbations=perturbations)
        dev = self.velocity_model.device

        def denoised(mod, vel):
            lat = torch.as_tensor(mod.latent)
            lat = (lat[None] if lat.dim() == 2 else lat).to(device=dev, dtype=torch.bfloat16).contiguous()
            vel = vel.contiguous()
            t = mod.timesteps
            if not isinstance(t, (int, float)) and torch.as_tensor(t).dim() == 2 and lat.shape[0] == 1 and \
                    torch.as_tensor(t).shape[1] == lat.shape[1]:
                # per-token timesteps: latent - t_token * velocity, per row group
                groups = token_timestep_groups(t)
                out = torch.empty(lat.shape, dtype=torch.float32, device=dev)
                for r0, r1, g in groups.segments:
                    out[0, r0:r1] = to_denoised(lat[0, r0:r1], vel[0, r0:r1], groups.values[g])
                return out
            return to_denoised(lat, vel, _uniform_value(t, "timesteps"))

        dv = denoised(video, v)
        if audio is None:
            return dv
        if a.shape[1] == 0:
            return dv, torch.zeros(a.shape, dtype=torch.float32, device=dev)
        return dv, denoised(audio, a)

