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
    """Input modality (model.py:103-118): patchified latent (B, T, 128) bf16,
    text context (B, S, D) bf16, scalar sigma, positions (B, n_dims, T, 2)."""

    latent: torch.Tensor
    context: torch.Tensor
    sigma: float
    positions: np.ndarray
    enabled: bool = True
    context_mask: torch.Tensor | None = None


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

    def _timestep_rows(self, sigma_dev: torch.Tensor, cross_sigma_dev: torch.Tensor, video: bool) -> None:
        """Fill the (16, D) timestep rows of one modality (model.py:160-187,
        :305-314, :418-497) and its embedded timestep."""
        d = self.video_dim if video else self.audio_dim
        temb = self._temb_v if video else self._temb_a
        emb = self._emb_v if video else self._emb_a
        ts = self.timestep_scale_multiplier
        if video:
            mlps = (self.adaln_single, self.prompt_adaln_single, self.av_ca_video_scale_shift_adaln_single,
                    self.av_ca_a2v_gate_adaln_single)
        else:
            mlps = (self.audio_adaln_single, self.audio_prompt_adaln_single,
                    self.av_ca_audio_scale_shift_adaln_single, self.av_ca_v2a_gate_adaln_single)
        flat = temb.view(-1)
        mlps[0](sigma_dev, ts, flat[: 9 * d], embedded=emb)
        mlps[1](sigma_dev, ts, flat[9 * d: 11 * d])
        if self.audio_config is not None:
            mlps[2](sigma_dev, ts, flat[11 * d: 15 * d])
            mlps[3](cross_sigma_dev, self.av_ca_timestep_scale_multiplier, flat[15 * d: 16 * d])
        else:
            flat[11 * d:].zero_()

    def velocity(self, video_latent: torch.Tensor, video_context: torch.Tensor, sigma_dev: torch.Tensor,
                 pes: tuple, audio_latent: torch.Tensor | None = None,
                 audio_context: torch.Tensor | None = None,
                 profile_events: list | None = None,
                 perturbations=None, passes: int = 1) -> tuple[torch.Tensor, torch.Tensor | None]:
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
        """
        vpe, vxpe, ape, axpe = pes
        run_audio = self.audio_config is not None and audio_latent is not None and audio_latent.shape[0] > 0

        def stacked(x):  # (T, C) -> (passes, T, C)
            return x if passes == 1 else x.unsqueeze(0).expand(passes, *x.shape).contiguous()

        # preprocess
        vx = stacked(gemm.linear(video_latent, self.patchify_proj))
        self._timestep_rows(sigma_dev, sigma_dev, video=True)
        stream = _lib.stream_of(vx)
        _lib.call("ltx_broadcast_add_f32", self.video_tables.data_ptr(), self._temb_v.data_ptr(),
                  self._ada_v.data_ptr(), self.num_layers, ADA_ROWS * self.video_dim, stream)
        video = TransformerArgs(x=vx, context=video_context, timesteps=self._temb_v[:9], positional_embeddings=vpe,
                                cross_positional_embeddings=vxpe)
        audio = None
        if run_audio:
            ax = stacked(gemm.linear(audio_latent, self.audio_patchify_proj))
            self._timestep_rows(sigma_dev, sigma_dev, video=False)
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
        for i, block in enumerate(blocks):
            block.ada_rows_video = self._ada_v[i]
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

        v_out = unstack(self._output(rows(video.x), self.scale_shift_table, self._emb_v, self.proj_out))
        a_out = None
        if run_audio:
            a_out = unstack(self._output(rows(audio.x), self.audio_scale_shift_table, self._emb_a,
                                         self.audio_proj_out))
        return v_out, a_out

    def _output(self, x: torch.Tensor, table: torch.Tensor, emb: torch.Tensor, proj: gemm.LinearWeight) -> torch.Tensor:
        t, d = x.shape
        h = torch.empty_like(x)
        _lib.call("ltx_output_norm_modulate_bf16", x.data_ptr(), d, table.data_ptr(), emb.data_ptr(), h.data_ptr(),
                  d, t, d, float(self.norm_eps), _lib.stream_of(x))
        return gemm.linear(h, proj)
