"""LTX-2.3 audio+video transformer block on gfx950 kernels.

Drop-in for ``BasicAVTransformerBlock`` (model/transformer/transformer.py:160-674):
same constructor arguments, same ``__call__(video, audio, perturbations=None,
profile_events=None) -> (video_args, audio_args)`` contract and the same
``TransformerArgs`` / ``TransformerConfig`` dataclasses (:113-157).  Tensors
are torch device tensors; batch size 1 (the T2V production shape).

Per-block data flow (rounding points follow the reference):
  1. video self-attn : AdaLN -> fused QKV+gate GEMM -> QK-norm+RoPE -> flash
     attention (gate fused) -> to_out GEMM with the gated residual add fused
     (fused_ops.py:345-348 / transformer.py:469).
  2. video text CA   : inline AdaLN (rms_norm rounded, :374), context
     modulation (:375), Q+gate / KV GEMMs, attention, to_out GEMM fused with
     ``vx + bf16(out*gate)`` (:387, :484).
  3. audio self-attn + text CA, same at D=2048.
  4. A2V / V2A       : shared bf16 rms_norm of vx/ax taken before A2V
     (:535-536), per-direction modulation (:579-580, :606-607), attention with
     temporal cross RoPE, to_out GEMM fused with the gated add (:598, :625).
  5. video / audio FF: AdaLN -> GEMM+GELU -> GEMM fused with the gated add.

The AdaLN modulation rows of a block are ``table + timestep embedding``
(:286-342).  They are packed per modality as 16 rows:
  0 shift_msa  1 scale_msa  2 gate_msa  3 shift_mlp  4 scale_mlp  5 gate_mlp
  6 shift_q    7 scale_q    8 gate_q    9 shift_kv  10 scale_kv
 11 scale_a2v 12 shift_a2v 13 scale_v2a 14 shift_v2a 15 gate (a2v for video,
 v2a for audio)
The 48-block scheduler computes all blocks' rows in one launch per step and
hands each block its slice (``ada_rows``); a block used on its own computes
its rows from its tables and the args' timestep fields.

With ``audio_stream`` set (the 48-block model sets it) and both streams
running, the audio stream's work (steps 3, the audio half of 4, and its FF) is
issued on that second HIP stream: the 68-token audio GEMMs and attentions use
a few CUs each and overlap with the video work.  The streams meet once per
block, at A2V / V2A: each direction waits for the other stream's modulated
inputs only (events), so the data flow and every rounding are unchanged.
"""

from __future__ import annotations

import contextlib
import os
import time
from collections.abc import Callable
from dataclasses import dataclass, replace as dc_replace

import torch

from ... import _lib
from ...kernels import fused_ops, gemm
from .attention import Attention
from .feed_forward import FeedForward
from ...components.perturbations import BatchedPerturbationConfig  # noqa: F401  (the block's perturbation type)
from .rope import LTXRopeType

# Dispatch shims (transformer.py:85-110): with LTX_FUSED_ADALN=1 the block's
# AdaLN uses the fused kernel's single rounding; by default the compiled
# inline form, whose rms_norm output is bf16 before the modulation.  Both run
# the same HIP kernel.  The gated residual add has one rounding either way.
_FUSED_ADALN_ENABLED = bool(os.environ.get("LTX_FUSED_ADALN"))
ADA_ROWS = 16
(ROW_SHIFT_MSA, ROW_SCALE_MSA, ROW_GATE_MSA, ROW_SHIFT_MLP, ROW_SCALE_MLP, ROW_GATE_MLP,
 ROW_SHIFT_Q, ROW_SCALE_Q, ROW_GATE_Q, ROW_SHIFT_KV, ROW_SCALE_KV,
 ROW_SCALE_A2V, ROW_SHIFT_A2V, ROW_SCALE_V2A, ROW_SHIFT_V2A, ROW_GATE_AV) = range(16)


@dataclass
class TransformerConfig:
    """Configuration for a transformer stream (transformer.py:113-122)."""

    dim: int
    heads: int
    d_head: int
    context_dim: int
    cross_attention_adaln: bool = False
    apply_gated_attention: bool = False


@dataclass
class TransformerArgs:
    """Arguments passed to transformer blocks (transformer.py:125-157).

    ``positional_embeddings`` / ``cross_positional_embeddings`` hold
    token-major (cos, sin) fp32 tables (T, D/2); reference-layout (1, H, T,
    dh/2) tables are accepted and converted.  ``timesteps`` is (B, 1, 9, D),
    ``prompt_timestep`` (B, 1, 2, D), ``cross_scale_shift_timestep`` (B, 1, 4,
    D) and ``cross_gate_timestep`` (B, 1, 1, D), all fp32.
    """

    x: torch.Tensor
    context: torch.Tensor
    timesteps: torch.Tensor
    positional_embeddings: tuple
    context_mask: torch.Tensor | None = None
    embedded_timestep: torch.Tensor | None = None
    cross_positional_embeddings: tuple | None = None
    cross_scale_shift_timestep: torch.Tensor | None = None
    cross_gate_timestep: torch.Tensor | None = None
    enabled: bool = True
    prompt_timestep: torch.Tensor | None = None

    def replace(self, **kwargs) -> "TransformerArgs":
        return dc_replace(self, **kwargs)


def _tables(pe):
    """Accept token-major (T, D/2) or reference (1, H, T, dh/2) tables."""
    if pe is None:
        return None
    cos, sin = pe
    if cos.dim() == 4:
        from ...kernels.rope_ops import tables_from_reference_layout

        return tables_from_reference_layout(cos, sin)
    return cos, sin


def adaln(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float, flags: int) -> torch.Tensor:
    """(T, C) bf16 -> new (T, C) bf16: AdaLN rows kernel (no gate, no fallback)."""
    t, c = x.shape
    xv, xs = _lib.row_view(x, c)
    out = torch.empty((t, c), dtype=torch.bfloat16, device=x.device)
    fused_ops.adaln_rows(xv, xs, scale, shift, out, c, t, c, eps, flags)
    return out


class BasicAVTransformerBlock:
    """Audio-video transformer block (transformer.py:160-674)."""

    def __init__(self, idx: int, video_config: TransformerConfig | None = None,
                 audio_config: TransformerConfig | None = None,
                 rope_type: LTXRopeType = LTXRopeType.SPLIT, norm_eps: float = 1e-6,
                 *, weights: dict | None = None, device: str | torch.device = "cuda",
                 weight_format: str = "bf16", generator: torch.Generator | None = None):
        from ...loader.weights import build_block

        self.idx = idx
        self.norm_eps = norm_eps
        self.rope_type = rope_type
        self.video_config = video_config
        self.audio_config = audio_config
        self.cross_attention_adaln = True
        if weights is None:
            weights = build_block(video_config, audio_config, device=device, weight_format=weight_format,
                                  generator=generator, norm_eps=norm_eps)
        self.attn1: Attention | None = weights.get("attn1")
        self.attn2: Attention | None = weights.get("attn2")
        self.ff: FeedForward | None = weights.get("ff")
        self.audio_attn1: Attention | None = weights.get("audio_attn1")
        self.audio_attn2: Attention | None = weights.get("audio_attn2")
        self.audio_ff: FeedForward | None = weights.get("audio_ff")
        self.audio_to_video_attn: Attention | None = weights.get("audio_to_video_attn")
        self.video_to_audio_attn: Attention | None = weights.get("video_to_audio_attn")
        # (16, D) fp32 tables: [scale_shift_table (9) | prompt table (2) | a2v_ca table (5)]
        self.video_tables: torch.Tensor | None = weights.get("video_tables")
        self.audio_tables: torch.Tensor | None = weights.get("audio_tables")
        # per-step modulation rows injected by the scheduler (see module doc)
        self.ada_rows_video: torch.Tensor | None = None
        self.ada_rows_audio: torch.Tensor | None = None
        self.audio_stream: torch.cuda.Stream | None = None
        self.audio_fork = True  # the audio stream waits for the caller's stream first
        self._adaln_flags = 0 if _FUSED_ADALN_ENABLED else _lib.ADALN_ROUND_NORM

    # -- parameters ---------------------------------------------------------
    def attentions(self) -> list[Attention]:
        return [a for a in (self.attn1, self.attn2, self.audio_attn1, self.audio_attn2,
                            self.audio_to_video_attn, self.video_to_audio_attn) if a is not None]

    def linear_weights(self) -> list[gemm.LinearWeight]:
        ws = [w for a in self.attentions() for w in a.weights()]
        for ff in (self.ff, self.audio_ff):
            if ff is not None:
                ws += ff.weights()
        return ws

    def nbytes(self) -> int:
        n = sum(w.nbytes() for w in self.linear_weights())
        for t in (self.video_tables, self.audio_tables):
            if t is not None:
                n += t.numel() * 4
        return n

    @staticmethod
    def temb_rows(args: TransformerArgs) -> torch.Tensor:
        """(16, D) timestep rows of one modality matching the table layout."""
        parts = [args.timesteps.reshape(-1, args.timesteps.shape[-1])[:9]]
        d = parts[0].shape[-1]
        for t, n in ((args.prompt_timestep, 2), (args.cross_scale_shift_timestep, 4), (args.cross_gate_timestep, 1)):
            parts.append(torch.zeros((n, d), device=parts[0].device) if t is None else t.reshape(-1, d)[:n].float())
        return torch.cat(parts, 0).contiguous()

    def _ada(self, args: TransformerArgs, tables: torch.Tensor, injected: torch.Tensor | None) -> torch.Tensor:
        if injected is not None:
            return injected
        temb = self.temb_rows(args)
        out = torch.empty_like(tables)
        _lib.call("ltx_broadcast_add_f32", tables.data_ptr(), temb.data_ptr(), out.data_ptr(), 1, tables.numel(),
                  _lib.stream_of(tables))
        return out

    # -- forward --------------------------------------------------------------
    def __call__(self, video: TransformerArgs | None, audio: TransformerArgs | None,
                 perturbations=None, profile_events: list | None = None) -> tuple:
        eps = self.norm_eps
        vx = video.x if video is not None else None
        ax = audio.x if audio is not None else None
        for x in (vx, ax):
            if x is not None and x.dim() == 3 and x.shape[0] != 1:
                raise NotImplementedError("batch size 1 only (the T2V hot path)")
        started = time.perf_counter()

        def mark(name: str) -> None:
            nonlocal started
            if profile_events is None:
                return
            torch.cuda.synchronize()
            now = time.perf_counter()
            profile_events.append((name, now - started))
            started = now

        run_vx = vx is not None and video.enabled and vx.numel() > 0
        run_ax = ax is not None and audio.enabled and ax.numel() > 0
        run_a2v = run_vx and ax is not None and ax.numel() > 0
        run_v2a = run_ax and vx is not None and vx.numel() > 0

        def skip(kind: str) -> bool:
            return perturbations is not None and perturbations.all_in_batch(kind, self.idx)

        flags = self._adaln_flags
        rn = _lib.ADALN_ROUND_NORM
        # 2-D working views; the first residual update of each stream writes a
        # fresh buffer so the caller's input tensors are never modified.
        v2 = vx[0] if (vx is not None and vx.dim() == 3) else vx
        a2 = ax[0] if (ax is not None and ax.dim() == 3) else ax
        v_owned = a_owned = False

        def residual_gemm(o, weight, stream_x, owned, gate, epi):
            out = stream_x if owned else torch.empty_like(stream_x)
            gemm.linear(o, weight, epilogue=epi, out=out, residual=stream_x, gate=gate)
            return out

        # A2V runs whenever video runs and audio tokens exist, even with the
        # audio stream disabled (transformer.py:426-427); it reads both tables.
        need_av = run_a2v or run_v2a
        ada_v = self._ada(video, self.video_tables, self.ada_rows_video) if run_vx or need_av else None
        ada_a = self._ada(audio, self.audio_tables, self.ada_rows_audio) if run_ax or need_av else None

        # Audio work on the second stream when both streams run.  Tensors that
        # cross streams are recorded on the consuming stream so the caching
        # allocator keeps them until that stream is done with them.
        side = self.audio_stream if (self.audio_stream is not None and run_vx and run_ax) else None
        main = torch.cuda.current_stream() if side is not None else None

        def on_audio():
            return torch.cuda.stream(side) if side is not None else contextlib.nullcontext()

        if side is not None:
            if self.audio_fork:  # audio input and modulation rows come from the caller's stream
                side.wait_stream(main)
            a2.record_stream(side)
            ada_a.record_stream(side)

        if run_vx:
            pe = _tables(video.positional_embeddings)
            if not skip("skip_video_self_attn"):
                h = adaln(v2, ada_v[ROW_SCALE_MSA], ada_v[ROW_SHIFT_MSA], eps, flags)
                o = self.attn1.core(h, pe=pe)
                v2 = residual_gemm(o, self.attn1.to_out, v2, v_owned, ada_v[ROW_GATE_MSA], gemm.EPI_RESIDUAL)
                v_owned = True
                mark("video self-attn")
            ctx = video.context[0] if video.context.dim() == 3 else video.context
            a = adaln(v2, ada_v[ROW_SCALE_Q], ada_v[ROW_SHIFT_Q], eps, rn)
            c = adaln(ctx, ada_v[ROW_SCALE_KV], ada_v[ROW_SHIFT_KV], eps, _lib.ADALN_NO_NORM)
            o = self.attn2.core(a, c)
            v2 = residual_gemm(o, self.attn2.to_out, v2, v_owned, ada_v[ROW_GATE_Q], gemm.EPI_RESIDUAL_ROUND)
            v_owned = True
            mark("video text-attn")

        if run_ax:
            with on_audio():
                pe = _tables(audio.positional_embeddings)
                if not skip("skip_audio_self_attn"):
                    h = adaln(a2, ada_a[ROW_SCALE_MSA], ada_a[ROW_SHIFT_MSA], eps, flags)
                    o = self.audio_attn1.core(h, pe=pe)
                    a2 = residual_gemm(o, self.audio_attn1.to_out, a2, a_owned, ada_a[ROW_GATE_MSA],
                                       gemm.EPI_RESIDUAL)
                    a_owned = True
                    mark("audio self-attn")
                ctx = audio.context[0] if audio.context.dim() == 3 else audio.context
                a = adaln(a2, ada_a[ROW_SCALE_Q], ada_a[ROW_SHIFT_Q], eps, rn)
                c = adaln(ctx, ada_a[ROW_SCALE_KV], ada_a[ROW_SHIFT_KV], eps, _lib.ADALN_NO_NORM)
                o = self.audio_attn2.core(a, c)
                a2 = residual_gemm(o, self.audio_attn2.to_out, a2, a_owned, ada_a[ROW_GATE_Q],
                                   gemm.EPI_RESIDUAL_ROUND)
                a_owned = True
                mark("audio text-attn")

        if run_a2v or run_v2a:
            vpe = _tables(video.cross_positional_embeddings)
            ape = _tables(audio.cross_positional_embeddings)
            # modulated inputs of both directions from the pre-A2V streams
            vs_a2v = adaln(v2, ada_v[ROW_SCALE_A2V], ada_v[ROW_SHIFT_A2V], eps, rn)
            vs_v2a = adaln(v2, ada_v[ROW_SCALE_V2A], ada_v[ROW_SHIFT_V2A], eps, rn)
            ev_v = main.record_event() if side is not None else None
            with on_audio():
                as_a2v = adaln(a2, ada_a[ROW_SCALE_A2V], ada_a[ROW_SHIFT_A2V], eps, rn)
                as_v2a = adaln(a2, ada_a[ROW_SCALE_V2A], ada_a[ROW_SHIFT_V2A], eps, rn)
            if side is not None:
                main.wait_event(side.record_event())
                as_a2v.record_stream(main)
                vs_v2a.record_stream(side)
            if run_a2v and not skip("skip_a2v_cross_attn"):
                o = self.audio_to_video_attn.core(vs_a2v, as_a2v, pe=vpe, k_pe=ape)
                v2 = residual_gemm(o, self.audio_to_video_attn.to_out, v2, v_owned, ada_v[ROW_GATE_AV],
                                   gemm.EPI_RESIDUAL)
                v_owned = True
                mark("audio->video attn")
            if run_v2a and not skip("skip_v2a_cross_attn"):
                with on_audio():
                    if side is not None:
                        side.wait_event(ev_v)
                    o = self.video_to_audio_attn.core(as_v2a, vs_v2a, pe=ape, k_pe=vpe)
                    a2 = residual_gemm(o, self.video_to_audio_attn.to_out, a2, a_owned, ada_a[ROW_GATE_AV],
                                       gemm.EPI_RESIDUAL)
                    a_owned = True
                    mark("video->audio attn")

        if run_vx:
            h = adaln(v2, ada_v[ROW_SCALE_MLP], ada_v[ROW_SHIFT_MLP], eps, flags)
            f = self.ff.hidden(h)
            v2 = residual_gemm(f, self.ff.project_out, v2, v_owned, ada_v[ROW_GATE_MLP], gemm.EPI_RESIDUAL)
            mark("video ff")
        if run_ax:
            with on_audio():
                h = adaln(a2, ada_a[ROW_SCALE_MLP], ada_a[ROW_SHIFT_MLP], eps, flags)
                f = self.audio_ff.hidden(h)
                a2 = residual_gemm(f, self.audio_ff.project_out, a2, a_owned, ada_a[ROW_GATE_MLP],
                                   gemm.EPI_RESIDUAL)
                mark("audio ff")

        def pack(args, x2, x_in, owned):
            if args is None or not owned:
                return args
            return args.replace(x=x2[None] if x_in.dim() == 3 else x2)

        return pack(video, v2, vx, v_owned), pack(audio, a2, ax, a_owned)


ProfileHook = Callable[[str], None]
