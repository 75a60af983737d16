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
from ...utils import signpost as _sp
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
    token-major (cos, sin) fp32 tables (T, D/2) or their factored (cos, sin,
    idx) form (``rope.factor_tables_np``); reference-layout (1, H, T, dh/2)
    tables are accepted and converted.  ``timesteps`` is (B, 1, 9, D),
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
    """Accept token-major (T, D/2) tables, their factored (cos, sin, idx) form
    or reference (1, H, T, dh/2) tables."""
    if pe is None or len(pe) == 3:
        return pe
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


def adaln_groups(x: torch.Tensor, groups: list, segments: list, row_scale: int, row_shift: int, eps: float,
                 flags: int) -> torch.Tensor:
    """AdaLN with per-token modulation as row groups: rows [r0, r1) of each
    segment take group g's (16, D) modulation rows."""
    t, c = x.shape
    out = torch.empty((t, c), dtype=torch.bfloat16, device=x.device)
    for r0, r1, g in segments:
        xv, xs = _lib.row_view(x[r0:r1], c)
        fused_ops.adaln_rows(xv, xs, groups[g][row_scale], groups[g][row_shift], out[r0:r1], c, r1 - r0, c, eps,
                             flags)
    return out


def adaln2_groups(x: torch.Tensor, groups: list, segments: list, rows: tuple, eps: float,
                  flags: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``adaln2`` with per-token modulation as row groups (rows = the
    (scale, shift, scale2, shift2) row indices)."""
    t, c = x.shape
    out = torch.empty((t, c), dtype=torch.bfloat16, device=x.device)
    out2 = torch.empty((t, c), dtype=torch.bfloat16, device=x.device)
    for r0, r1, g in segments:
        xv, xs = _lib.row_view(x[r0:r1], c)
        a = groups[g]
        fused_ops.adaln_rows2(xv, xs, a[rows[0]], a[rows[1]], out[r0:r1], a[rows[2]], a[rows[3]], out2[r0:r1],
                              r1 - r0, c, eps, flags)
    return out, out2


def adaln2(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, scale2: torch.Tensor, shift2: torch.Tensor,
           eps: float, flags: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Two AdaLN modulations of the same rows (one read of x, one norm)."""
    t, c = x.shape
    xv, xs = _lib.row_view(x, c)
    out = torch.empty((t, c), dtype=torch.bfloat16, device=x.device)
    out2 = torch.empty((t, c), dtype=torch.bfloat16, device=x.device)
    fused_ops.adaln_rows2(xv, xs, scale, shift, out, scale2, shift2, out2, t, c, eps, flags)
    return out, out2


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
        self.ada_rows_video: torch.Tensor | list | None = None
        self.ada_rows_audio: torch.Tensor | None = None
        # per-token video timesteps: ada_rows_video is then a list of (16, D)
        # row groups and segments_video the (r0, r1, group) row runs
        self.segments_video: list | None = None
        self.audio_stream: torch.cuda.Stream | None = None
        self.audio_fork = True  # the audio stream waits for the caller's stream first
        # The next block of the same forward (set by the scheduler): its text
        # keys / values are computed on the audio stream during this block,
        # ahead of this block's A2V event, so that event also covers them.
        self.next_block: "BasicAVTransformerBlock | None" = None
        self._prefetched_kv: tuple | None = None
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
        """One block on P stacked passes.  ``x`` is (T, C) for one pass or
        (P, T, C) for P passes (the batched passes of a guided step: same
        latents and timestep, their own text contexts and perturbations);
        ``context`` is (S, D) / (1, S, D) shared by every pass, or (P, S, D).
        ``perturbations`` holds one config per pass (or one for all): a pass
        whose sub-layer is skipped keeps its rows unchanged there, like the
        reference's per-sample mask (transformer.py:425-465)."""
        eps = self.norm_eps
        vx = video.x if video is not None else None
        ax = audio.x if audio is not None else None
        npass = 1
        for x in (vx, ax):
            if x is not None and x.dim() == 3 and x.shape[0] != 1:
                npass = x.shape[0]
        for x in (vx, ax):
            if x is not None and x.dim() == 3 and x.shape[0] not in (1, npass):
                raise ValueError(f"video and audio pass counts differ ({vx.shape[0]} vs {ax.shape[0]})")
            if x is not None and x.dim() == 2 and npass > 1:
                raise ValueError("stacked passes need (P, T, C) inputs for both modalities")
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

        def keep(kind: str) -> list[bool]:
            """Per pass: does the sub-layer run?"""
            if perturbations is None:
                return [True] * npass
            m = perturbations.mask(kind, self.idx)
            if len(m) == 1:
                m = m * npass
            if len(m) != npass:
                raise ValueError(f"{len(m)} perturbation configs for {npass} passes")
            return [v != 0.0 for v in m]

        def runs(mask: list[bool]) -> list[tuple[int, int]]:
            """Maximal ranges [p0, p1) of consecutive running passes."""
            out, p = [], 0
            while p < npass:
                if mask[p]:
                    q = p
                    while q < npass and mask[q]:
                        q += 1
                    out.append((p, q))
                    p = q
                else:
                    p += 1
            return out

        flags = self._adaln_flags
        rn = _lib.ADALN_ROUND_NORM
        # 2-D working views (passes stacked by rows); the first residual update
        # of each stream writes a fresh buffer so the caller's input tensors are
        # never modified.
        v2 = vx.reshape(-1, vx.shape[-1]) if (vx is not None and vx.dim() == 3) else vx
        a2 = ax.reshape(-1, ax.shape[-1]) if (ax is not None and ax.dim() == 3) else ax
        tv = v2.shape[0] // npass if v2 is not None else 0
        ta = a2.shape[0] // npass if a2 is not None else 0
        v_owned = a_owned = False

        def residual_gemm(o, weight, stream_x, owned, gate, epi, phase="attn_out"):
            out = stream_x if owned else torch.empty_like(stream_x)
            _sp.begin(phase)
            gemm.linear(o, weight, epilogue=epi, out=out, residual=stream_x, gate=gate)
            _sp.end(phase)
            return out

        def partial_residual(x2, owned, t, rng, sublayer):
            """Run ``sublayer(dst, src, p0, p1) -> None`` (dst = src + the
            sub-layer's gated branch; dst may be src) on the passes of each
            range of ``rng``; the other passes' rows stay as they are (copied
            once into a fresh stream when the input is not owned).  Returns the
            (owned) stream."""
            out = x2 if owned else torch.empty_like(x2)
            p = 0
            for p0, p1 in rng + [(npass, npass)]:
                if not owned and p0 > p:
                    out[p * t:p0 * t].copy_(x2[p * t:p0 * t])
                if p1 > p0:
                    sublayer(out[p0 * t:p1 * t], x2[p0 * t:p1 * t], p0, p1)
                p = p1
            return out

        def ctx_rows(args, p0, p1):
            """Text-context rows of passes [p0, p1): per-pass contexts are
            stacked (P, S, D); a shared (S, D) context serves every pass."""
            c = args.context
            if c.dim() == 3 and c.shape[0] == npass and npass > 1:
                return c[p0:p1].reshape(-1, c.shape[-1]), p1 - p0
            c2 = c[0] if c.dim() == 3 else c
            return c2, 1

        # A2V runs whenever video runs and audio tokens exist, even with the
        # audio stream disabled (transformer.py:426-427); it reads both tables.
        need_av = run_a2v or run_v2a
        ada_v = self._ada(video, self.video_tables, self.ada_rows_video) if run_vx or need_av else None
        ada_a = self._ada(audio, self.audio_tables, self.ada_rows_audio) if run_ax or need_av else None
        # per-token video timesteps (row groups): the AdaLN inputs and gated
        # residual adds of the video stream use each row group's rows; the
        # prompt rows and the cross gate are the same in every group
        v_groups = v_segs = None
        if isinstance(ada_v, list):
            if npass != 1 or perturbations is not None or not self.segments_video:
                raise NotImplementedError("per-token timesteps: one unperturbed pass with row segments")
            v_groups, v_segs, ada_v = ada_v, self.segments_video, ada_v[0]

        def v_adaln(x, row_scale, row_shift, fl):
            if v_groups is None:
                return adaln(x, ada_v[row_scale], ada_v[row_shift], eps, fl)
            return adaln_groups(x, v_groups, v_segs, row_scale, row_shift, eps, fl)

        def v_residual(o, weight, stream_x, owned, row_gate, epi, phase="attn_out"):
            if v_groups is None:
                return residual_gemm(o, weight, stream_x, owned, ada_v[row_gate], epi, phase=phase)
            out = stream_x if owned else torch.empty_like(stream_x)
            _sp.begin(phase)
            for r0, r1, g in v_segs:
                gemm.linear(o[r0:r1], weight, epilogue=epi, out=out[r0:r1], residual=stream_x[r0:r1],
                            gate=v_groups[g][row_gate])
            _sp.end(phase)
            return out

        # Audio work on the second stream when both streams run.  Tensors that
        # cross streams are recorded on the consuming stream so the caching
        # allocator keeps them until that stream is done with them.
        side = self.audio_stream if (self.audio_stream is not None and run_vx and run_ax) else None
        main = torch.cuda.current_stream() if side is not None else None

        def on_audio():
            return torch.cuda.stream(side) if side is not None else contextlib.nullcontext()

        # The audio stream's first kernel of a forked block must depend on the
        # caller's stream as it is now, but be issued only after the video
        # stream's first kernel: a HIP graph replay keeps the first-issued
        # child of a fork on the parent's queue and moves the others to
        # queues it shares with later branches, where the video kernels would
        # wait behind audio work.
        ev_fork = main.record_event() if side is not None and self.audio_fork else None

        def fork_side():
            nonlocal ev_fork
            if ev_fork is not None:
                side.wait_event(ev_fork)
                ev_fork = None

        if side is not None:
            a2.record_stream(side)
            ada_a.record_stream(side)
            for t in (v_groups or []) + ([ada_v] if ada_v is not None else []):
                t.record_stream(side)

        ev_kv = kv_v = None
        prefetched, self._prefetched_kv = self._prefetched_kv, None

        def context_kv_on_side():
            # the text context's keys and values do not depend on the video
            # rows: computed on the audio stream while the video self-attention
            # runs, off the video stream's path.  The previous block of the
            # forward computed this block's before its A2V event, which the
            # video stream has waited for already; otherwise they are made
            # here and joined by their own event.  The next block's are made
            # right after, ahead of this block's A2V event.
            nonlocal ev_kv, kv_v
            with on_audio():
                fork_side()
                c, cp = ctx_rows(video, 0, npass)
                if prefetched is not None:
                    kv_v = prefetched
                else:
                    cm = adaln(c, ada_v[ROW_SCALE_KV], ada_v[ROW_SHIFT_KV], eps, _lib.ADALN_NO_NORM)
                    kv_v = (self.attn2.context_kv(cm), cp)
                    ev_kv = side.record_event()
                    kv_v[0].record_stream(main)
                nb = self.next_block
                if nb is not None and nb.attn2 is not None and nb.ada_rows_video is not None and \
                        (run_a2v or run_v2a):
                    ada_n = nb.ada_rows_video
                    ada_n = ada_n[0] if isinstance(ada_n, list) else ada_n  # prompt rows: every group's
                    cm = adaln(c, ada_n[ROW_SCALE_KV], ada_n[ROW_SHIFT_KV], eps, _lib.ADALN_NO_NORM)
                    nb._prefetched_kv = (nb.attn2.context_kv(cm), cp)
                    nb._prefetched_kv[0].record_stream(main)

        if run_vx:
            _sp.begin("video_self_attn")
            pe = _tables(video.positional_embeddings)
            rng = runs(keep("skip_video_self_attn"))
            if rng == [(0, npass)]:
                h = v_adaln(v2, ROW_SCALE_MSA, ROW_SHIFT_MSA, flags)
                if side is not None:
                    context_kv_on_side()
                o = self.attn1.core(h, pe=pe, passes=npass)
                v2 = v_residual(o, self.attn1.to_out, v2, v_owned, ROW_GATE_MSA, gemm.EPI_RESIDUAL)
                v_owned = True
            elif rng:
                def video_self(dst, src, p0, p1):
                    h = adaln(src, ada_v[ROW_SCALE_MSA], ada_v[ROW_SHIFT_MSA], eps, flags)
                    o = self.attn1.core(h, pe=pe, passes=p1 - p0)
                    gemm.linear(o, self.attn1.to_out, epilogue=gemm.EPI_RESIDUAL, out=dst, residual=src,
                                gate=ada_v[ROW_GATE_MSA])
                v2 = partial_residual(v2, v_owned, tv, rng, video_self)
                v_owned = True
            _sp.signpost_barrier(v2)
            _sp.end("video_self_attn")
            mark("video self-attn")
            _sp.begin("video_text_ca")
            if side is not None and kv_v is None:
                context_kv_on_side()
            a = v_adaln(v2, ROW_SCALE_Q, ROW_SHIFT_Q, rn)
            if kv_v is not None:
                kv, cp = kv_v
                if cp == npass:
                    o = self.attn2.core(a, kv=kv, passes=npass, kv_ready=ev_kv)
                else:
                    o = torch.cat([self.attn2.core(a[p * tv:(p + 1) * tv], kv=kv, kv_ready=ev_kv)
                                   for p in range(npass)], 0) if npass > 1 else \
                        self.attn2.core(a, kv=kv, kv_ready=ev_kv)
            else:
                c, cp = ctx_rows(video, 0, npass)
                c = adaln(c, ada_v[ROW_SCALE_KV], ada_v[ROW_SHIFT_KV], eps, _lib.ADALN_NO_NORM)
                if cp == npass:
                    o = self.attn2.core(a, c, passes=npass)
                else:
                    o = torch.cat([self.attn2.core(a[p * tv:(p + 1) * tv], c) for p in range(npass)], 0) \
                        if npass > 1 else self.attn2.core(a, c)
            v2 = v_residual(o, self.attn2.to_out, v2, v_owned, ROW_GATE_Q, gemm.EPI_RESIDUAL_ROUND)
            v_owned = True
            _sp.signpost_barrier(v2)
            _sp.end("video_text_ca")
            mark("video text-attn")

        if run_ax:
            with on_audio():
                fork_side()
                _sp.begin("audio_self_attn")
                pe = _tables(audio.positional_embeddings)
                rng = runs(keep("skip_audio_self_attn"))
                if rng == [(0, npass)]:
                    h = adaln(a2, ada_a[ROW_SCALE_MSA], ada_a[ROW_SHIFT_MSA], eps, flags)
                    o = self.audio_attn1.core(h, pe=pe, passes=npass)
                    a2 = residual_gemm(o, self.audio_attn1.to_out, a2, a_owned, ada_a[ROW_GATE_MSA],
                                       gemm.EPI_RESIDUAL)
                    a_owned = True
                elif rng:
                    def audio_self(dst, src, p0, p1):
                        h = adaln(src, ada_a[ROW_SCALE_MSA], ada_a[ROW_SHIFT_MSA], eps, flags)
                        o = self.audio_attn1.core(h, pe=pe, passes=p1 - p0)
                        gemm.linear(o, self.audio_attn1.to_out, epilogue=gemm.EPI_RESIDUAL, out=dst, residual=src,
                                    gate=ada_a[ROW_GATE_MSA])
                    a2 = partial_residual(a2, a_owned, ta, rng, audio_self)
                    a_owned = True
                _sp.signpost_barrier(a2)
                _sp.end("audio_self_attn")
                mark("audio self-attn")
                _sp.begin("audio_text_ca")
                a = adaln(a2, ada_a[ROW_SCALE_Q], ada_a[ROW_SHIFT_Q], eps, rn)
                c, cp = ctx_rows(audio, 0, npass)
                c = adaln(c, ada_a[ROW_SCALE_KV], ada_a[ROW_SHIFT_KV], eps, _lib.ADALN_NO_NORM)
                if cp == npass:
                    o = self.audio_attn2.core(a, c, passes=npass)
                else:
                    o = torch.cat([self.audio_attn2.core(a[p * ta:(p + 1) * ta], c) for p in range(npass)], 0) \
                        if npass > 1 else self.audio_attn2.core(a, c)
                a2 = residual_gemm(o, self.audio_attn2.to_out, a2, a_owned, ada_a[ROW_GATE_Q],
                                   gemm.EPI_RESIDUAL_ROUND)
                a_owned = True
                _sp.signpost_barrier(a2)
                _sp.end("audio_text_ca")
                mark("audio text-attn")

        if run_a2v or run_v2a:
            _sp.begin("a2v_cross")
            vpe = _tables(video.cross_positional_embeddings)
            ape = _tables(audio.cross_positional_embeddings)
            # modulated inputs of both directions from the pre-A2V streams
            if v_groups is None:
                vs_a2v, vs_v2a = adaln2(v2, ada_v[ROW_SCALE_A2V], ada_v[ROW_SHIFT_A2V], ada_v[ROW_SCALE_V2A],
                                        ada_v[ROW_SHIFT_V2A], eps, rn)
            else:
                vs_a2v, vs_v2a = adaln2_groups(v2, v_groups, v_segs, (ROW_SCALE_A2V, ROW_SHIFT_A2V, ROW_SCALE_V2A,
                                                                      ROW_SHIFT_V2A), eps, rn)
            ev_v = main.record_event() if side is not None else None
            rng = runs(keep("skip_a2v_cross_attn")) if run_a2v else []
            kv_a2v = None
            with on_audio():
                as_a2v, as_v2a = adaln2(a2, ada_a[ROW_SCALE_A2V], ada_a[ROW_SHIFT_A2V], ada_a[ROW_SCALE_V2A],
                                        ada_a[ROW_SHIFT_V2A], eps, rn)
                if side is not None and rng == [(0, npass)]:
                    # A2V keys / values from the audio rows, on the audio stream
                    kv_a2v = self.audio_to_video_attn.context_kv(as_a2v, k_pe=ape, passes=npass)
            ev_a = None
            if side is not None:
                ev_a = side.record_event()
                vs_v2a.record_stream(side)
                if kv_a2v is not None:
                    kv_a2v.record_stream(main)
                else:
                    main.wait_event(ev_a)
                    as_a2v.record_stream(main)
            if rng == [(0, npass)]:
                if kv_a2v is not None:
                    o = self.audio_to_video_attn.core(vs_a2v, pe=vpe, passes=npass, kv=kv_a2v, kv_ready=ev_a)
                else:
                    o = self.audio_to_video_attn.core(vs_a2v, as_a2v, pe=vpe, k_pe=ape, passes=npass)
                v2 = residual_gemm(o, self.audio_to_video_attn.to_out, v2, v_owned, ada_v[ROW_GATE_AV],
                                   gemm.EPI_RESIDUAL)
                v_owned = True
            elif rng:
                def a2v(dst, src, p0, p1):
                    o = self.audio_to_video_attn.core(vs_a2v[p0 * tv:p1 * tv], as_a2v[p0 * ta:p1 * ta], pe=vpe,
                                                      k_pe=ape, passes=p1 - p0)
                    gemm.linear(o, self.audio_to_video_attn.to_out, epilogue=gemm.EPI_RESIDUAL, out=dst,
                                residual=src, gate=ada_v[ROW_GATE_AV])
                v2 = partial_residual(v2, v_owned, tv, rng, a2v)
                v_owned = True
            _sp.signpost_barrier(v2)
            _sp.end("a2v_cross")
            if run_a2v:
                mark("audio->video attn")
            _sp.begin("v2a_cross")
            rng = runs(keep("skip_v2a_cross_attn")) if run_v2a else []
            if rng:
                with on_audio():
                    if side is not None:
                        side.wait_event(ev_v)
                    if rng == [(0, npass)]:
                        o = self.video_to_audio_attn.core(as_v2a, vs_v2a, pe=ape, k_pe=vpe, passes=npass)
                        a2 = residual_gemm(o, self.video_to_audio_attn.to_out, a2, a_owned, ada_a[ROW_GATE_AV],
                                           gemm.EPI_RESIDUAL)
                    else:
                        def v2a(dst, src, p0, p1):
                            o = self.video_to_audio_attn.core(as_v2a[p0 * ta:p1 * ta], vs_v2a[p0 * tv:p1 * tv],
                                                              pe=ape, k_pe=vpe, passes=p1 - p0)
                            gemm.linear(o, self.video_to_audio_attn.to_out, epilogue=gemm.EPI_RESIDUAL, out=dst,
                                        residual=src, gate=ada_a[ROW_GATE_AV])
                        a2 = partial_residual(a2, a_owned, ta, rng, v2a)
                    a_owned = True
                    mark("video->audio attn")
            _sp.signpost_barrier(a2)
            _sp.end("v2a_cross")

        if run_vx:
            _sp.begin("video_ff")
            _sp.begin("v_ff_adaln")
            h = v_adaln(v2, ROW_SCALE_MLP, ROW_SHIFT_MLP, flags)
            _sp.end("v_ff_adaln")
            _sp.begin("v_ff_inner")
            f = self.ff.hidden(h)
            v2 = v_residual(f, self.ff.project_out, v2, v_owned, ROW_GATE_MLP, gemm.EPI_RESIDUAL, phase=None)
            _sp.end("v_ff_inner")
            _sp.signpost_barrier(v2)
            _sp.end("video_ff")
            mark("video ff")
        if run_ax:
            with on_audio():
                _sp.begin("audio_ff")
                h = adaln(a2, ada_a[ROW_SCALE_MLP], ada_a[ROW_SHIFT_MLP], eps, flags)
                f = self.audio_ff.hidden(h)
                a2 = residual_gemm(f, self.audio_ff.project_out, a2, a_owned, ada_a[ROW_GATE_MLP],
                                   gemm.EPI_RESIDUAL, phase=None)
                _sp.signpost_barrier(a2)
                _sp.end("audio_ff")
                mark("audio ff")

        def pack(args, x2, x_in, owned):
            if args is None or not owned:
                return args
            return args.replace(x=x2.reshape(x_in.shape) if x_in.dim() == 3 else x2)

        return pack(video, v2, vx, v_owned), pack(audio, a2, ax, a_owned)


ProfileHook = Callable[[str], None]
