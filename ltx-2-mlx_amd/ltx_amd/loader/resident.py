"""Named transformer weights -> the resident fused layout in HBM.

A ``WeightSource`` addresses the tensors of one transformer by the module
paths of the reference model (``transformer_blocks.3.attn1.to_q``,
``adaln_single.linear``, ...; model/transformer/model.py:637-735,
transformer.py:192-284, attention.py:403-418) whatever the file layout:

* ``CacheSource``      a transformer cache built by the reference
                       (loader/transformer_cache.py:1121-1341): plain tensors,
                       ``__layout__.<path>.weight_t`` (W^T) and
                       ``__quant__.<path>.{weight,scales}`` (MXFP8 codes packed
                       in uint32 words + E8M0 scales), single file or shards;
* ``CheckpointSource`` a stock PyTorch checkpoint (``model.diffusion_model.*``
                       keys through ``convert_pytorch_key_to_mlx``), bf16 or
                       FP8 E4M3 with ``weight_scale`` companions.

``install_weights`` writes them into an ``LTXModel`` in its fused layout:

  attn self (attn1, audio_attn1)  proj_q  = [to_q; to_k; to_v; to_gate_logits]
  attn cross (attn2, audio_attn2,  proj_q  = [to_q; to_gate_logits]
   audio_to_video_attn,            proj_kv = [to_k; to_v]
   video_to_audio_attn)            to_out, q_norm, k_norm as named
  ff / audio_ff                   project_in <- project_in.proj, project_out
  per-block tables (16, D) fp32   [scale_shift_table (9) | prompt_scale_shift_table (2)
                                   | scale_shift_table_a2v_ca_{video,audio} (5)]
  top level                       patchify_proj, proj_out, scale_shift_table, the
                                   AdaLN MLPs (emb.timestep_embedder.linear_1/2, linear)
                                   and their audio counterparts

The fused rows are filled part by part, so a quantised format's per-row
blocks (MXFP8 along K, int8 per row) are those of the separate projections.
Resident formats: MXFP8 cache weights stay MXFP8 (bytes copied); plain and
pretransposed weights load as bf16; MXFP8 caches quantised along N
(``mxfp8-blocks-pretranspose``) are decoded exactly to bf16, because the
GEMMs read scales blocked along K.  ``weight_format`` forces a resident
format ("bf16", "int8" or "mxfp8", quantised on the device).  A projection
that the reference runs as a quantised linear keeps that arithmetic
(``LinearWeight.qlinear``: bias added after the bf16 product), also when
decoded to bf16.

Everything is checked before the model is touched: missing tensors, tensors
the model has no place for (the reference's strict ``Module.update``) and
shape mismatches raise ``ValueError``.  Existing device tensors of matching
format and shape are written in place (their addresses stay valid for
captured graphs); others are replaced.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from .. import _lib
from ..kernels import gemm
from . import fp8_checkpoint as fp8
from .safetensors_file import SafetensorsFile
from .weight_converter import CHECKPOINT_PREFIX, convert_pytorch_key_to_mlx

LAYOUT_KEY_PREFIX = "__layout__."
QUANT_KEY_PREFIX = "__quant__."

SELF_ATTENTIONS = ("attn1", "audio_attn1")
CROSS_ATTENTIONS = ("attn2", "audio_attn2", "audio_to_video_attn", "video_to_audio_attn")
VIDEO_MLPS = ("adaln_single", "prompt_adaln_single")
VIDEO_AV_MLPS = ("av_ca_video_scale_shift_adaln_single", "av_ca_a2v_gate_adaln_single")
AUDIO_MLPS = ("audio_adaln_single", "audio_prompt_adaln_single")
AUDIO_AV_MLPS = ("av_ca_audio_scale_shift_adaln_single", "av_ca_v2a_gate_adaln_single")
# block table -> rows of the packed (16, D) table
VIDEO_TABLES = (("scale_shift_table", 0, 9), ("prompt_scale_shift_table", 9, 11),
                ("scale_shift_table_a2v_ca_video", 11, 16))
AUDIO_TABLES = (("audio_scale_shift_table", 0, 9), ("audio_prompt_scale_shift_table", 9, 11),
                ("scale_shift_table_a2v_ca_audio", 11, 16))


@dataclass(frozen=True)
class LinearRecord:
    """Where one linear's weight lives in a source.

    fmt: "bf16" (N, K) | "bf16_t" (K, N) | "mxfp8" codes (N, K) + scales
    (N, K/32) | "mxfp8_t" codes (K, N) + scales (K, N/32) | "e4m3" FP8
    checkpoint codes (N, K) (+ weight_scale).  ``shape`` is (N, K).
    """

    base: str
    fmt: str
    shape: tuple[int, int]
    keys: tuple[str, ...]

    @property
    def quantized(self) -> bool:
        return self.fmt in ("mxfp8", "mxfp8_t")


class WeightSource:
    """Tensors of one transformer addressed by module path."""

    def source_keys(self) -> set[str]:
        raise NotImplementedError

    def linear(self, base: str) -> LinearRecord | None:
        raise NotImplementedError

    def tensor_key(self, name: str) -> str | None:
        raise NotImplementedError

    def shape(self, key: str) -> tuple[int, ...]:
        raise NotImplementedError

    def load_bf16(self, rec: LinearRecord, device) -> torch.Tensor:
        raise NotImplementedError

    def load_mxfp8(self, rec: LinearRecord, device) -> tuple[torch.Tensor, torch.Tensor]:
        raise NotImplementedError

    def load_f32(self, key: str, device) -> torch.Tensor:
        raise NotImplementedError

    def check(self, rec: LinearRecord | None = None, key: str | None = None) -> str | None:
        """Why a weight record / float tensor cannot be loaded, or None."""
        return None


def _decode_mxfp8_rows(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """bf16 (R, C) of codes (R, C) with E8M0 scales per 32 along C (exact)."""
    r, c = codes.shape
    out = torch.empty((r, c), dtype=torch.bfloat16, device=codes.device)
    _lib.call("ltx_dequantize_mxfp8_bf16", _lib.ptr(codes), c, _lib.ptr(scales), scales.stride(0), r, c,
              _lib.ptr(out), c, _lib.stream_of(out), detail=f"R={r} C={c}")
    return out


class _FileSource(WeightSource):
    """Shared fetch logic over a set of safetensors files."""

    def __init__(self):
        self._where: dict[str, SafetensorsFile] = {}

    def shape(self, key: str) -> tuple[int, ...]:
        return self._where[key].shape(key)

    def dtype(self, key: str) -> str:
        return self._where[key].dtype(key)

    def _tensor(self, key: str, device) -> torch.Tensor:
        return self._where[key].tensor(key, device)

    def check(self, rec: LinearRecord | None = None, key: str | None = None) -> str | None:
        if rec is not None and rec.fmt in ("bf16", "bf16_t") and self.dtype(rec.keys[0]) != "BF16":
            return (f"{rec.keys[0]} is stored as {self.dtype(rec.keys[0])}; the resident GEMMs run bf16 "
                    "weights (a cache baked to another transformer dtype is not supported)")
        if key is not None and self.dtype(key) not in ("F32", "BF16", "F16", "F8_E4M3"):
            return f"{key} is stored as {self.dtype(key)}, expected a float tensor"
        return None

    def _bf16_tensor(self, key: str, device) -> torch.Tensor:
        dt = self.dtype(key)
        if dt != "BF16":
            raise ValueError(f"{key} is stored as {dt}; the resident GEMMs run bf16 weights")
        return self._tensor(key, device)

    def load_bf16(self, rec: LinearRecord, device) -> torch.Tensor:
        if rec.fmt == "bf16":
            return self._bf16_tensor(rec.keys[0], device)
        if rec.fmt == "bf16_t":
            return self._bf16_tensor(rec.keys[0], device).t().contiguous()
        if rec.fmt == "mxfp8":
            return _decode_mxfp8_rows(*self.load_mxfp8(rec, device))
        if rec.fmt == "mxfp8_t":
            codes, scales = self._mxfp8_arrays(rec, device)
            return _decode_mxfp8_rows(codes, scales).t().contiguous()
        if rec.fmt == "e4m3":
            codes = self._tensor(rec.keys[0], device)
            scale = self._tensor(rec.keys[1], device) if len(rec.keys) > 1 else None
            return fp8.dequantize_checkpoint_tensor(codes, scale, torch.bfloat16, rec.keys[0])
        raise ValueError(f"unknown weight record format {rec.fmt}")

    def _mxfp8_arrays(self, rec: LinearRecord, device) -> tuple[torch.Tensor, torch.Tensor]:
        qk, sk = rec.keys
        # uint32 words of 4 E4M3 codes, code j of a word in bits [8j, 8j+8):
        # the little-endian bytes are the codes in column order
        codes = torch.from_numpy(np.array(self._where[qk].raw_bytes(qk))).to(device)
        scales = self._tensor(sk, device)
        return codes, scales

    def load_mxfp8(self, rec: LinearRecord, device) -> tuple[torch.Tensor, torch.Tensor]:
        if rec.fmt != "mxfp8":
            raise ValueError(f"{rec.base} is not stored as K-blocked MXFP8")
        return self._mxfp8_arrays(rec, device)

    def load_f32(self, key: str, device) -> torch.Tensor:
        dt = self.dtype(key)
        if dt in ("F8_E4M3",):
            return fp8.dequantize_checkpoint_tensor(self._tensor(key, device), None, torch.float32, key)
        if dt not in ("F32", "BF16", "F16"):
            raise ValueError(f"{key} is stored as {dt}, expected a float tensor")
        return self._tensor(key, device).to(torch.float32)


# -- transformer cache ---------------------------------------------------------
TRANSFORMER_CACHE_QUANTIZE_OFF = "off"
TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS = "mxfp8-blocks"
TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS_PRETRANSPOSE = "mxfp8-blocks-pretranspose"
TRANSFORMER_CACHE_QUANTIZE_MODES = (TRANSFORMER_CACHE_QUANTIZE_OFF, TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS,
                                    TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS_PRETRANSPOSE)
ATTENTION_QUANT_PROJECTIONS = ("to_q", "to_k", "to_v", "to_out", "to_gate_logits")
BLOCK_ATTENTION_MODULES = ("attn1", "attn2", "audio_attn1", "audio_attn2", "audio_to_video_attn",
                           "video_to_audio_attn")
CACHE_QUANTIZED_BLOCK_LINEAR_BASES = tuple(
    f"{a}.{p}" for a in BLOCK_ATTENTION_MODULES for p in ATTENTION_QUANT_PROJECTIONS
) + ("ff.project_in.proj", "ff.project_out", "audio_ff.project_in.proj", "audio_ff.project_out")
# (mode) -> (group size, bits) defaults of the quantised formats (transformer_cache.py:797-811)
QUANT_DEFAULTS = {"affine": (64, 4), "mxfp4": (32, 4), "mxfp8": (32, 8), "nvfp4": (16, 4)}


def quant_defaults(mode: str, group_size: int | None, bits: int | None) -> tuple[int, int]:
    if mode not in QUANT_DEFAULTS:
        raise ValueError(f"Unsupported FF quantization mode: {mode}")
    g, b = QUANT_DEFAULTS[mode]
    return group_size or g, bits or b


def quant_mode_for_base(base: str, *, transformer_cache_quantize: str,
                        quantization_specs: tuple[tuple[str, str], ...]) -> str | None:
    """Quantisation mode of a block linear (block-relative ``base``) in a cache
    (transformer_cache.py:1506-1524): every block linear under the mxfp8 cache
    modes, else the FF targets named in the specs."""
    if (transformer_cache_quantize in (TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS,
                                       TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS_PRETRANSPOSE)
            and base in CACHE_QUANTIZED_BLOCK_LINEAR_BASES):
        return "mxfp8"
    target = {"ff.project_in.proj": "project_in", "ff.project_out": "project_out"}.get(base)
    if target is not None:
        for spec_target, mode in quantization_specs:
            if spec_target == target:
                return mode
    return None


class CacheSource(_FileSource):
    """A reference transformer cache: one ``transformer.safetensors`` or its
    shards ``transformer-NNNNN.safetensors`` (later shards override earlier
    keys, as the reference's merge does, transformer_cache.py:113-125)."""

    def __init__(self, files: list[Path], *, transformer_cache_quantize: str = TRANSFORMER_CACHE_QUANTIZE_OFF,
                 video_ff_quantize_specs: tuple[tuple[str, str], ...] = (),
                 video_ff_quantize_group_size: int | None = None, video_ff_quantize_bits: int | None = None):
        super().__init__()
        if transformer_cache_quantize not in TRANSFORMER_CACHE_QUANTIZE_MODES:
            raise ValueError(f"Unsupported transformer cache quantization mode: {transformer_cache_quantize}")
        self.mode = transformer_cache_quantize
        self.specs = tuple(tuple(s) for s in video_ff_quantize_specs)
        self.group_size = video_ff_quantize_group_size
        self.bits = video_ff_quantize_bits
        self.files = [SafetensorsFile(p) for p in files]
        for f in self.files:
            for k in f.keys():
                self._where[k] = f
        self.plain: dict[str, str] = {}
        self.layout: dict[str, str] = {}
        self.quant: dict[str, str] = {}
        for k in self._where:
            if k.startswith(LAYOUT_KEY_PREFIX):
                self.layout[k[len(LAYOUT_KEY_PREFIX):]] = k
            elif k.startswith(QUANT_KEY_PREFIX):
                self.quant[k[len(QUANT_KEY_PREFIX):]] = k
            else:
                self.plain[k] = k

    def source_keys(self) -> set[str]:
        return set(self._where)

    def tensor_key(self, name: str) -> str | None:
        return self.plain.get(name)

    def linear(self, base: str) -> LinearRecord | None:
        qk = self.quant.get(base + ".weight")
        if qk is not None:
            parts = base.split(".")
            rel = ".".join(parts[2:]) if parts[0] == "transformer_blocks" else base
            mode = quant_mode_for_base(rel, transformer_cache_quantize=self.mode, quantization_specs=self.specs)
            if mode is None:
                raise ValueError(f"Missing cached quantization mode for transformer target: {rel}")
            group, bits = quant_defaults(mode, self.group_size, self.bits)
            if (mode, group, bits) != ("mxfp8", 32, 8):
                raise ValueError(f"{base}: cached {mode} (group {group}, {bits} bits) is not a resident format; "
                                 "only mxfp8 with groups of 32 is")
            if base + ".biases" in self.quant:
                raise ValueError(f"{base}: affine quantisation biases are not supported")
            sk = self.quant.get(base + ".scales")
            if sk is None:
                raise ValueError(f"{base}: quantized weight without scales")
            if self.dtype(qk) != "U32" or self.dtype(sk) != "U8":
                raise ValueError(f"{base}: expected uint32 packed codes and uint8 scales, got "
                                 f"{self.dtype(qk)} / {self.dtype(sk)}")
            rows, words = self.shape(qk)
            cols = 4 * words
            if self.shape(sk) != (rows, cols // 32) or cols % 32:
                raise ValueError(f"{base}: scales {self.shape(sk)} do not match codes ({rows}, {cols})")
            if self.mode == TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS_PRETRANSPOSE:
                return LinearRecord(base, "mxfp8_t", (cols, rows), (qk, sk))
            return LinearRecord(base, "mxfp8", (rows, cols), (qk, sk))
        lk = self.layout.get(base + ".weight_t")
        if lk is not None:
            k, n = self.shape(lk)
            return LinearRecord(base, "bf16_t", (n, k), (lk,))
        pk = self.plain.get(base + ".weight")
        if pk is not None:
            n, k = self.shape(pk)
            return LinearRecord(base, "bf16", (n, k), (pk,))
        return None


class CheckpointSource(_FileSource):
    """A stock PyTorch LTX-2 checkpoint (weight_converter.py:55-108): keys
    under ``model.diffusion_model.`` renamed by ``convert_pytorch_key_to_mlx``;
    other keys (VAE, vocoder, text encoder) are not the transformer's and are
    ignored.  FP8 E4M3 tensors decode with their ``weight_scale`` to bf16 (the
    value the reference's cache build stores); ``input_scale`` and
    ``comfy_quant`` companions are dropped (transformer_cache.py:605-708)."""

    def __init__(self, path: str | Path, *, include_audio: bool):
        super().__init__()
        f = SafetensorsFile(path)
        self.file = f
        dtypes = {k: f.dtype(k) for k in f.keys()}
        if any(d == "F8_E5M2" for d in dtypes.values()):
            raise ValueError("F8_E5M2 checkpoints are not supported (E4M3 only).")
        fp8_keys, weight_scale_keys, input_scale_keys, comfy_keys = fp8.fp8_scale_companions(dtypes)
        skip = weight_scale_keys | input_scale_keys | comfy_keys
        self.fp8_keys = fp8_keys
        self.weight_scale_keys = weight_scale_keys
        self.names: dict[str, str] = {}
        self.skipped = 0
        for k in f.keys():
            self._where[k] = f
            if k in skip or not k.startswith(CHECKPOINT_PREFIX):
                continue
            name = convert_pytorch_key_to_mlx(k[len(CHECKPOINT_PREFIX):], include_audio=include_audio)
            if name is None:
                self.skipped += 1
                continue
            self.names[name] = k

    def source_keys(self) -> set[str]:
        return set(self.names.values())

    def tensor_key(self, name: str) -> str | None:
        return self.names.get(name)

    def linear(self, base: str) -> LinearRecord | None:
        k = self.names.get(base + ".weight")
        if k is None:
            return None
        n, kk = self.shape(k)
        if k in self.fp8_keys:
            sk = k + "_scale"
            return LinearRecord(base, "e4m3", (n, kk), (k, sk) if sk in self.weight_scale_keys else (k,))
        return LinearRecord(base, "bf16", (n, kk), (k,))

    def load_f32(self, key: str, device) -> torch.Tensor:
        if key in self.fp8_keys:
            sk = key + "_scale"
            scale = self._tensor(sk, device) if sk in self.weight_scale_keys else None
            return fp8.dequantize_checkpoint_tensor(self._tensor(key, device), scale, torch.float32, key)
        return super().load_f32(key, device)


# -- installation --------------------------------------------------------------
@dataclass
class InstallCounts:
    """Tensors consumed from the source: all, ``__layout__`` ones and
    ``__quant__`` ones (the reference's load counts)."""

    loaded: int = 0
    layout: int = 0
    quant: int = 0


@dataclass
class _LinearJob:
    owner: object
    attr: str
    parts: list[LinearRecord]
    bias_keys: list[str]
    forced: str | None = None


@dataclass
class _MatrixJob:
    owner: object
    attr: str
    rec: LinearRecord
    transform: object = None  # optional layout change applied to the loaded (N, K) bf16 matrix


@dataclass
class _VectorJob:
    dst: torch.Tensor
    key: str


@dataclass
class _Plan:
    jobs: list = field(default_factory=list)
    missing: list[str] = field(default_factory=list)
    consumed: set[str] = field(default_factory=set)
    errors: list[str] = field(default_factory=list)


class _Planner:
    def __init__(self, src: WeightSource):
        self.src = src
        self.plan = _Plan()

    def linear(self, owner, attr: str, bases: list[str], shapes: list[tuple[int, int]], forced: str | None = None):
        recs, bias_keys = [], []
        ok = True
        for base, shape in zip(bases, shapes):
            rec = self.src.linear(base)
            if rec is None:
                self.plan.missing.append(base + ".weight")
                ok = False
                continue
            self.plan.consumed.update(rec.keys)
            if rec.shape != tuple(shape):
                self.plan.errors.append(f"{base}.weight: shape (N, K) = {rec.shape}, the model expects {tuple(shape)}")
                ok = False
            why = self.src.check(rec=rec)
            if why:
                self.plan.errors.append(why)
                ok = False
            bk = self.src.tensor_key(base + ".bias")
            if bk is None:
                self.plan.missing.append(base + ".bias")
                ok = False
            else:
                self.plan.consumed.add(bk)
                why = self.src.check(key=bk)
                if self.src.shape(bk) != (shape[0],) or why:
                    self.plan.errors.append(why or f"{base}.bias: shape {self.src.shape(bk)}, expected ({shape[0]},)")
                    ok = False
            recs.append(rec)
            bias_keys.append(bk)
        if ok:
            q = [r.quantized for r in recs]
            if any(q) and not all(q):
                self.plan.errors.append(f"{', '.join(bases)}: one fused projection mixes quantised and plain parts")
            else:
                self.plan.jobs.append(_LinearJob(owner, attr, recs, bias_keys, forced))

    def matrix(self, owner, attr: str, base: str, transform=None):
        rec = self.src.linear(base)
        if rec is None:
            self.plan.missing.append(base + ".weight")
            return
        self.plan.consumed.update(rec.keys)
        want = tuple(getattr(owner, attr).shape)
        why = self.src.check(rec=rec)
        if rec.shape != want:
            self.plan.errors.append(f"{base}.weight: shape (N, K) = {rec.shape}, the model expects {want}")
        elif why:
            self.plan.errors.append(why)
        elif rec.quantized:
            self.plan.errors.append(f"{base}.weight: quantised, the model keeps it bf16")
        else:
            self.plan.jobs.append(_MatrixJob(owner, attr, rec, transform))

    def vector(self, dst: torch.Tensor, name: str):
        key = self.src.tensor_key(name)
        if key is None:
            self.plan.missing.append(name)
            return
        self.plan.consumed.add(key)
        why = self.src.check(key=key)
        if tuple(self.src.shape(key)) != tuple(dst.shape):
            self.plan.errors.append(f"{name}: shape {tuple(self.src.shape(key))}, the model expects {tuple(dst.shape)}")
        elif why:
            self.plan.errors.append(why)
        else:
            self.plan.jobs.append(_VectorJob(dst, key))

    def attention(self, a, prefix: str):
        q, kd, inner, h = a.query_dim, a.context_dim, a.inner_dim, a.heads
        if a.self_attention:
            self.linear(a, "proj_q", [f"{prefix}.{p}" for p in ("to_q", "to_k", "to_v", "to_gate_logits")],
                        [(inner, q), (inner, q), (inner, q), (h, q)])
        else:
            self.linear(a, "proj_q", [f"{prefix}.to_q", f"{prefix}.to_gate_logits"], [(inner, q), (h, q)])
            self.linear(a, "proj_kv", [f"{prefix}.to_k", f"{prefix}.to_v"], [(inner, kd), (inner, kd)])
        self.linear(a, "to_out", [f"{prefix}.to_out"], [(q, inner)])
        self.vector(a.q_norm, f"{prefix}.q_norm.weight")
        self.vector(a.k_norm, f"{prefix}.k_norm.weight")

    def ff(self, f, prefix: str):
        self.linear(f, "project_in", [f"{prefix}.project_in.proj"], [(f.inner_dim, f.dim)])
        self.linear(f, "project_out", [f"{prefix}.project_out"], [(f.dim_out, f.inner_dim)])

    def mlp(self, m, prefix: str):
        self.matrix(m, "w1", f"{prefix}.emb.timestep_embedder.linear_1")
        self.vector(m.b1, f"{prefix}.emb.timestep_embedder.linear_1.bias")
        self.matrix(m, "w2", f"{prefix}.emb.timestep_embedder.linear_2")
        self.vector(m.b2, f"{prefix}.emb.timestep_embedder.linear_2.bias")
        self.matrix(m, "w", f"{prefix}.linear")
        self.vector(m.b, f"{prefix}.linear.bias")


def plan_model(model, src: WeightSource) -> _Plan:
    """Every tensor the model takes, resolved against ``src`` (no data read)."""
    p = _Planner(src)
    audio = model.audio_config is not None
    p.linear(model, "patchify_proj", ["patchify_proj"], [tuple(model.patchify_proj.w.shape)], forced="bf16")
    p.linear(model, "proj_out", ["proj_out"], [tuple(model.proj_out.w.shape)], forced="bf16")
    p.vector(model.scale_shift_table, "scale_shift_table")
    mlps = VIDEO_MLPS + (VIDEO_AV_MLPS + AUDIO_MLPS + AUDIO_AV_MLPS if audio else ())
    for name in mlps:
        p.mlp(getattr(model, name), name)
    if audio:
        p.linear(model, "audio_patchify_proj", ["audio_patchify_proj"], [tuple(model.audio_patchify_proj.w.shape)],
                 forced="bf16")
        p.linear(model, "audio_proj_out", ["audio_proj_out"], [tuple(model.audio_proj_out.w.shape)], forced="bf16")
        p.vector(model.audio_scale_shift_table, "audio_scale_shift_table")
    for i, blk in enumerate(model.transformer_blocks):
        pre = f"transformer_blocks.{i}"
        for name in SELF_ATTENTIONS + CROSS_ATTENTIONS:
            a = getattr(blk, name)
            if a is not None:
                p.attention(a, f"{pre}.{name}")
        if blk.ff is not None:
            p.ff(blk.ff, f"{pre}.ff")
        if blk.audio_ff is not None:
            p.ff(blk.audio_ff, f"{pre}.audio_ff")
        for tables, spec in ((blk.video_tables, VIDEO_TABLES), (blk.audio_tables if audio else None, AUDIO_TABLES)):
            if tables is None:
                continue
            for name, r0, r1 in spec if audio else spec[:2]:
                p.vector(tables[r0:r1], f"{pre}.{name}")
    return p.plan


def _block_index(key: str) -> int | None:
    for prefix in ("", LAYOUT_KEY_PREFIX, QUANT_KEY_PREFIX):
        if key.startswith(prefix + "transformer_blocks."):
            part = key[len(prefix) + len("transformer_blocks."):].split(".", 1)[0]
            return int(part) if part.isdigit() else None
    return None


def _run_linear(job: _LinearJob, src: WeightSource, weight_format: str | None, device) -> None:
    parts = job.parts
    n_total = sum(r.shape[0] for r in parts)
    k = parts[0].shape[1]
    quantized = all(r.quantized for r in parts)
    if job.forced is not None:
        target = job.forced
    elif weight_format is not None:
        target = weight_format
    else:
        target = "mxfp8" if all(r.fmt == "mxfp8" for r in parts) else "bf16"
    qlinear = target == "mxfp8" or (target == "bf16" and quantized)
    cur = getattr(job.owner, job.attr)
    reuse = cur is not None and cur.kind == target and tuple(cur.w.shape) == (n_total, k)
    if target == "bf16":
        w = cur.w if reuse else torch.empty((n_total, k), dtype=torch.bfloat16, device=device)
        scale = None
    elif target == "mxfp8":
        w = cur.w if reuse else torch.empty((n_total, k), dtype=torch.uint8, device=device)
        scale = cur.scale if reuse else torch.empty((n_total, k // 32), dtype=torch.uint8, device=device)
    elif target == "int8":
        w = cur.w if reuse else torch.empty((n_total, k), dtype=torch.int8, device=device)
        scale = cur.scale if reuse else torch.empty((n_total,), dtype=torch.float32, device=device)
    else:
        raise ValueError(f"unknown resident weight format {target!r}")
    bias = cur.bias if reuse and cur.bias is not None else torch.empty((n_total,), dtype=torch.float32,
                                                                      device=device)
    r0 = 0
    for rec, bk in zip(parts, job.bias_keys):
        n = rec.shape[0]
        rows = slice(r0, r0 + n)
        if target == "mxfp8" and rec.fmt == "mxfp8":
            codes, sc = src.load_mxfp8(rec, device)
            w[rows].copy_(codes)
            scale[rows].copy_(sc)
        else:
            vals = src.load_bf16(rec, device)
            if target == "bf16":
                w[rows].copy_(vals)
            elif target == "mxfp8":
                _lib.call("ltx_quantize_mxfp8_bf16", _lib.ptr(vals), k, n, k, _lib.ptr(w[rows]), k,
                          _lib.ptr(scale[rows]), k // 32, _lib.stream_of(vals), detail=rec.base)
            else:
                _lib.call("ltx_quantize_w8_bf16", _lib.ptr(vals), k, n, k, _lib.ptr(w[rows]), k,
                          _lib.ptr(scale[rows]), _lib.stream_of(vals), detail=rec.base)
        bias[rows].copy_(src.load_f32(bk, device).reshape(n))
        r0 += n
    setattr(job.owner, job.attr, gemm.LinearWeight(target, w, scale, bias, qlinear=qlinear))


def run_plan(plan: _Plan, src: WeightSource, weight_format: str | None, device) -> None:
    """Execute a checked plan: fill every resident tensor from the source."""
    device = torch.device(device)
    for job in plan.jobs:
        if isinstance(job, _LinearJob):
            _run_linear(job, src, weight_format, device)
        elif isinstance(job, _MatrixJob):
            getattr(job.owner, job.attr).copy_(job.transform(src.load_bf16(job.rec, device))
                                               if job.transform else src.load_bf16(job.rec, device))
        else:
            job.dst.copy_(src.load_f32(job.key, device).reshape(job.dst.shape))
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def install_weights(model, src: WeightSource, *, weight_format: str | None = None,
                    strict: bool = True) -> InstallCounts:
    """Load every tensor of ``model`` from ``src`` (see the module docstring)."""
    if weight_format is not None and weight_format not in gemm.FORMATS:
        raise ValueError(f"weight_format must be one of {gemm.FORMATS} or None, got {weight_format!r}")
    plan = plan_model(model, src)
    n_layers = len(model.transformer_blocks)
    extra = sorted(src.source_keys() - plan.consumed)
    beyond = sorted({b for b in map(_block_index, extra) if b is not None and b >= n_layers})
    if beyond:
        raise ValueError(f"weights have block {beyond[0]}, but the model only has {n_layers} blocks")
    if plan.errors:
        raise ValueError("weights do not fit the model: " + "; ".join(plan.errors[:8]))
    if strict and plan.missing:
        raise ValueError(f"{len(plan.missing)} tensors missing, e.g. " + ", ".join(plan.missing[:8]))
    if strict and extra:
        raise ValueError(f"{len(extra)} tensors have no place in the model, e.g. " + ", ".join(extra[:8]))
    run_plan(plan, src, weight_format, model.device)
    used = plan.consumed
    return InstallCounts(loaded=len(used), layout=sum(k.startswith(LAYOUT_KEY_PREFIX) for k in used),
                         quant=sum(k.startswith(QUANT_KEY_PREFIX) for k in used))
