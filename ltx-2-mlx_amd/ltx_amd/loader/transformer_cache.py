"""The reference's transformer weight cache, read into (and written from) the
resident model.

Mirrors the loading half of loader/transformer_cache.py:

* cache files (:85-125): ``transformer.safetensors`` or its shards
  ``transformer-00000.safetensors, ...`` beside it (sorted; later shards
  override earlier keys); ``metadata.json`` in the same directory holds the
  build options (:453-525, :1009-1014);
* key kinds (:22-34): plain module paths, ``__layout__.<path>.weight_t``
  (a pretransposed bf16 weight) and ``__quant__.<path>.{weight,scales}``
  (MXFP8: uint32 words of 4 E4M3 codes + uint8 E8M0 scales per 32 along K;
  along N for ``mxfp8-blocks-pretranspose``);
* ``load_transformer_cache(model, cache_file, ...) -> (loaded, layout,
  quant)`` (:1668-1746) and the restore-state helpers (:128-164).

``build_transformer_cache`` writes a cache of the same format from a stock
checkpoint (:1121-1341): keys renamed, FP8 tensors dequantised, block linears
optionally MXFP8-quantised (with this library's encoder), 4 GiB shards
written through a temporary file and renamed, metadata last.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np
import torch

from .resident import (  # noqa: F401  (re-exported names of the reference module)
    ATTENTION_QUANT_PROJECTIONS,
    BLOCK_ATTENTION_MODULES,
    CACHE_QUANTIZED_BLOCK_LINEAR_BASES,
    LAYOUT_KEY_PREFIX,
    QUANT_KEY_PREFIX,
    TRANSFORMER_CACHE_QUANTIZE_MODES,
    TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS,
    TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS_PRETRANSPOSE,
    TRANSFORMER_CACHE_QUANTIZE_OFF,
    CacheSource,
    CheckpointSource,
    LinearRecord,
    install_weights,
    quant_defaults,
    quant_mode_for_base,
)
from .safetensors_file import write_safetensors

CACHE_SCHEMA_VERSION = 1
TRANSFORMER_CACHE_RESTORE_ATTR = "_transformer_cache_restore_source"
TRANSFORMER_SHARD_LIMIT_BYTES = 4 * 1024 ** 3
METADATA_FILENAME = "metadata.json"


@dataclass(frozen=True)
class TransformerCacheResult:
    """Result metadata for a transformer cache load or build."""

    cache_path: Path
    rebuilt: bool
    loaded_count: int
    layout_count: int
    quant_count: int = 0


def cache_shard_path(cache_file: Path, index: int) -> Path:
    cache_file = Path(cache_file)
    return cache_file.with_name(f"{cache_file.stem}-{index:05d}{cache_file.suffix}")


def existing_cache_shards(cache_file: Path) -> list[Path]:
    cache_file = Path(cache_file)
    return sorted(cache_file.parent.glob(f"{cache_file.stem}-[0-9]*{cache_file.suffix}"))


def cache_artifacts_exist(cache_file: Path) -> bool:
    """True if a cache is present as a single file or as shards."""
    return Path(cache_file).exists() or bool(existing_cache_shards(cache_file))


def clear_cache_artifacts(cache_file: Path) -> None:
    """Remove a cache before a rebuild: ``metadata.json`` first (a cache
    without it is an incomplete build), then the single file and any shards."""
    cache_file = Path(cache_file)
    meta = cache_file.parent / METADATA_FILENAME
    if meta.exists():
        meta.unlink()
    if cache_file.exists():
        cache_file.unlink()
    for shard in existing_cache_shards(cache_file):
        shard.unlink()


def cache_payload(weights_path: str | Path, *, include_audio: bool,
                  transformer_cache_quantize: str = TRANSFORMER_CACHE_QUANTIZE_OFF) -> dict[str, Any]:
    """The build description stored as ``metadata.json``, with the fields and
    values the reference's cache payload has for the builds made here
    (loader/transformer_cache.py:453-514): schema version, the source file's
    resolved path / size / mtime, the audio flag, the (empty) layout
    pretranspose lists, the quantisation mode when not off, and
    ``fp8_dequant_policy`` 2 for checkpoints holding FP8 tensors -- so the
    reference's metadata comparison accepts a cache built here."""
    from .fp8_checkpoint import checkpoint_has_fp8_tensors

    src = Path(weights_path).expanduser().resolve()
    st = src.stat()
    payload: dict[str, Any] = {
        "schema_version": CACHE_SCHEMA_VERSION,
        "source": {"path": str(src), "size": st.st_size, "mtime_ns": st.st_mtime_ns},
        "include_audio": bool(include_audio),
        "video_ff_layout_specs": [],
        "video_ff_layout_layers": [],
        "video_attn_layout_specs": [],
        "video_attn_layout_layers": [],
    }
    if transformer_cache_quantize != TRANSFORMER_CACHE_QUANTIZE_OFF:
        payload["transformer_cache_quantize"] = transformer_cache_quantize
    if checkpoint_has_fp8_tensors(src):
        payload["fp8_dequant_policy"] = 2
    return payload


def _write_metadata(cache_file: Path, payload: dict[str, Any]) -> None:
    """``metadata.json`` through a temporary file and an atomic rename: a
    reader sees the old file, no file, or the whole new one."""
    final = Path(cache_file).parent / METADATA_FILENAME
    tmp = final.with_name(final.name + ".tmp")
    tmp.write_text(json.dumps(payload, indent=2, sort_keys=True) + "\n")
    os.replace(tmp, final)


def cache_files(cache_file: Path) -> list[Path]:
    """The files of a cache: the single file if present, else its shards."""
    cache_file = Path(cache_file)
    if cache_file.exists():
        return [cache_file]
    shards = existing_cache_shards(cache_file)
    if not shards:
        raise FileNotFoundError(f"No cache at {cache_file} and no shards beside it.")
    return shards


def read_cache_metadata(cache_file: Path) -> dict[str, Any] | None:
    """The build options stored beside the cache, or None."""
    path = Path(cache_file).parent / METADATA_FILENAME
    try:
        with path.open("r", encoding="utf-8") as f:
            return json.load(f)
    except (OSError, json.JSONDecodeError):
        return None


def _options_from_metadata(meta: dict[str, Any] | None) -> dict[str, Any]:
    meta = meta or {}
    specs = tuple((s["target"], s["mode"]) for s in meta.get("video_ff_quantize_specs", ()))
    return {
        "transformer_cache_quantize": meta.get("transformer_cache_quantize", TRANSFORMER_CACHE_QUANTIZE_OFF),
        "video_ff_quantize_specs": specs,
        "video_ff_quantize_group_size": meta.get("transformer_cache_quantize_group_size",
                                                 meta.get("video_ff_quantize_group_size")),
        "video_ff_quantize_bits": meta.get("transformer_cache_quantize_bits", meta.get("video_ff_quantize_bits")),
    }


def open_transformer_cache(cache_file: Path, *, transformer_cache_quantize: str | None = None,
                           video_ff_quantize_specs: tuple[tuple[str, str], ...] | None = None,
                           video_ff_quantize_group_size: int | None = None,
                           video_ff_quantize_bits: int | None = None) -> CacheSource:
    """Index a cache (headers only).  Options left None come from the cache's
    ``metadata.json`` when present (else: no quantisation)."""
    opts = _options_from_metadata(read_cache_metadata(cache_file))
    if transformer_cache_quantize is not None:
        opts["transformer_cache_quantize"] = transformer_cache_quantize
    if video_ff_quantize_specs is not None:
        opts["video_ff_quantize_specs"] = tuple(video_ff_quantize_specs)
    if video_ff_quantize_group_size is not None:
        opts["video_ff_quantize_group_size"] = video_ff_quantize_group_size
    if video_ff_quantize_bits is not None:
        opts["video_ff_quantize_bits"] = video_ff_quantize_bits
    return CacheSource(cache_files(cache_file), **opts)


def load_transformer_cache(model, cache_file: Path, *, transformer_cache_quantize: str | None = None,
                           video_ff_quantize_specs: tuple[tuple[str, str], ...] | None = None,
                           video_ff_quantize_group_size: int | None = None,
                           video_ff_quantize_bits: int | None = None, weight_format: str | None = None,
                           strict: bool = True) -> tuple[int, int, int]:
    """Load a transformer cache into the resident ``model``; returns
    ``(loaded_count, layout_count, quant_count)``.  ``weight_format`` forces a
    resident format for the block projections (default: as cached)."""
    src = open_transformer_cache(cache_file, transformer_cache_quantize=transformer_cache_quantize,
                                 video_ff_quantize_specs=video_ff_quantize_specs,
                                 video_ff_quantize_group_size=video_ff_quantize_group_size,
                                 video_ff_quantize_bits=video_ff_quantize_bits)
    counts = install_weights(model, src, weight_format=weight_format, strict=strict)
    setattr(model, TRANSFORMER_CACHE_RESTORE_ATTR, {
        "valid": True,
        "cache_path": Path(cache_file),
        "transformer_cache_quantize": src.mode,
        "video_ff_quantize_specs": src.specs,
        "video_ff_quantize_group_size": src.group_size,
        "video_ff_quantize_bits": src.bits,
        "weight_format": weight_format,
    })
    return counts.loaded, counts.layout, counts.quant


def get_transformer_cache_restore_state(model) -> dict:
    """The cache a model was loaded from, for reloading it after in-place
    weight changes (transformer_cache.py:128-137)."""
    source = getattr(model, TRANSFORMER_CACHE_RESTORE_ATTR, None)
    if source and source.get("valid"):
        return dict(source)
    raise RuntimeError("Transformer cache restore requires a valid cache-backed transformer. "
                       "Reload from cache before temporary or stage-specific in-place mutation.")


def restore_transformer_cache_state(model, state: dict) -> None:
    """Reload the transformer weights from a restore state."""
    load_transformer_cache(model, state["cache_path"],
                           transformer_cache_quantize=state["transformer_cache_quantize"],
                           video_ff_quantize_specs=state["video_ff_quantize_specs"],
                           video_ff_quantize_group_size=state["video_ff_quantize_group_size"],
                           video_ff_quantize_bits=state["video_ff_quantize_bits"],
                           weight_format=state.get("weight_format"))


def invalidate_transformer_cache_restore_state(model) -> None:
    """Mark the restore state stale after an in-place weight change."""
    source = getattr(model, TRANSFORMER_CACHE_RESTORE_ATTR, None)
    if source:
        source = dict(source)
        source["valid"] = False
        setattr(model, TRANSFORMER_CACHE_RESTORE_ATTR, source)


# -- build -----------------------------------------------------------------------
def _quantize_mxfp8(w: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """(uint32 words (R, C/4), uint8 scales (R, C/32)) of a bf16 (R, C) device
    tensor, blocks of 32 along C."""
    from .. import _lib

    r, c = w.shape
    w = w.contiguous()
    q = torch.empty((r, c), dtype=torch.uint8, device=w.device)
    s = torch.empty((r, c // 32), dtype=torch.uint8, device=w.device)
    _lib.call("ltx_quantize_mxfp8_bf16", w.data_ptr(), c, r, c, q.data_ptr(), c, s.data_ptr(), c // 32,
              _lib.stream_of(w), detail=f"R={r} C={c}")
    words = q.cpu().numpy().view(np.uint32).reshape(r, c // 4)  # little-endian: code j in bits [8j, 8j+8)
    return words, s.cpu().numpy()


def build_transformer_cache(weights_path: str | Path, cache_file: Path, *, include_audio: bool,
                            transformer_cache_quantize: str = TRANSFORMER_CACHE_QUANTIZE_OFF,
                            shard_limit_bytes: int = TRANSFORMER_SHARD_LIMIT_BYTES,
                            device: str | torch.device = "cuda") -> TransformerCacheResult:
    """Convert a stock checkpoint (bf16 or FP8 E4M3) into a transformer cache.

    Block linears (``CACHE_QUANTIZED_BLOCK_LINEAR_BASES``) are stored as
    ``__quant__`` MXFP8 under the mxfp8 modes (W^T quantised for the
    pretranspose mode); every other tensor is stored as its module path, FP8
    tensors dequantised to bf16.  Returns the counts like a load.
    """
    if transformer_cache_quantize not in TRANSFORMER_CACHE_QUANTIZE_MODES:
        raise ValueError(f"Unsupported transformer cache quantization mode: {transformer_cache_quantize}")
    cache_file = Path(cache_file)
    cache_file.parent.mkdir(parents=True, exist_ok=True)
    clear_cache_artifacts(cache_file)
    src = CheckpointSource(weights_path, include_audio=include_audio)
    quantize = transformer_cache_quantize != TRANSFORMER_CACHE_QUANTIZE_OFF
    pretranspose = transformer_cache_quantize == TRANSFORMER_CACHE_QUANTIZE_MXFP8_BLOCKS_PRETRANSPOSE
    pending: list[tuple[str, Any, str | None]] = []
    pending_bytes = 0
    shard = 0
    loaded = quant = 0

    def flush():
        nonlocal pending, pending_bytes, shard
        if pending:
            write_safetensors(cache_shard_path(cache_file, shard), pending)
            shard += 1
            pending, pending_bytes = [], 0

    for name in sorted(src.names):
        if pending_bytes >= shard_limit_bytes:
            flush()
        parts = name.split(".")
        base = ".".join(parts[:-1])
        rel = ".".join(parts[2:-1]) if parts[0] == "transformer_blocks" else None
        if quantize and parts[-1] == "weight" and rel in CACHE_QUANTIZED_BLOCK_LINEAR_BASES:
            w = src.load_bf16(src.linear(base), device)
            words, scales = _quantize_mxfp8(w.t() if pretranspose else w)
            pending += [(f"{QUANT_KEY_PREFIX}{base}.weight", words, "U32"),
                        (f"{QUANT_KEY_PREFIX}{base}.scales", scales, "U8")]
            pending_bytes += words.nbytes + scales.nbytes
            quant += 2
            loaded += 1
            continue
        key = src.names[name]
        if src.dtype(key) == "F8_E4M3":  # dequantised once into bf16, as the reference's build does
            sk = key + "_scale"
            keys = (key, sk) if sk in src.weight_scale_keys else (key,)
            t = src.load_bf16(LinearRecord(name, "e4m3", (0, 0), keys), device)
        else:
            t = src._tensor(key, "cpu")
        pending.append((name, t, None))
        pending_bytes += t.numel() * t.element_size()
        loaded += 1
    flush()
    _write_metadata(cache_file, cache_payload(weights_path, include_audio=include_audio,
                                              transformer_cache_quantize=transformer_cache_quantize))
    return TransformerCacheResult(cache_file, True, loaded, 0, quant)
