"""Stock-checkpoint key mapping and direct checkpoint loading.

``convert_pytorch_key_to_mlx`` maps a key of the PyTorch LTX-2 checkpoint
(after the ``model.diffusion_model.`` prefix) to the module path of the
transformer, with the reference's rules (loader/weight_converter.py:10-52):

* without audio, keys naming ``av_ca``, ``a2v`` or ``audio`` (any case) are
  dropped;
* the text-embedding connectors (``video_embeddings_connector``,
  ``audio_embeddings_connector``) are dropped -- they belong to the text
  encoder, not the transformer;
* ``to_out.0.`` -> ``to_out.`` (PyTorch's Sequential index);
* ``ff.net.0.proj.`` -> ``ff.project_in.proj.`` and ``ff.net.2.`` ->
  ``ff.project_out.``, also under ``audio_ff``.

``load_transformer_weights`` (weight_converter.py:55-108) loads a stock
checkpoint into a resident model: bf16 tensors as stored, FP8 E4M3 tensors
dequantised on the device with their ``weight_scale`` (the FP8 rules of
loader/transformer_cache.py:605-708).
"""

from __future__ import annotations

import re
from pathlib import Path

CHECKPOINT_PREFIX = "model.diffusion_model."

_RENAMES = (
    (re.compile(r"\.to_out\.0\."), ".to_out."),
    (re.compile(r"(^|\.)ff\.net\.0\.proj\."), r"\1ff.project_in.proj."),
    (re.compile(r"(^|\.)ff\.net\.2\."), r"\1ff.project_out."),
    (re.compile(r"(^|\.)audio_ff\.net\.0\.proj\."), r"\1audio_ff.project_in.proj."),
    (re.compile(r"(^|\.)audio_ff\.net\.2\."), r"\1audio_ff.project_out."),
)
_CONNECTOR_NAMES = ("video_embeddings_connector", "audio_embeddings_connector")


def convert_pytorch_key_to_mlx(pytorch_key: str, include_audio: bool = False) -> str | None:
    """The transformer module path of a checkpoint key, or None to skip it."""
    key = pytorch_key
    if not include_audio and ("av_ca" in key or "a2v" in key or "audio" in key.lower()):
        return None
    if any(name in key for name in _CONNECTOR_NAMES):
        return None
    for pattern, repl in _RENAMES:
        key = pattern.sub(repl, key)
    return key


def load_transformer_weights(model, weights_path: str | Path, include_audio: bool | None = None, *,
                             weight_format: str | None = None, strict: bool = True) -> int:
    """Load a stock LTX-2 checkpoint (bf16 or FP8 E4M3 safetensors) into the
    resident ``model``; returns the number of tensors loaded.

    ``include_audio`` defaults to whether the model has the audio stream.
    ``weight_format`` picks the resident format of the block projections
    (``None``/"bf16" as stored, "mxfp8" or "int8" quantised on the device).
    """
    from .resident import CheckpointSource, install_weights

    if include_audio is None:
        include_audio = model.audio_config is not None
    src = CheckpointSource(weights_path, include_audio=include_audio)
    counts = install_weights(model, src, weight_format=weight_format, strict=strict)
    return counts.loaded
