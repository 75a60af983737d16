"""Sidecar I/O: named latents / conditioning plus string metadata next to a
run's output (LTX_2_MLX/sidecars.py:1-163).

Two formats, chosen by ``$LTX_SIDECAR_FORMAT`` (default ``safetensors``):

* ``safetensors``: tensors in their native dtype (bf16 included), string
  metadata in the header's ``__metadata__`` -- the file the reference writes
  with ``mx.save_safetensors`` and reads with ``mx.load(...,
  return_metadata=True)``;
* ``npz`` (legacy): numpy has no bf16, so bf16 tensors are widened to fp32 and
  their dtype recorded as ``<key>_mlx_dtype`` (the reference writes MLX's dtype
  name, e.g. ``mlx.core.bfloat16``); metadata as 0-d string arrays; read with
  ``allow_pickle=False``.

Tensors are torch tensors (device tensors are copied to the host to write);
``load_sidecar(path, device=...)`` returns them on ``device``.
"""

from __future__ import annotations

import os

import numpy as np
import torch

from .loader.safetensors_file import SafetensorsFile, write_safetensors

SIDECAR_FORMAT_ENV = "LTX_SIDECAR_FORMAT"
_DEFAULT_FORMAT = "safetensors"
_FORMATS = ("npz", "safetensors")
_MLX_NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32",
              torch.int32: "int32", torch.int64: "int64", torch.uint8: "uint8", torch.int8: "int8",
              torch.bool: "bool_"}
_FROM_MLX = {v: k for k, v in _MLX_NAMES.items()}


def default_format() -> str:
    """The format named by ``$LTX_SIDECAR_FORMAT`` (else the default)."""
    fmt = os.environ.get(SIDECAR_FORMAT_ENV, _DEFAULT_FORMAT).lower()
    if fmt not in _FORMATS:
        raise ValueError(f"{SIDECAR_FORMAT_ENV}={fmt!r}; expected one of {_FORMATS}")
    return fmt


def _ext_for(fmt: str) -> str:
    return ".safetensors" if fmt == "safetensors" else ".npz"


def sidecar_path(base_path: str, suffix: str = "", fmt: str | None = None) -> str:
    """``base_path`` without its extension, plus ``suffix`` and the format's extension."""
    fmt = fmt or default_format()
    stem = os.path.splitext(base_path)[0]
    return f"{stem}{suffix}{_ext_for(fmt)}"


def find_sidecar(base_path: str, suffix: str = "") -> str | None:
    """The existing sidecar next to ``base_path`` (safetensors first, then npz)."""
    stem = os.path.splitext(str(base_path))[0]
    for ext in (".safetensors", ".npz"):
        candidate = f"{stem}{suffix}{ext}"
        if os.path.exists(candidate):
            return candidate
    return None


def save_sidecar(path: str, arrays: dict[str, torch.Tensor], metadata: dict[str, str] | None = None, *,
                 fmt: str | None = None) -> str:
    """Write ``arrays`` and string ``metadata``; the extension follows the
    format.  Returns the path written."""
    metadata = {str(k): str(v) for k, v in (metadata or {}).items()}
    fmt = (fmt or default_format()).lower()
    if fmt not in _FORMATS:
        raise ValueError(f"fmt={fmt!r}; expected one of {_FORMATS}")
    out = os.path.splitext(path)[0] + _ext_for(fmt)
    out_dir = os.path.dirname(out)
    if out_dir:
        os.makedirs(out_dir, exist_ok=True)
    arrays = {k: torch.as_tensor(v) for k, v in arrays.items()}
    if fmt == "safetensors":
        write_safetensors(out, [(k, v, None) for k, v in arrays.items()], metadata=metadata)
    else:
        payload = {}
        for key, t in arrays.items():
            t = t.detach().cpu()
            payload[key] = (t.float() if t.dtype == torch.bfloat16 else t).numpy()
            payload[f"{key}_mlx_dtype"] = np.array(f"mlx.core.{_MLX_NAMES.get(t.dtype, str(t.dtype))}")
        for mkey, mval in metadata.items():
            payload[mkey] = np.array(mval)
        np.savez(out, **payload)
    return out


def load_sidecar(path: str, device: str | torch.device = "cpu") -> tuple[dict[str, torch.Tensor], dict[str, str]]:
    """``(arrays, metadata)`` of a sidecar in either format; tensors in their
    original dtype on ``device``."""
    if str(path).endswith(".safetensors"):
        f = SafetensorsFile(path)
        arrays = {k: f.tensor(k, device) for k in f.keys()}
        return arrays, {str(k): str(v) for k, v in f.metadata.items()}
    arrays: dict[str, torch.Tensor] = {}
    metadata: dict[str, str] = {}
    with np.load(path, allow_pickle=False) as data:
        tags = {k[: -len("_mlx_dtype")]: str(data[k]) for k in data.files if k.endswith("_mlx_dtype")}
        for key in data.files:
            if key.endswith("_mlx_dtype"):
                continue
            val = data[key]
            if val.dtype.kind in ("U", "S"):
                metadata[key] = str(val)
                continue
            t = torch.from_numpy(np.array(val))
            target = _FROM_MLX.get(tags.get(key, "").rsplit(".", 1)[-1])
            if target is not None:
                t = t.to(target)
            arrays[key] = t.to(device)
    metadata.update({f"{k}_mlx_dtype": v for k, v in tags.items()})
    return arrays, metadata
