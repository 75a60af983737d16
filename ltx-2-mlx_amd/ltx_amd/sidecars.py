"""Sidecars: named tensors plus string metadata stored beside a run's output
(latents of each stage, text conditioning).

The on-disk formats are the reference's (LTX_2_MLX/sidecars.py), so files move
between the two implementations in both directions:

* ``safetensors`` -- tensors in their own dtype (bf16 stays bf16), metadata as
  the header's ``__metadata__`` string map;
* ``npz`` (legacy) -- a numpy zip archive.  numpy has no bf16, so every tensor
  is stored widened where needed, with an entry ``<key>_mlx_dtype`` naming its
  original dtype the way MLX prints it (``mlx.core.bfloat16``); metadata
  entries are 0-d string arrays.

The writer's format comes from the ``fmt`` argument or ``$LTX_SIDECAR_FORMAT``
(``safetensors`` when unset); the written file's extension always matches
it.  Readers look at the file itself (a zip archive is the npz form,
anything else must be safetensors), and ``find_sidecar`` prefers a
``.safetensors`` file over an ``.npz`` one of the same stem.

Tensors are torch tensors; device tensors are copied to the host to write,
and ``load_sidecar(path, device=...)`` places what it reads on ``device``.
"""

from __future__ import annotations

import io
import os
from pathlib import Path

import numpy as np
import torch

from .loader.safetensors_file import SafetensorsFile, write_safetensors

SIDECAR_FORMAT_ENV = "LTX_SIDECAR_FORMAT"
DTYPE_TAG_SUFFIX = "_mlx_dtype"
_ZIP_MAGIC = b"PK\x03\x04"


def _mlx_dtype_name(dtype: torch.dtype) -> str:
    """How MLX prints the dtype that matches a torch dtype."""
    short = str(dtype).split(".")[-1]
    return "mlx.core." + ("bool_" if short == "bool" else short)


def _torch_dtype_from_tag(tag: str) -> torch.dtype | None:
    """Inverse of ``_mlx_dtype_name``; None for a name torch does not know."""
    short = tag.strip().split(".")[-1].rstrip("_")
    found = getattr(torch, short, None)
    return found if isinstance(found, torch.dtype) else None


class _SafetensorsSidecar:
    name, suffix = "safetensors", ".safetensors"

    @staticmethod
    def write(path: Path, tensors: dict[str, torch.Tensor], metadata: dict[str, str]) -> None:
        write_safetensors(path, ((k, t, None) for k, t in tensors.items()), metadata=metadata)

    @staticmethod
    def read(path: Path, device) -> tuple[dict[str, torch.Tensor], dict[str, str]]:
        f = SafetensorsFile(path)
        try:
            return ({key: f.tensor(key, device) for key in f.keys()},
                    {str(k): str(v) for k, v in f.metadata.items()})
        finally:
            f.close()


class _NpzSidecar:
    name, suffix = "npz", ".npz"

    @staticmethod
    def write(path: Path, tensors: dict[str, torch.Tensor], metadata: dict[str, str]) -> None:
        entries: dict[str, np.ndarray] = {}
        for key, t in tensors.items():
            host = t.detach().cpu()
            entries[key] = (host.to(torch.float32) if host.dtype == torch.bfloat16 else host).numpy()
            entries[key + DTYPE_TAG_SUFFIX] = np.array(_mlx_dtype_name(host.dtype))
        entries.update({k: np.array(v) for k, v in metadata.items()})
        buf = io.BytesIO()
        np.savez(buf, **entries)
        tmp = path.with_name(f".{path.name}.tmp")
        tmp.write_bytes(buf.getvalue())
        os.replace(tmp, path)

    @staticmethod
    def read(path: Path, device) -> tuple[dict[str, torch.Tensor], dict[str, str]]:
        tensors: dict[str, torch.Tensor] = {}
        metadata: dict[str, str] = {}
        with np.load(path, allow_pickle=False) as archive:
            names = set(archive.files)
            for name in sorted(names):
                value = archive[name]
                if name.endswith(DTYPE_TAG_SUFFIX) or value.dtype.kind in "US":
                    # dtype tags are reported with the metadata, as the reference does
                    metadata[name] = str(value)
                    continue
                t = torch.from_numpy(np.array(value))
                tag = name + DTYPE_TAG_SUFFIX
                want = _torch_dtype_from_tag(str(archive[tag])) if tag in names else None
                tensors[name] = (t if want is None else t.to(want)).to(device)
        return tensors, metadata


_FORMATS = {c.name: c for c in (_SafetensorsSidecar, _NpzSidecar)}
_DEFAULT = _SafetensorsSidecar.name
# when both files of a stem exist, the first suffix here wins
_LOOKUP_SUFFIXES = (_SafetensorsSidecar.suffix, _NpzSidecar.suffix)


def _resolve(fmt: str | None):
    source = "fmt" if fmt is not None else SIDECAR_FORMAT_ENV
    name = (fmt if fmt is not None else os.environ.get(SIDECAR_FORMAT_ENV, _DEFAULT)).lower()
    if name not in _FORMATS:
        raise ValueError(f"unsupported sidecar format {name!r} (from {source}); "
                         f"expected one of {tuple(sorted(_FORMATS))}")
    return _FORMATS[name]


def default_format() -> str:
    """The writer's format when none is passed: ``$LTX_SIDECAR_FORMAT``
    (case-insensitive) or ``safetensors``."""
    return _resolve(None).name


def _stem(path) -> str:
    root, _ext = os.path.splitext(os.fspath(path))
    return root


def sidecar_path(base_path: str, suffix: str = "", fmt: str | None = None) -> str:
    """Sidecar file name for ``base_path``: its extension replaced by
    ``suffix`` plus the format's extension (``run.mp4`` -> ``run_text.npz``)."""
    return _stem(base_path) + suffix + _resolve(fmt).suffix


def find_sidecar(base_path: str, suffix: str = "") -> str | None:
    """The existing sidecar for ``base_path`` and ``suffix`` in either format,
    or None."""
    candidates = (_stem(base_path) + suffix + ext for ext in _LOOKUP_SUFFIXES)
    return next((c for c in candidates if os.path.exists(c)), None)


def save_sidecar(path: str, arrays: dict[str, torch.Tensor], metadata: dict[str, str] | None = None, *,
                 fmt: str | None = None) -> str:
    """Write ``arrays`` and ``metadata`` (values stringified) at ``path`` with
    its extension set by the format; creates the parent directory.  Returns
    the path written."""
    codec = _resolve(fmt)
    out = Path(_stem(path) + codec.suffix)
    out.parent.mkdir(parents=True, exist_ok=True)
    tensors = {str(k): torch.as_tensor(v) for k, v in arrays.items()}
    codec.write(out, tensors, {str(k): str(v) for k, v in (metadata or {}).items()})
    return str(out)


def load_sidecar(path: str, device: str | torch.device = "cpu") -> tuple[dict[str, torch.Tensor], dict[str, str]]:
    """``(tensors, metadata)`` of a sidecar in either format, tensors in the
    dtype they were saved from, on ``device``.  For the npz form the dtype
    tags appear in the metadata too."""
    p = Path(path)
    with open(p, "rb") as fh:
        magic = fh.read(len(_ZIP_MAGIC))
    codec = _NpzSidecar if magic == _ZIP_MAGIC else _SafetensorsSidecar
    return codec.read(p, device)
