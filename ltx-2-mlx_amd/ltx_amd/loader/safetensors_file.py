"""Memory-mapped safetensors files: header-only indexing, per-tensor reads and
a sharded writer.

The reference reads its checkpoints and caches with ``mx.load`` (lazy, mmap;
loader/transformer_cache.py:113-125) and writes shards with
``mx.save_safetensors`` behind an atomic rename (:1229-1241).  Here a file is
indexed from its JSON header alone; a tensor's bytes are read only when it is
fetched, so a 40 GB checkpoint is never resident in host memory.

Layout of a safetensors file: an 8-byte little-endian header length, the JSON
header ``{key: {"dtype", "shape", "data_offsets": [begin, end]}, ...,
"__metadata__": {...}}``, then the tensor bytes (offsets relative to the end of
the header).
"""

from __future__ import annotations

import json
import os
import struct
from pathlib import Path
from typing import Any, Iterable

import numpy as np
import torch

# safetensors dtype -> (numpy storage dtype, element bytes)
STORAGE_DTYPES: dict[str, np.dtype] = {
    "F64": np.dtype(np.float64),
    "F32": np.dtype(np.float32),
    "F16": np.dtype(np.float16),
    "BF16": np.dtype(np.uint16),
    "I64": np.dtype(np.int64),
    "I32": np.dtype(np.int32),
    "I16": np.dtype(np.int16),
    "I8": np.dtype(np.int8),
    "U64": np.dtype(np.uint64),
    "U32": np.dtype(np.uint32),
    "U16": np.dtype(np.uint16),
    "U8": np.dtype(np.uint8),
    "BOOL": np.dtype(np.bool_),
    "F8_E4M3": np.dtype(np.uint8),
    "F8_E5M2": np.dtype(np.uint8),
}

# torch dtype of a fetched tensor (8-bit floats and unsigned words stay raw)
_TORCH_DTYPES = {
    "F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
    "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8,
    "U8": torch.uint8, "BOOL": torch.bool, "F8_E4M3": torch.uint8, "F8_E5M2": torch.uint8,
}

_TORCH_TO_SAFETENSORS = {
    torch.float64: "F64", torch.float32: "F32", torch.float16: "F16", torch.bfloat16: "BF16",
    torch.int64: "I64", torch.int32: "I32", torch.int16: "I16", torch.int8: "I8",
    torch.uint8: "U8", torch.bool: "BOOL",
}


class SafetensorsFile:
    """One safetensors file, indexed from its header; tensors read on demand."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        with open(self.path, "rb") as f:
            raw = f.read(8)
            if len(raw) != 8:
                raise ValueError(f"{self.path}: not a safetensors file (short header)")
            header_len = struct.unpack("<Q", raw)[0]
            header = json.loads(f.read(header_len))
        self.data_start = 8 + header_len
        self.metadata: dict[str, str] = header.pop("__metadata__", None) or {}
        self.entries: dict[str, dict[str, Any]] = header
        self._mm: np.memmap | None = None
        size = self.path.stat().st_size
        for key, e in self.entries.items():
            b, end = e["data_offsets"]
            if e["dtype"] not in STORAGE_DTYPES:
                raise ValueError(f"{self.path}: tensor {key} has unsupported dtype {e['dtype']}")
            if not 0 <= b <= end or self.data_start + end > size:
                raise ValueError(f"{self.path}: tensor {key} lies outside the file")
            want = int(np.prod(e["shape"], dtype=np.int64)) * STORAGE_DTYPES[e["dtype"]].itemsize
            if end - b != want:
                raise ValueError(f"{self.path}: tensor {key} holds {end - b} bytes, shape {e['shape']} "
                                 f"of {e['dtype']} needs {want}")

    def keys(self) -> list[str]:
        return list(self.entries)

    def __contains__(self, key: str) -> bool:
        return key in self.entries

    def dtype(self, key: str) -> str:
        return self.entries[key]["dtype"]

    def shape(self, key: str) -> tuple[int, ...]:
        return tuple(self.entries[key]["shape"])

    def nbytes(self, key: str) -> int:
        b, e = self.entries[key]["data_offsets"]
        return e - b

    def array(self, key: str) -> np.ndarray:
        """Read-only view of the stored elements (bf16 as uint16 words)."""
        if self._mm is None:
            self._mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        e = self.entries[key]
        b, end = e["data_offsets"]
        dt = STORAGE_DTYPES[e["dtype"]]
        raw = self._mm[self.data_start + b: self.data_start + end]
        return raw.view(dt).reshape(e["shape"])

    def raw_bytes(self, key: str) -> np.ndarray:
        """The stored bytes as a uint8 array of shape (*shape[:-1], bytes per row)."""
        e = self.entries[key]
        shape = list(e["shape"]) or [1]
        row = shape[-1] * STORAGE_DTYPES[e["dtype"]].itemsize
        return self.array(key).reshape(-1).view(np.uint8).reshape(*shape[:-1], row)

    def tensor(self, key: str, device: str | torch.device = "cpu") -> torch.Tensor:
        """The tensor in its stored dtype (8-bit floats as uint8 codes)."""
        dt = self.dtype(key)
        if dt not in _TORCH_DTYPES:
            raise ValueError(f"{self.path}: {key} is {dt}; read it with raw_bytes()")
        arr = np.array(self.array(key))  # one host copy, writable for torch
        t = torch.from_numpy(arr)
        if dt == "BF16":
            t = t.view(torch.bfloat16)
        return t.to(device)

    def close(self) -> None:
        self._mm = None


def write_safetensors(path: str | Path, tensors: Iterable[tuple[str, torch.Tensor | np.ndarray, str | None]],
                      metadata: dict[str, str] | None = None) -> int:
    """Write ``(key, tensor, dtype)`` triples (dtype None: from the tensor) to
    ``path`` through a temporary file and an atomic rename; returns the bytes
    of tensor data written.  Tensors may live on the device."""
    path = Path(path)
    header: dict[str, Any] = {}
    blobs = []
    offset = 0
    for key, t, dtype in tensors:
        if isinstance(t, torch.Tensor):
            t = t.detach().contiguous().cpu()
            dt = dtype or _TORCH_TO_SAFETENSORS[t.dtype]
            if t.dtype == torch.bfloat16:
                t = t.view(torch.int16)
            blob = t.numpy().tobytes()
            shape = list(t.shape)
        else:
            if dtype is None:
                raise ValueError(f"{key}: numpy tensors need an explicit safetensors dtype")
            dt = dtype
            blob = np.ascontiguousarray(t).tobytes()
            shape = list(t.shape)
        header[key] = {"dtype": dt, "shape": shape, "data_offsets": [offset, offset + len(blob)]}
        blobs.append(blob)
        offset += len(blob)
    if metadata:
        header["__metadata__"] = dict(metadata)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)  # keep the data 8-byte aligned
    tmp = path.with_name(f".{path.stem}.tmp{path.suffix}")
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for blob in blobs:
            f.write(blob)
    os.replace(tmp, path)
    return offset
