"""Tiny safetensors writer for tests (header JSON + raw little-endian data)."""

from __future__ import annotations

import json
import struct


def write_safetensors(path, entries, metadata=None) -> None:
    """entries: [(key, dtype_str, shape, raw_bytes)] in file order."""
    header = {}
    offset = 0
    blobs = []
    for key, dtype, shape, raw in entries:
        header[key] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + len(raw)]}
        offset += len(raw)
        blobs.append(raw)
    if metadata:
        header["__metadata__"] = metadata
    hb = json.dumps(header).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for b in blobs:
            f.write(b)
