"""FP8 (E4M3) safetensors checkpoints, dequantised at load time.

Mirrors the reference's FP8 checkpoint path (loader/transformer_cache.py:553-708
and safetensors_header.py:20-60):

* ``read_safetensors_header`` / ``read_safetensors_dtypes`` parse only the
  8-byte length prefix and the JSON header, never the tensor data.
* ``fp8_scale_companions`` classifies the FP8 keys and their companions with
  the reference's rules (``_fp8_scale_companions``, transformer_cache.py:605-655):
  ``<base>.weight_scale`` (consumed: the dequant factor), ``<base>.input_scale``
  (dropped: static activation quantisation of real FP8 GEMMs) and ComfyUI's
  ``<base>.comfy_quant`` metadata tag (dropped); a ``*_scale`` key whose base
  is not FP8 is an ordinary tensor.
* ``iter_fp8_checkpoint_weights`` yields ``(key, tensor)`` like
  ``_iter_fp8_checkpoint_weights`` (transformer_cache.py:658-708): E5M2
  checkpoints are rejected, companions are skipped, a scaled FP8 tensor becomes
  ``from_fp8(w) * weight_scale`` in fp32 rounded once to ``value_dtype`` (with
  the float16 range check of ``_cast_for_cache``, :557-576), an unscaled one is
  decoded exactly, every other tensor is yielded as stored.  The decode runs in
  the HIP kernel ``ltx_dequantize_fp8_e4m3`` on the device; the file is read
  one tensor at a time (memory-mapped), so the whole checkpoint is never held.
"""

from __future__ import annotations

import json
import struct
from pathlib import Path
from typing import Any, Iterator

import numpy as np
import torch

from .. import _lib

FP8_SAFETENSORS_DTYPES = frozenset({"F8_E4M3", "F8_E5M2"})
FP16_MAX = 65504.0

# safetensors dtype -> (numpy storage dtype, torch dtype)
_DTYPES = {
    "F64": (np.float64, torch.float64),
    "F32": (np.float32, torch.float32),
    "F16": (np.float16, torch.float16),
    "BF16": (np.int16, torch.bfloat16),
    "I64": (np.int64, torch.int64),
    "I32": (np.int32, torch.int32),
    "I16": (np.int16, torch.int16),
    "I8": (np.int8, torch.int8),
    "U8": (np.uint8, torch.uint8),
    "BOOL": (np.bool_, torch.bool),
    "F8_E4M3": (np.uint8, torch.uint8),
}


def read_safetensors_header(path: str | Path) -> dict[str, Any]:
    """The full JSON header of a safetensors file (no tensor data)."""
    with open(path, "rb") as f:
        header_len = struct.unpack("<Q", f.read(8))[0]
        return json.loads(f.read(header_len))


def read_safetensors_dtypes(path: str | Path) -> dict[str, str]:
    """Tensor key -> raw safetensors dtype string (``F32``, ``F8_E4M3``, ...)."""
    header = read_safetensors_header(path)
    return {k: v["dtype"] for k, v in header.items()
            if k != "__metadata__" and isinstance(v, dict) and "dtype" in v}


def checkpoint_has_fp8_tensors(path: str | Path) -> bool:
    """True when the safetensors file stores any FP8 tensor."""
    try:
        dtypes = set(read_safetensors_dtypes(path).values())
    except Exception:
        return False
    return bool(FP8_SAFETENSORS_DTYPES & dtypes)


def fp8_scale_companions(header_dtypes: dict[str, str]) -> tuple[set, set, set, set]:
    """``(fp8_keys, weight_scale_keys, input_scale_keys, comfy_quant_keys)``."""
    fp8_keys = {k for k, d in header_dtypes.items() if d in FP8_SAFETENSORS_DTYPES}
    weight_scale_keys = {k for k in header_dtypes if k.endswith("_scale") and k[: -len("_scale")] in fp8_keys}
    input_scale_keys = set()
    for k in fp8_keys:
        if k.endswith(".weight"):
            cand = k[: -len(".weight")] + ".input_scale"
            if cand in header_dtypes:
                input_scale_keys.add(cand)
    comfy_quant_keys = {k for k in header_dtypes
                        if k.endswith(".comfy_quant") and k[: -len(".comfy_quant")] + ".weight" in fp8_keys}
    return fp8_keys, weight_scale_keys, input_scale_keys, comfy_quant_keys


def dequantize_fp8_e4m3(codes: torch.Tensor, scale: torch.Tensor | None = None,
                        dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``dtype(from_fp8(codes) * scale)`` with the product in fp32 (exact decode
    without a scale).  ``codes``: uint8 E4M3 device tensor of any shape;
    ``scale``: fp32 scalar device tensor or None; ``dtype``: bf16 or fp32."""
    if codes.dtype != torch.uint8:
        raise TypeError(f"E4M3 codes must be uint8, got {codes.dtype}")
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"dequantize_fp8_e4m3 writes bfloat16 or float32, not {dtype}")
    codes = codes.contiguous()
    out = torch.empty(codes.shape, dtype=dtype, device=codes.device)
    sc = None
    if scale is not None:
        if scale.numel() != 1:
            raise ValueError("the kernel takes a per-tensor scale")
        sc = scale.to(device=codes.device, dtype=torch.float32).reshape(1).contiguous()
    if codes.numel():
        _lib.call("ltx_dequantize_fp8_e4m3", _lib.ptr(codes), codes.numel(), _lib.ptr(sc), _lib.ptr(out),
                  0 if dtype == torch.bfloat16 else 1, _lib.stream_of(out))
    return out


def _load_tensor(mm: np.memmap, data_start: int, entry: dict, device) -> torch.Tensor:
    np_dtype, t_dtype = _DTYPES[entry["dtype"]]
    begin, end = entry["data_offsets"]
    arr = np.frombuffer(mm, dtype=np.uint8, count=end - begin, offset=data_start + begin)
    arr = arr.view(np_dtype).reshape(entry["shape"])
    t = torch.from_numpy(arr.copy())
    if t_dtype == torch.bfloat16:
        t = t.view(torch.bfloat16)
    return t.to(device)


def _cast_for_cache(value: torch.Tensor, target: torch.dtype, key: str) -> torch.Tensor:
    if target == torch.float16 and value.dtype != torch.float16:
        max_abs = float(value.float().abs().max()) if value.numel() else 0.0
        if max_abs > FP16_MAX:
            raise ValueError(f"{key}: max|w|={max_abs:.4g} exceeds the float16 range ({FP16_MAX:.0f}); "
                             "cannot bake this tensor to float16. Use bfloat16 for this checkpoint.")
    return value.to(target)


def iter_fp8_checkpoint_weights(weights_path: str | Path, value_dtype: torch.dtype = torch.bfloat16,
                                device: str | torch.device = "cuda") -> Iterator[tuple[str, torch.Tensor]]:
    """Yield ``(key, tensor)`` of an FP8 safetensors checkpoint, FP8 tensors
    dequantised on ``device`` (see the module docstring)."""
    header = read_safetensors_header(weights_path)
    dtypes = {k: v["dtype"] for k, v in header.items() if k != "__metadata__" and isinstance(v, dict)}
    if any(d == "F8_E5M2" for d in dtypes.values()):
        raise ValueError("F8_E5M2 checkpoints are not supported (E4M3 only).")
    if value_dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"unsupported value dtype {value_dtype}")
    fp8_keys, weight_scale_keys, input_scale_keys, comfy_quant_keys = fp8_scale_companions(dtypes)
    skip = weight_scale_keys | input_scale_keys | comfy_quant_keys
    with open(weights_path, "rb") as f:
        header_len = struct.unpack("<Q", f.read(8))[0]
    data_start = 8 + header_len
    mm = np.memmap(weights_path, dtype=np.uint8, mode="r")
    for key, entry in header.items():
        if key == "__metadata__" or not isinstance(entry, dict) or key in skip:
            continue
        stored = _load_tensor(mm, data_start, entry, device)
        if key in fp8_keys:
            scale_key = f"{key}_scale"
            scale = None
            if scale_key in weight_scale_keys:
                scale = _load_tensor(mm, data_start, header[scale_key], device)
            stored = dequantize_checkpoint_tensor(stored, scale, value_dtype, key)
        yield key, stored


def dequantize_checkpoint_tensor(codes: torch.Tensor, scale: torch.Tensor | None, value_dtype: torch.dtype,
                                 key: str = "") -> torch.Tensor:
    """One FP8 checkpoint tensor in ``value_dtype`` (transformer_cache.py:691-705):
    ``from_fp8(codes) * weight_scale`` in fp32 rounded once, or the exact
    decode without a scale (|w| <= 448 fits every value dtype)."""
    if scale is None:
        inter = torch.bfloat16 if value_dtype == torch.bfloat16 else torch.float32
        return dequantize_fp8_e4m3(codes, None, inter).to(value_dtype)
    scale = scale.to(device=codes.device, dtype=torch.float32)
    if scale.numel() == 1:
        inter = torch.float32 if value_dtype != torch.bfloat16 else torch.bfloat16
        value = dequantize_fp8_e4m3(codes, scale, inter)
    else:  # broadcast scale: exact decode, then the fp32 product
        value = dequantize_fp8_e4m3(codes, None, torch.float32) * scale
    return _cast_for_cache(value, value_dtype, key)
