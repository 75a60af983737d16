"""ctypes binding of libltx_hip.so (declarations mirror include/ltx_hip.h).

The library is loaded lazily on first use.  A missing or unloadable library
raises immediately: there is no silent CPU or eager fallback behind these
entry points.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_NAME = "libltx_hip.so"
LIB_PATH = Path(os.environ.get("LTX_HIP_LIB", Path(__file__).with_name(LIB_NAME)))

_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_vp = ctypes.c_void_p

# name -> argtypes (every function returns int status)
SIGNATURES: dict[str, list] = {
    "ltx_version": [],
    "ltx_device_clock_stamp": [_vp, _vp],
    "ltx_adaln_norm_fused_bf16": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _int, _vp],
    "ltx_gated_add_fused_bf16": [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _int, _vp],
    "ltx_qknorm_rope_bf16": [
        _vp, _i64, _i64, _vp, _vp, _vp,
        _vp, _i64, _i64, _vp, _vp, _vp,
        _i64, _i64, _f32, _vp,
    ],
    "ltx_output_norm_modulate_bf16": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _vp],
    "ltx_euler_x0_step_bf16": [_vp, _vp, _f32, _f32, _vp, _i64, _vp],
    "ltx_timestep_embedding_f32": [_vp, _i64, _f32, _vp, _i64, _vp],
    "ltx_gemv_f32_bf16w": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _int, _vp],
    "ltx_gemm_bf16": [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, _i64, _vp],
    "ltx_gemm_w8a16_bf16": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp,
                            _i64, _vp],
    "ltx_gemm_mxfp8_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64,
                            _vp, _i64, _vp],
    "ltx_gemm_rowss_bf16": [_int, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _i64,
                            _vp, _i64, _i64, _vp],
    "ltx_gemm_splitk_bf16": [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, _i64,
                             _int, _vp, _i64, _vp],
    "ltx_gemm_splitk_w8a16_bf16": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64,
                                   _vp, _i64, _int, _vp, _i64, _vp],
    "ltx_gemm_splitk_mxfp8_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp,
                                   _i64, _vp, _i64, _int, _vp, _i64, _vp],
    "ltx_gemm_rows_bf16": [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, _i64,
                           _int, _vp, _i64, _vp, _i64, _vp],
    "ltx_gemm_rows_w8a16_bf16": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64,
                                 _vp, _i64, _int, _vp, _i64, _vp, _i64, _vp],
    "ltx_gemm_rows_mxfp8_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp,
                                 _i64, _vp, _i64, _int, _vp, _i64, _vp, _i64, _vp],
    "ltx_gemm_mx_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp,
                         _i64, _vp, _i64, _vp],
    "ltx_gemm_mx_gelu_mxfp8": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                               _i64, _int, _vp],
    "ltx_quantize_mxfp8_bf16": [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp],
    "ltx_dequantize_mxfp8_bf16": [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp],
    "ltx_quantize_w8_bf16": [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp],
    "ltx_dequantize_w8_bf16": [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp],
    "ltx_dequantize_fp8_e4m3": [_vp, _i64, _vp, _vp, _int, _vp],
    "ltx_attn_transpose_v_bf16": [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp],
    "ltx_flash_attn_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp],
    "ltx_flash_attn_splitkv_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
                                    _f32, _i64, _vp, _i64, _vp],
    "ltx_flash_attn_splitkv_noalloc_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64,
                                            _i64, _i64, _f32, _i64, _vp],
    "ltx_adaln_norm_fused2_bf16": [_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _int,
                                   _vp],
    "ltx_qknorm_rope_axes_bf16": [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp,
                                  _vp, _i64, _i64, _i64, _i64, _f32, _vp],
    "ltx_flash_attn_v_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _f32,
                              _vp],
    "ltx_flash_attn_qnorm_v_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                                    _i64, _f32, _vp, _i64, _i64, _vp, _f32, _vp, _vp, _vp, _i64, _i64, _vp],
    "ltx_flash_attn_splitkv_v_bf16": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                                      _i64, _f32, _i64, _vp, _i64, _vp],
    "ltx_broadcast_add_f32": [_vp, _vp, _vp, _i64, _i64, _vp],
    "ltx_x0_from_velocity_f32": [_vp, _vp, _f32, _vp, _i64, _vp],
    "ltx_guidance_f32": [_vp, _vp, _vp, _vp, _f32, _f32, _f32, _vp, _vp, _vp, _i64, _int, _vp],
    "ltx_guidance_stats_f32": [_vp, _vp, _i64, _int, _f32, _f32, _vp, _vp],
    "ltx_ge_correct_f32": [_vp, _vp, _vp, _int, _f32, _f32, _i64, _vp],
    "ltx_euler_step_bf16": [_vp, _vp, _f32, _vp, _i64, _vp],
    "ltx_swap_axes": [_vp, _i64, _i64, _i64, _int, _vp, _vp],
    "ltx_gemma_features_bf16": [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _f32, _f32, _f32, _vp, _vp, _i64, _vp],
}

# Flag values (include/ltx_hip.h)
ADALN_ROUND_NORM = 1
ADALN_NO_NORM = 2
GATED_ROUND_PRODUCT = 1
GEMV_SILU_INPUT = 1
GEMV_SILU_OUTPUT = 2
GEMM_EPI_BIAS = 0
GEMM_EPI_GELU = 1
GEMM_EPI_RESIDUAL = 2
GEMM_EPI_RESIDUAL_ROUND = 3
GEMM_EPI_SIGMOID2 = 4
GEMM_TILE_256 = 1 << 8
GEMM_TILE_128 = 2 << 8
GEMM_TILE_256_DMA = 3 << 8
GEMM_TILE_256x128 = 4 << 8
GEMM_TILE_G8 = 5 << 8
GEMM_TILE_G8_128 = 6 << 8
GEMM_ROUND_THEN_BIAS = 1 << 12
# Status of a request above the fixed scratch of a no-allocation entry point
ERR_SCRATCH_LIMIT = -5
ATTN_NOALLOC_SCRATCH_BYTES = 32 << 20

_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Return the loaded library, loading it on first call."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python ltx-2-mlx_amd/build_lib.py` "
                "(or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        handle.ltx_attn_vt_padded_len.argtypes = [_i64]
        handle.ltx_attn_vt_padded_len.restype = _i64
        handle.ltx_attn_splitkv_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
        handle.ltx_attn_splitkv_workspace_bytes.restype = _i64
        handle.ltx_gemm_splitk_workspace_bytes.argtypes = [_i64, _i64, _i64]
        handle.ltx_gemm_splitk_workspace_bytes.restype = _i64
        handle.ltx_gemm_rows_workspace_bytes.argtypes = [_i64, _i64, _i64]
        handle.ltx_gemm_rows_workspace_bytes.restype = _i64
        handle.ltx_gemm_rows_counter_words.argtypes = [_i64, _i64]
        handle.ltx_gemm_rows_counter_words.restype = _i64
        handle.ltx_status_string.argtypes = [ctypes.c_int]
        handle.ltx_status_string.restype = ctypes.c_char_p
        _LIB = handle
    return _LIB


class LtxKernelError(RuntimeError):
    """A libltx_hip entry point returned a non-zero status."""

    def __init__(self, name: str, status: int, detail: str = ""):
        msg = lib().ltx_status_string(status).decode()
        super().__init__(f"{name} failed with status {status} ({msg}){': ' + detail if detail else ''}")
        self.status = status


def call(name: str, *args, detail: str = "") -> None:
    status = getattr(lib(), name)(*args)
    if status != 0:
        raise LtxKernelError(name, status, detail)


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError(f"expected a device tensor, got one on {t.device}")
    return t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def row_view(t: torch.Tensor, cols: int) -> tuple[torch.Tensor, int]:
    """Return (tensor, row_stride) such that `t` is seen as (rows, cols) rows
    of unit column stride.  Copies only if the layout is not row-uniform."""
    if t.shape[-1] != cols:
        raise ValueError(f"last dim {t.shape[-1]} != {cols}")
    if t.dim() == 1:
        return t.contiguous(), cols
    if t.stride(-1) == 1:
        # leading dims must collapse to one uniform stride
        lead = t.shape[:-1]
        strides = t.stride()[:-1]
        row_stride = strides[-1]
        expect = row_stride
        ok = True
        for size, stride in zip(reversed(lead), reversed(strides)):
            if size != 1 and stride != expect:
                ok = False
                break
            expect = stride * size if size != 1 else expect
        if ok:
            return t, row_stride
    t = t.contiguous()
    return t, cols
