"""The C-ABI library loads on the host and exports every declared symbol."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ltx_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+\*?(ltx_[a-z0-9_]+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for must in ("ltx_adaln_norm_fused_bf16", "ltx_gated_add_fused_bf16", "ltx_qknorm_rope_bf16",
                 "ltx_gemm_bf16", "ltx_gemm_w8a16_bf16", "ltx_gemm_mxfp8_bf16", "ltx_flash_attn_bf16"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    from ltx_amd import _lib

    path = _lib.LIB_PATH
    if not path.exists():
        pytest.skip("libltx_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # every declared symbol is bound with a signature in the ctypes layer
    bound = set(_lib.SIGNATURES) | {"ltx_status_string", "ltx_attn_vt_padded_len",
                                     "ltx_attn_splitkv_workspace_bytes", "ltx_gemm_splitk_workspace_bytes",
                                     "ltx_gemm_rows_workspace_bytes", "ltx_gemm_rows_counter_words"}
    assert set(declared_symbols()) <= bound, set(declared_symbols()) - bound


def test_status_strings_and_pure_helpers():
    from ltx_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libltx_hip.so not built")
    lib = _lib.lib()
    assert lib.ltx_status_string(0) == b"ok"
    assert b"unsupported" in lib.ltx_status_string(-2)
    assert lib.ltx_attn_vt_padded_len(68) == 128 and lib.ltx_attn_vt_padded_len(3456) == 3456
    assert lib.ltx_version() >= 100


def test_argument_validation_without_gpu():
    """Shape/argument checks run on the host before any launch."""
    from ltx_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libltx_hip.so not built")
    lib = _lib.lib()
    # C not a multiple of 512 -> unsupported; null pointers -> invalid
    assert lib.ltx_adaln_norm_fused_bf16(16, 3584, 16, 16, 16, 3584, 4, 3584, 1e-6, 0, None) == -2
    assert lib.ltx_adaln_norm_fused_bf16(None, 4096, 16, 16, 16, 4096, 4, 4096, 1e-6, 0, None) == -1
    assert lib.ltx_gemm_bf16(16, 96, 16, 96, None, 16, 64, 4, 64, 96, 0, None, 0, None, 64, None) == -2
    assert lib.ltx_flash_attn_bf16(16, 4096, 16, 4096, 16, 64, 16, 4096, None, 0, 4, 4, 32, 96, 0.1, None) == -2
    # token-major V: head_dim 96 unsupported, V row stride below H*dh invalid,
    # misaligned V / odd stride rejected -- all before any launch
    assert lib.ltx_flash_attn_v_bf16(16, 4096, 16, 4096, 16, 4096, 16, 4096, None, 0, 4, 4, 32, 96, 0.1, None) == -2
    assert lib.ltx_flash_attn_v_bf16(16, 4096, 16, 4096, 16, 2048, 16, 4096, None, 0, 4, 4, 32, 128, 0.1,
                                     None) == -1
    assert lib.ltx_flash_attn_v_bf16(16, 4096, 16, 4096, 24, 4096, 16, 4096, None, 0, 4, 4, 32, 128, 0.1,
                                     None) == -4
    assert lib.ltx_flash_attn_splitkv_v_bf16(16, 4096, 16, 4096, 16, 4100, 16, 4096, None, 0, 4, 4, 32, 128, 0.1,
                                             4, 16, 1 << 20, None) == -4
    # device clock stamp: null or misaligned destination rejected before any launch
    assert lib.ltx_device_clock_stamp(None, None) == -1
    assert lib.ltx_device_clock_stamp(12, None) == -4
    # zero rows is a no-op success
    assert lib.ltx_adaln_norm_fused_bf16(16, 4096, 16, 16, 16, 4096, 0, 4096, 1e-6, 0, None) == 0
    # FP8 checkpoint dequant: null codes -> invalid, fp16 output -> unsupported,
    # misaligned codes -> alignment, zero elements -> no-op success
    assert lib.ltx_dequantize_fp8_e4m3(None, 16, None, 16, 0, None) == -1
    assert lib.ltx_dequantize_fp8_e4m3(16, 16, None, 16, 2, None) == -2
    assert lib.ltx_dequantize_fp8_e4m3(17, 16, None, 16, 0, None) == -4
    assert lib.ltx_dequantize_fp8_e4m3(16, 0, None, 16, 0, None) == 0
    # GEMM flags: the quantised-linear bias form is accepted (M = 0: no launch),
    # an unknown flag bit is rejected
    assert lib.ltx_gemm_bf16(16, 64, 16, 64, None, 16, 64, 0, 64, 64, _lib.GEMM_ROUND_THEN_BIAS, None, 0, None,
                             64, None) == 0
    assert lib.ltx_gemm_bf16(16, 64, 16, 64, None, 16, 64, 0, 64, 64, 1 << 13, None, 0, None, 64, None) == -1
    # split-K: workspace size, and too-small workspace / bad split counts rejected before any launch
    assert lib.ltx_gemm_splitk_workspace_bytes(68, 2048, 4) == 4 * 68 * 2048 * 4
    assert lib.ltx_gemm_splitk_bf16(16, 2048, 16, 2048, None, 16, 64, 4, 64, 2048, 0, None, 0, None, 64, 4,
                                    16, 16, None) == -1
    assert lib.ltx_gemm_splitk_bf16(16, 2048, 16, 2048, None, 16, 64, 4, 64, 2048, 0, None, 0, None, 64, 3,
                                    16, 1 << 30, None) == -2
    # few-row GEMM: workspace and counter sizes; missing counters with splits > 1,
    # a K not divisible by 128 * splits (8-bit weights), a misaligned scale row
    # and a bad split count rejected before any launch
    assert lib.ltx_gemm_rows_workspace_bytes(68, 2048, 4) == 4 * 68 * 2048 * 4
    assert lib.ltx_gemm_rows_counter_words(68, 2048) == 16
    assert lib.ltx_gemm_rows_counter_words(121, 6176) == 49
    assert lib.ltx_gemm_rows_counter_words(256, 4096) == 64
    assert lib.ltx_gemm_rows_bf16(16, 2048, 16, 2048, None, 16, 2048, 68, 2048, 2048, 0, None, 0, None, 2048, 4,
                                  16, 1 << 30, None, 0, None) == -1
    assert lib.ltx_gemm_rows_mxfp8_bf16(16, 2048, 16, 2048, 16, 64, None, 16, 2048, 68, 2048, 2048, 0, None, 0,
                                        None, 2048, 32, 16, 1 << 30, 16, 1 << 10, None) == -2
    assert lib.ltx_gemm_rows_mxfp8_bf16(16, 2048, 16, 2048, 16, 66, None, 16, 2048, 68, 2048, 2048, 0, None, 0,
                                        None, 2048, 4, 16, 1 << 30, 16, 1 << 10, None) == -4
    assert lib.ltx_gemm_rows_w8a16_bf16(16, 2048, 16, 2048, 16, None, 16, 2048, 68, 2048, 2048, 0, None, 0,
                                        None, 2048, 65, 16, 1 << 30, 16, 1 << 10, None) == -1
