"""FP8 checkpoint loading, host logic (loader/transformer_cache.py:553-708)."""

import struct

import numpy as np
import pytest
import torch

from _safetensors import write_safetensors
from ltx_amd.loader import fp8_checkpoint as fc
from oracle import quant as oq


def test_fp8_companion_filter_scopes_comfy_quant_to_fp8_weights():
    # the reference's own case (tests/test_transformer_cache.py:47-61)
    header_dtypes = {
        "layer.weight": "F8_E4M3",
        "layer.weight_scale": "F32",
        "layer.input_scale": "F32",
        "layer.comfy_quant": "U8",
        "unrelated.comfy_quant": "U8",
    }
    fp8, weight_scales, input_scales, comfy = fc.fp8_scale_companions(header_dtypes)
    assert fp8 == {"layer.weight"}
    assert weight_scales == {"layer.weight_scale"}
    assert input_scales == {"layer.input_scale"}
    assert comfy == {"layer.comfy_quant"}


def test_scale_key_of_a_non_fp8_tensor_is_ordinary():
    fp8, ws, _, _ = fc.fp8_scale_companions({"adaln.scale_shift_table": "F32", "x.weight": "BF16",
                                             "x.weight_scale": "F32"})
    assert fp8 == set() and ws == set()


def test_header_readers(tmp_path):
    path = tmp_path / "m.safetensors"
    write_safetensors(path, [("a", "F32", [2], struct.pack("<2f", 1.0, 2.0)),
                             ("b", "F8_E4M3", [3], bytes([1, 2, 3]))], metadata={"format": "pt"})
    assert fc.read_safetensors_dtypes(path) == {"a": "F32", "b": "F8_E4M3"}
    assert fc.read_safetensors_header(path)["__metadata__"] == {"format": "pt"}
    assert fc.checkpoint_has_fp8_tensors(path)
    plain = tmp_path / "p.safetensors"
    write_safetensors(plain, [("a", "F32", [1], struct.pack("<f", 1.0))])
    assert not fc.checkpoint_has_fp8_tensors(plain)
    assert not fc.checkpoint_has_fp8_tensors(tmp_path / "missing.safetensors")


def test_e5m2_checkpoint_is_rejected(tmp_path):
    path = tmp_path / "e5m2.safetensors"
    write_safetensors(path, [("layer.weight", "F8_E5M2", [1], bytes([0x3C]))])
    with pytest.raises(ValueError, match="E5M2"):
        next(fc.iter_fp8_checkpoint_weights(path, device="cpu"))


def test_oracle_dequant_matches_torch_casts():
    codes = np.arange(256, dtype=np.uint8)
    f8 = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    for scale in (None, 2.0, 0.0137, -0.5, 3.0e38, 1e-30):
        ref = f8 if scale is None else f8 * torch.tensor(scale, dtype=torch.float32)
        got_f32 = oq.fp8_checkpoint_dequant(codes, scale, out="f32")
        got_bf = oq.fp8_checkpoint_dequant(codes, scale)
        nan = torch.isnan(ref).numpy()
        assert (np.isnan(got_f32) == nan).all() and (np.isnan(got_bf) == nan).all()
        np.testing.assert_array_equal(got_f32[~nan], ref.numpy()[~nan])
        np.testing.assert_array_equal(got_bf[~nan], ref.bfloat16().float().numpy()[~nan])
    # the reference's known answer (tests/test_transformer_cache.py:64-95)
    assert oq.fp8_checkpoint_dequant([0x38], 2.0)[0] == 2.0
