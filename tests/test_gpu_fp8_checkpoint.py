"""FP8 checkpoint dequantisation on the GPU vs the oracle, bit-exact
(loader/transformer_cache.py:658-708)."""

import struct

import numpy as np
import pytest
import torch

from _safetensors import write_safetensors
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _bits(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float32).view(np.uint32)


@pytest.mark.parametrize("n", [0, 1, 15, 16, 17, 256 * 37 + 13, 1 << 20])
@pytest.mark.parametrize("scale", [None, 2.0, 0.0137, -0.5, 3.0e38, 1e-30])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_dequant_matches_oracle_bit_exact(n, scale, out):
    from ltx_amd.loader.fp8_checkpoint import dequantize_fp8_e4m3

    print(f"fp8 dequant n={n} scale={scale} out={out}", flush=True)
    codes = (np.arange(n) * 7919 % 256).astype(np.uint8)  # every code, scrambled
    dev = torch.from_numpy(codes).cuda()
    sc = None if scale is None else torch.tensor(scale, dtype=torch.float32, device="cuda")
    got = dequantize_fp8_e4m3(dev, sc, torch.bfloat16 if out == "bf16" else torch.float32)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    ref = oq.fp8_checkpoint_dequant(codes, scale, out=out)
    nan = np.isnan(ref)
    assert (np.isnan(got) == nan).all()
    np.testing.assert_array_equal(_bits(got[~nan]), _bits(ref[~nan]))


def test_iterator_reference_case(tmp_path):
    """The reference's own case (tests/test_transformer_cache.py:64-95): scaled
    E4M3 dequantised, companions dropped."""
    from ltx_amd.loader.fp8_checkpoint import iter_fp8_checkpoint_weights

    path = tmp_path / "fp8.safetensors"
    write_safetensors(path, [
        ("model.diffusion_model.layer.weight", "F8_E4M3", [1], bytes([0x38])),
        ("model.diffusion_model.layer.weight_scale", "F32", [1], struct.pack("<f", 2.0)),
        ("model.diffusion_model.layer.input_scale", "F32", [1], struct.pack("<f", 7.0)),
        ("model.diffusion_model.layer.comfy_quant", "U8", [26], b'{"format":"float8_e4m3fn"}'),
    ])
    items = dict(iter_fp8_checkpoint_weights(path, torch.bfloat16))
    assert set(items) == {"model.diffusion_model.layer.weight"}
    w = items["model.diffusion_model.layer.weight"]
    assert w.dtype == torch.bfloat16 and w.is_cuda and float(w.item()) == 2.0


def test_iterator_formats_and_passthrough(tmp_path):
    from ltx_amd.loader.fp8_checkpoint import iter_fp8_checkpoint_weights

    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, size=(64, 48), dtype=np.uint8)
    codes[codes & 0x7F == 0x7F] = 0x11  # no NaN codes in a real weight
    bias = rng.standard_normal(64).astype(np.float32)
    table = rng.standard_normal((6, 32)).astype(np.float32)
    tbl_bf = torch.from_numpy(table).bfloat16()
    path = tmp_path / "ckpt.safetensors"
    write_safetensors(path, [
        ("blk.proj.weight", "F8_E4M3", [64, 48], codes.tobytes()),
        ("blk.proj.weight_scale", "F32", [], struct.pack("<f", 0.0371)),
        ("blk.proj.bias", "F32", [64], bias.tobytes()),
        ("blk.plain.weight", "F8_E4M3", [64, 48], codes.tobytes()),
        ("blk.scale_shift_table", "BF16", [6, 32], tbl_bf.view(torch.int16).numpy().tobytes()),
    ])
    for dtype in (torch.bfloat16, torch.float32, torch.float16):
        items = dict(iter_fp8_checkpoint_weights(path, dtype))
        assert set(items) == {"blk.proj.weight", "blk.proj.bias", "blk.plain.weight", "blk.scale_shift_table"}
        scaled = oq.fp8_checkpoint_dequant(codes, 0.0371, out="f32")
        ref = {torch.bfloat16: torch.from_numpy(scaled).bfloat16(), torch.float32: torch.from_numpy(scaled),
               torch.float16: torch.from_numpy(scaled).half()}[dtype]
        assert items["blk.proj.weight"].dtype == dtype
        assert torch.equal(items["blk.proj.weight"].cpu(), ref)
        plain = torch.from_numpy(oq.fp8_checkpoint_dequant(codes, None, out="f32")).to(dtype)
        assert torch.equal(items["blk.plain.weight"].cpu(), plain)
        # other tensors pass through as stored
        assert items["blk.proj.bias"].dtype == torch.float32
        assert torch.equal(items["blk.proj.bias"].cpu(), torch.from_numpy(bias))
        assert torch.equal(items["blk.scale_shift_table"].cpu(), tbl_bf)


def test_iterator_float16_range_guard(tmp_path):
    from ltx_amd.loader.fp8_checkpoint import iter_fp8_checkpoint_weights

    path = tmp_path / "big.safetensors"
    write_safetensors(path, [
        ("w.weight", "F8_E4M3", [2], bytes([0x7E, 0x38])),  # 448, 1.0
        ("w.weight_scale", "F32", [1], struct.pack("<f", 1000.0)),
    ])
    with pytest.raises(ValueError, match="float16 range"):
        dict(iter_fp8_checkpoint_weights(path, torch.float16))
    w = dict(iter_fp8_checkpoint_weights(path, torch.bfloat16))["w.weight"]
    assert w.float().cpu().tolist() == [448512.0, 1000.0]  # bf16(448000) = 448512
