"""Latent sidecars (LTX_2_MLX/sidecars.py, av_pipeline.py:233-290,
scripts/stage2_harness.py:56-85) on the host."""

import json
import struct

import numpy as np
import pytest
import torch


def test_paths_and_format_selection(tmp_path, monkeypatch):
    from ltx_amd import sidecars as sc

    monkeypatch.delenv(sc.SIDECAR_FORMAT_ENV, raising=False)
    assert sc.default_format() == "safetensors"
    assert sc.sidecar_path("out/run.mp4", "_text") == "out/run_text.safetensors"
    monkeypatch.setenv(sc.SIDECAR_FORMAT_ENV, "NPZ")
    assert sc.sidecar_path("out/run.mp4") == "out/run.npz"
    monkeypatch.setenv(sc.SIDECAR_FORMAT_ENV, "pickle")
    with pytest.raises(ValueError, match="expected one of"):
        sc.default_format()
    base = tmp_path / "run.mp4"
    assert sc.find_sidecar(str(base)) is None
    (tmp_path / "run.npz").write_bytes(b"")
    assert sc.find_sidecar(str(base)).endswith("run.npz")
    (tmp_path / "run.safetensors").write_bytes(b"")
    assert sc.find_sidecar(str(base)).endswith("run.safetensors")  # safetensors first


def test_safetensors_round_trip_native_dtypes(tmp_path):
    from ltx_amd import sidecars as sc

    v = torch.randn(1, 128, 3, 4, 6).bfloat16()
    a = torch.randn(1, 8, 5, 16)
    s = torch.tensor(1, dtype=torch.int32)
    out = sc.save_sidecar(str(tmp_path / "lat.npz"), {"final_video_latent": v, "final_audio_latent": a,
                                                       "schema_version": s},
                          {"pipeline": "distilled_two_stage", "n": 3}, fmt="safetensors")
    assert out.endswith("lat.safetensors")  # extension follows the format
    # the header is plain safetensors with string metadata
    raw = open(out, "rb").read()
    hdr = json.loads(raw[8:8 + struct.unpack("<Q", raw[:8])[0]])
    assert hdr["__metadata__"] == {"pipeline": "distilled_two_stage", "n": "3"}
    assert hdr["final_video_latent"]["dtype"] == "BF16" and hdr["final_video_latent"]["shape"] == [1, 128, 3, 4, 6]
    arrays, meta = sc.load_sidecar(out)
    assert torch.equal(arrays["final_video_latent"], v) and arrays["final_video_latent"].dtype == torch.bfloat16
    assert torch.equal(arrays["final_audio_latent"], a) and arrays["schema_version"].item() == 1
    assert meta == {"pipeline": "distilled_two_stage", "n": "3"}


def test_npz_legacy_round_trip_and_reference_written_file(tmp_path):
    from ltx_amd import sidecars as sc

    v = torch.randn(1, 128, 2, 3, 4).bfloat16()
    out = sc.save_sidecar(str(tmp_path / "lat"), {"final_video_latent": v}, {"prompt": "a cat"}, fmt="npz")
    with np.load(out, allow_pickle=False) as d:
        assert d["final_video_latent"].dtype == np.float32  # bf16 widened
        assert str(d["final_video_latent_mlx_dtype"]) == "mlx.core.bfloat16"
        assert str(d["prompt"]) == "a cat"
    arrays, meta = sc.load_sidecar(out)
    assert arrays["final_video_latent"].dtype == torch.bfloat16 and torch.equal(arrays["final_video_latent"], v)
    assert meta["prompt"] == "a cat" and meta["final_video_latent_mlx_dtype"] == "mlx.core.bfloat16"
    # a file in the reference's npz layout written by numpy alone
    ref = tmp_path / "ref.npz"
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    np.savez(ref, x=x, x_mlx_dtype=np.array("mlx.core.bfloat16"), y=np.ones(2, np.int32),
             pipeline=np.array("distilled_two_stage"))
    arrays, meta = sc.load_sidecar(str(ref))
    assert arrays["x"].dtype == torch.bfloat16 and torch.equal(arrays["x"].float(), torch.from_numpy(x))
    assert arrays["y"].dtype == torch.int32 and meta["pipeline"] == "distilled_two_stage"


def test_stage_sidecars(tmp_path):
    from ltx_amd import pipeline as pl

    v1, v2 = torch.randn(1, 128, 3, 4, 6).bfloat16(), torch.randn(1, 128, 3, 8, 12).bfloat16()
    a1 = torch.randn(1, 8, 5, 16).bfloat16()
    out = pl.save_distilled_two_stage_latents(str(tmp_path / "run"), v1, v2, a1, a1)
    from ltx_amd.sidecars import load_sidecar

    arrays, meta = load_sidecar(out)
    assert set(arrays) == {"stage_1_video_latent", "stage_2_video_latent", "final_video_latent",
                           "stage_1_audio_latent", "stage_2_audio_latent", "final_audio_latent"}
    assert meta == {"pipeline": "distilled_two_stage"} and torch.equal(arrays["final_video_latent"], v2)
    video, audio, md = pl.load_stage1_latents(out)
    assert torch.equal(video, v1) and torch.equal(audio, a1)
    assert md == {"pipeline": "distilled_two_stage", "video_shape": (1, 128, 3, 4, 6), "audio_shape": (1, 8, 5, 16)}
    assert pl.infer_dimensions_from_stage1(video) == (256, 384, 17)
    final = pl.save_final_latents(str(tmp_path / "final"), v2)
    with pytest.raises(ValueError, match="does not contain stage_1_video_latent"):
        pl.load_stage1_latents(final)
    with pytest.raises(ValueError, match="must be 5D"):
        pl.infer_dimensions_from_stage1(v2[0])


def test_text_conditioning_sidecars(tmp_path):
    from ltx_amd import pipeline as pl
    from ltx_amd.sidecars import save_sidecar

    pv, nv = torch.randn(1, 1024, 64).bfloat16(), torch.randn(1, 1024, 64).bfloat16()
    pa = torch.randn(1, 1024, 32).bfloat16()
    m = torch.ones(1, 1024, dtype=torch.int32)
    p = save_sidecar(str(tmp_path / "run_text"), {"schema_version": torch.tensor(1, dtype=torch.int32),
                                                  "positive_video_encoding": pv, "positive_attention_mask": m,
                                                  "negative_video_encoding": nv, "positive_audio_encoding": pa},
                     {"prompt": "p", "negative_prompt": ""})
    c = pl.load_text_conditioning(p)
    assert c["format"] == "text_conditioning" and torch.equal(c["positive_video_encoding"], pv)
    assert c["negative_audio_encoding"] is None and torch.equal(c["positive_audio_encoding"], pa)
    legacy = save_sidecar(str(tmp_path / "emb"), {"embedding": pv, "attention_mask": m})
    c = pl.load_text_conditioning(legacy)
    assert c["format"] == "legacy" and torch.equal(c["positive_video_encoding"], pv)
    assert c["positive_audio_encoding"] is None
