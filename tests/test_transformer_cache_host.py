"""Checkpoint / transformer-cache loading on the host (no GPU).

Key renames against the reference's own cases (tests/test_loaders.py:34-90),
the safetensors reader (and the byte order of MLX's packed uint32 words),
shard discovery and merge order (tests/test_transformer_cache.py:174-190),
and the full mapping of named tensors into the fused resident layout: a
synthetic model written under the reference's names is installed into a CPU
model (formats whose install is a copy: bf16, pretransposed bf16, K-blocked
MXFP8 bytes) and every resident tensor is compared bit for bit with the
tensor it came from, read back by name.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

import _cache_fixture as fx


def _model(layers=2, audio=False, fmt="bf16"):
    from ltx_amd.model.transformer.model import LTXModel

    return LTXModel(num_layers=layers, num_attention_heads=2, attention_head_dim=64, cross_attention_dim=192,
                    weight_format=fmt, device="cpu", audio=audio, init="empty", audio_attention_heads=4,
                    audio_attention_head_dim=64)


def _W(layers=2, audio=False, seed=0, mxfp8=False):
    """Small widths: video 2x64 heads (context 192), audio 4x64 heads."""
    return fx.synthetic_weights(layers, 128, 2, 192, audio, seed=seed, mxfp8_blocks=mxfp8, ad=256, ah=4)


# -- key conversion --------------------------------------------------------------
def test_converter_reference_cases():
    """The reference's known answers (tests/test_loaders.py:34-90)."""
    from ltx_amd.loader import convert_pytorch_key_to_mlx as conv

    for key in ("av_ca.to_q.weight", "audio_ff.net.0.proj.weight"):
        assert conv(key, include_audio=False) is None
    assert conv("audio_ff.net.0.proj.weight", include_audio=True) == "audio_ff.project_in.proj.weight"
    assert conv("video_embeddings_connector.proj.weight") is None
    assert conv("attn.to_out.0.weight") == "attn.to_out.weight"
    assert conv("ff.net.0.proj.weight") == "ff.project_in.proj.weight"
    assert conv("ff.net.2.weight") == "ff.project_out.weight"
    assert conv("audio_ff.net.2.weight", include_audio=True) == "audio_ff.project_out.weight"
    assert conv("audio_embeddings_connector.proj.weight", include_audio=True) is None


def test_converter_block_keys():
    from ltx_amd.loader import convert_pytorch_key_to_mlx as conv

    assert conv("transformer_blocks.7.attn2.to_out.0.bias") == "transformer_blocks.7.attn2.to_out.bias"
    assert conv("transformer_blocks.7.ff.net.0.proj.bias") == "transformer_blocks.7.ff.project_in.proj.bias"
    assert (conv("transformer_blocks.0.audio_ff.net.0.proj.weight", include_audio=True)
            == "transformer_blocks.0.audio_ff.project_in.proj.weight")
    assert conv("transformer_blocks.0.scale_shift_table_a2v_ca_video") is None  # "a2v" without audio
    assert conv("transformer_blocks.0.AUDIO_attn1.to_q.weight") is None  # case-insensitive "audio"
    assert conv("transformer_blocks.0.q_norm.weight") == "transformer_blocks.0.q_norm.weight"
    # every fixture name survives the round trip through the checkpoint names
    for base in fx.linear_shapes(1, 128, 2, 192, True):
        assert conv(fx.pytorch_name(base + ".weight")[len("model.diffusion_model."):], True) == base + ".weight"


# -- safetensors -------------------------------------------------------------------
def test_safetensors_reader_dtypes_and_u32_byte_order(tmp_path):
    from ltx_amd.loader.safetensors_file import SafetensorsFile

    rng = np.random.default_rng(0)
    codes = rng.integers(0, 256, size=(3, 64), dtype=np.uint8)
    vals = fx.bf16r(rng.standard_normal((5, 7)).astype(np.float32))
    f32 = rng.standard_normal(9).astype(np.float32)
    p = tmp_path / "a.safetensors"
    fx.write_safetensors(p, [("q", "U32", fx._pack_u32(codes)), ("b", "BF16", vals), ("f", "F32", f32)])
    f = SafetensorsFile(p)
    assert f.dtype("q") == "U32" and f.shape("q") == (3, 16)
    np.testing.assert_array_equal(f.raw_bytes("q"), codes)  # little-endian words: codes in k order
    np.testing.assert_array_equal(f.tensor("b").float().numpy(), vals)
    np.testing.assert_array_equal(f.tensor("f").numpy(), f32)
    # a truncated file is rejected from its header
    data = p.read_bytes()
    (tmp_path / "t.safetensors").write_bytes(data[:-4])
    with pytest.raises(ValueError, match="outside the file"):
        SafetensorsFile(tmp_path / "t.safetensors")


def test_safetensors_writer_round_trip(tmp_path):
    from ltx_amd.loader.safetensors_file import SafetensorsFile, write_safetensors

    t = torch.randn(4, 6).bfloat16()
    u = np.arange(12, dtype=np.uint32).reshape(3, 4)
    write_safetensors(tmp_path / "w.safetensors", [("t", t, None), ("u", u, "U32")], metadata={"k": "v"})
    f = SafetensorsFile(tmp_path / "w.safetensors")
    assert torch.equal(f.tensor("t"), t) and f.metadata == {"k": "v"}
    np.testing.assert_array_equal(f.array("u"), u)
    assert not list(tmp_path.glob(".*tmp*"))  # the temporary file was renamed away


# -- cache files ---------------------------------------------------------------------
def test_sharded_cache_discovery_and_override(tmp_path):
    """Shards beside the cache name are merged in order, a later shard's key
    overriding an earlier one (tests/test_transformer_cache.py:174-190)."""
    from ltx_amd.loader.transformer_cache import cache_files, cache_shard_path, open_transformer_cache

    cache = tmp_path / "transformer.safetensors"
    assert cache_shard_path(cache, 3).name == "transformer-00003.safetensors"
    with pytest.raises(FileNotFoundError, match="No cache at"):
        cache_files(cache)
    fx.write_safetensors(tmp_path / "transformer-00000.safetensors",
                         [("transformer_blocks.0.weight", "F32", np.array([1.0], np.float32)),
                          ("shared", "F32", np.array([1.0], np.float32))])
    fx.write_safetensors(tmp_path / "transformer-00001.safetensors",
                         [("transformer_blocks.1.weight", "F32", np.array([2.0], np.float32)),
                          ("shared", "F32", np.array([2.0], np.float32))])
    src = open_transformer_cache(cache)
    assert len(src.files) == 2
    assert float(src.load_f32("transformer_blocks.1.weight", "cpu")) == 2.0
    assert float(src.load_f32("shared", "cpu")) == 2.0
    # a single file takes precedence over shards
    fx.write_safetensors(cache, [("only", "F32", np.array([3.0], np.float32))])
    assert [p.name for p in cache_files(cache)] == ["transformer.safetensors"]


# -- installation (CPU model) ------------------------------------------------------
@pytest.mark.parametrize("shards", [1, 3])
def test_install_bf16_cache(tmp_path, shards):
    from ltx_amd.loader import load_transformer_cache

    W = _W(layers=2)
    layout = ("transformer_blocks.1.attn1.to_v", "transformer_blocks.0.ff.project_out", "adaln_single.linear")
    items = fx.cache_items(W, layout=layout)
    cache = tmp_path / "c" / "transformer.safetensors"
    fx.write_cache(cache, items, shards=shards)
    model = _model(layers=2)
    loaded, n_layout, n_quant = load_transformer_cache(model, cache)
    assert (loaded, n_layout, n_quant) == (len(items), len(layout), 0)
    fx.check_against_named(model, W)
    for b in model.transformer_blocks:
        assert all(not w.qlinear and w.kind == "bf16" for w in b.linear_weights())


def test_install_av_cache(tmp_path):
    from ltx_amd.loader import load_transformer_cache

    W = _W(layers=1, audio=True, seed=4)
    cache = tmp_path / "transformer.safetensors"
    fx.write_cache(cache, fx.cache_items(W), shards=2)
    model = _model(layers=1, audio=True)
    load_transformer_cache(model, cache)
    fx.check_against_named(model, W)


def test_install_mxfp8_cache_copies_bytes(tmp_path):
    """``mxfp8-blocks``: codes and scales land byte for byte in the fused rows;
    the weights keep the quantised-linear arithmetic."""
    from ltx_amd.loader import load_transformer_cache

    W = _W(layers=1, audio=True, seed=2, mxfp8=True)
    items = fx.cache_items(W, mode="mxfp8-blocks")
    cache = tmp_path / "transformer.safetensors"
    fx.write_cache(cache, items, metadata={"transformer_cache_quantize": "mxfp8-blocks"})
    model = _model(layers=1, audio=True, fmt="mxfp8")
    loaded, n_layout, n_quant = load_transformer_cache(model, cache)
    n_block_linears = sum(fx.is_block_linear(b) for b in W["linears"])
    assert (loaded, n_layout, n_quant) == (len(items), 0, 2 * n_block_linears)
    blk = model.transformer_blocks[0]
    lin = W["linears"]
    for name in ("attn1", "audio_attn1"):
        a = getattr(blk, name)
        parts = [f"transformer_blocks.0.{name}.{p}" for p in ("to_q", "to_k", "to_v", "to_gate_logits")]
        np.testing.assert_array_equal(a.proj_q.w.numpy(), np.concatenate([lin[p]["codes"] for p in parts]))
        np.testing.assert_array_equal(a.proj_q.scale.numpy(), np.concatenate([lin[p]["scales"] for p in parts]))
        np.testing.assert_array_equal(a.proj_q.bias.numpy(), np.concatenate([lin[p]["b"] for p in parts]))
    for name in ("attn2", "audio_to_video_attn", "video_to_audio_attn"):
        a = getattr(blk, name)
        q = [f"transformer_blocks.0.{name}.{p}" for p in ("to_q", "to_gate_logits")]
        kv = [f"transformer_blocks.0.{name}.{p}" for p in ("to_k", "to_v")]
        np.testing.assert_array_equal(a.proj_q.w.numpy(), np.concatenate([lin[p]["codes"] for p in q]))
        np.testing.assert_array_equal(a.proj_kv.w.numpy(), np.concatenate([lin[p]["codes"] for p in kv]))
        np.testing.assert_array_equal(a.proj_kv.scale.numpy(), np.concatenate([lin[p]["scales"] for p in kv]))
        np.testing.assert_array_equal(a.to_out.w.numpy(), lin[f"transformer_blocks.0.{name}.to_out"]["codes"])
    np.testing.assert_array_equal(blk.ff.project_in.w.numpy(), lin["transformer_blocks.0.ff.project_in.proj"]["codes"])
    np.testing.assert_array_equal(blk.audio_ff.project_out.scale.numpy(),
                                  lin["transformer_blocks.0.audio_ff.project_out"]["scales"])
    assert all(w.kind == "mxfp8" and w.qlinear for w in blk.linear_weights())
    # top-level projections stay bf16 nn.Linear
    assert model.patchify_proj.kind == "bf16" and not model.patchify_proj.qlinear


def test_install_in_place_keeps_storage(tmp_path):
    """A resident weight of the same format and shape is overwritten in place
    (captured graphs keep valid addresses); a different format replaces it."""
    from ltx_amd.loader import load_transformer_cache

    W = _W(layers=1)
    cache = tmp_path / "transformer.safetensors"
    fx.write_cache(cache, fx.cache_items(W))
    model = _model(layers=1)
    a = model.transformer_blocks[0].attn1
    ptr_q, ptr_tab = a.proj_q.w.data_ptr(), model.video_tables.data_ptr()
    load_transformer_cache(model, cache)
    assert a.proj_q.w.data_ptr() == ptr_q and model.video_tables.data_ptr() == ptr_tab
    m8 = _model(layers=1, fmt="int8")
    with pytest.raises(ValueError, match="device tensor"):  # the quantiser is a HIP kernel: no CPU path
        load_transformer_cache(m8, cache, weight_format="int8")


def test_quant_mode_comes_from_metadata_or_argument(tmp_path):
    from ltx_amd.loader import load_transformer_cache

    W = _W(layers=1, mxfp8=True, seed=3)
    cache = tmp_path / "transformer.safetensors"
    fx.write_cache(cache, fx.cache_items(W, mode="mxfp8-blocks"))  # no metadata.json
    model = _model(layers=1, fmt="mxfp8")
    with pytest.raises(ValueError, match="Missing cached quantization mode"):
        load_transformer_cache(model, cache)
    load_transformer_cache(model, cache, transformer_cache_quantize="mxfp8-blocks")
    (tmp_path / "metadata.json").write_text(json.dumps({"transformer_cache_quantize": "mxfp8-blocks"}))
    load_transformer_cache(model, cache)
    # FF-only quantisation specs (transformer_cache.py:861-890): attention stays plain
    W2 = _W(layers=1, seed=5)
    items = fx.cache_items(W2)
    ff = "transformer_blocks.0.ff.project_out"
    codes = fx.random_codes(np.random.default_rng(0), W2["linears"][ff]["w"].shape)
    scales = np.full((codes.shape[0], codes.shape[1] // 32), 120, np.uint8)
    items = [it for it in items if it[0] != f"{ff}.weight"]
    items += [(f"__quant__.{ff}.weight", "U32", fx._pack_u32(codes)), (f"__quant__.{ff}.scales", "U8", scales)]
    c2 = tmp_path / "ff" / "transformer.safetensors"
    fx.write_cache(c2, items)
    m2 = _model(layers=1)
    load_transformer_cache(m2, c2, video_ff_quantize_specs=(("project_out", "mxfp8"),))
    po = m2.transformer_blocks[0].ff.project_out
    assert po.kind == "mxfp8" and po.qlinear and np.array_equal(po.w.numpy(), codes)
    assert m2.transformer_blocks[0].ff.project_in.kind == "bf16"
    with pytest.raises(ValueError, match="not a resident format"):
        load_transformer_cache(m2, c2, video_ff_quantize_specs=(("project_out", "mxfp4"),))


def test_install_errors_leave_model_untouched(tmp_path):
    from ltx_amd.loader import load_transformer_cache

    W = _W(layers=2)
    items = fx.cache_items(W)
    model = _model(layers=2)
    before = model.transformer_blocks[0].attn1.proj_q.w.fill_(0.5).clone()  # (empty storage may hold NaNs)

    def write(its, name):
        c = tmp_path / name / "transformer.safetensors"
        fx.write_cache(c, its)
        return c

    missing = [it for it in items if it[0] != "transformer_blocks.1.attn2.to_k.weight"]
    with pytest.raises(ValueError, match="missing, e.g. transformer_blocks.1.attn2.to_k.weight"):
        load_transformer_cache(model, write(missing, "missing"))
    extra = items + [("transformer_blocks.0.attn1.bogus", "BF16", np.zeros(4, np.float32))]
    with pytest.raises(ValueError, match="no place in the model, e.g. transformer_blocks.0.attn1.bogus"):
        load_transformer_cache(model, write(extra, "extra"))
    beyond = items + [("transformer_blocks.5.scale_shift_table", "BF16", np.zeros((9, 128), np.float32))]
    with pytest.raises(ValueError, match="block 5, but the model only has 2 blocks"):
        load_transformer_cache(model, write(beyond, "beyond"))
    bad = [(k, d, a[:, :-64] if k == "transformer_blocks.0.attn2.to_k.weight" else a) for k, d, a in items]
    with pytest.raises(ValueError, match=r"attn2.to_k.weight: shape \(N, K\) = \(128, 128\)"):
        load_transformer_cache(model, write(bad, "shape"))
    f32 = [(k, "F32" if k == "transformer_blocks.0.ff.project_in.proj.weight" else d, a) for k, d, a in items]
    with pytest.raises(ValueError, match="stored as F32"):
        load_transformer_cache(model, write(f32, "f32"))
    assert torch.equal(model.transformer_blocks[0].attn1.proj_q.w, before)
    # non-strict: the missing projection keeps its storage, the rest loads
    load_transformer_cache(model, tmp_path / "missing" / "transformer.safetensors", strict=False)
    np.testing.assert_array_equal(model.transformer_blocks[0].attn2.proj_kv.w.float().numpy()[:128],
                                  W["linears"]["transformer_blocks.0.attn2.to_k"]["w"])


def test_stock_checkpoint_bf16(tmp_path):
    """A stock checkpoint (PyTorch names, non-transformer keys beside them)."""
    from ltx_amd.loader import load_transformer_weights

    W = _W(layers=2, audio=True, seed=7)
    p = tmp_path / "ltx.safetensors"
    fx.write_safetensors(p, fx.checkpoint_items(W))
    model = _model(layers=2, audio=True)
    n = load_transformer_weights(model, p)
    assert n == len(W["linears"]) * 2 + len(W["vectors"])
    fx.check_against_named(model, W)
    # a video-only model skips every audio / AV key of the same checkpoint
    mv = _model(layers=2, audio=False)
    load_transformer_weights(mv, p)
    Wv = _W(layers=2, audio=False, seed=7)  # names of the video model only
    for base in Wv["linears"]:
        Wv["linears"][base] = W["linears"][base]
    for path in Wv["vectors"]:
        Wv["vectors"][path] = W["vectors"][path]
    fx.check_against_named(mv, Wv)


def test_build_writes_reference_metadata_last_and_atomically(tmp_path, monkeypatch):
    """build_transformer_cache on a stock bf16 checkpoint (mode off, host):
    metadata.json holds the reference's payload fields for such a build
    (loader/transformer_cache.py:453-514 -- schema version, source path /
    size / mtime_ns, audio flag, the four empty layout lists; no
    quantisation key when off), written last with no temporary file left; a
    rebuild deletes the old metadata.json before it writes any shard, so a
    build interrupted mid-way leaves no metadata beside partial shards."""
    import os

    from ltx_amd.loader import transformer_cache as tc

    W = _W(layers=2, audio=True, seed=3)
    ckpt = tmp_path / "ltx.safetensors"
    fx.write_safetensors(ckpt, fx.checkpoint_items(W))
    cache = tmp_path / "cache" / "transformer.safetensors"
    tc.build_transformer_cache(ckpt, cache, include_audio=True, device="cpu", shard_limit_bytes=1 << 16)
    meta_path = cache.parent / "metadata.json"
    meta = json.loads(meta_path.read_text())
    st = os.stat(ckpt)
    assert meta == {
        "schema_version": 1,
        "source": {"path": str(ckpt.resolve()), "size": st.st_size, "mtime_ns": st.st_mtime_ns},
        "include_audio": True,
        "video_ff_layout_specs": [], "video_ff_layout_layers": [],
        "video_attn_layout_specs": [], "video_attn_layout_layers": [],
    }
    assert not list(cache.parent.glob("*.tmp"))
    shards = tc.existing_cache_shards(cache)
    assert len(shards) >= 2
    # every shard is older than (or as old as) the metadata written after it
    assert all(s.stat().st_mtime_ns <= meta_path.stat().st_mtime_ns for s in shards)
    # the quantisation mode enters the payload when not off
    assert tc.cache_payload(ckpt, include_audio=False, transformer_cache_quantize="mxfp8-blocks") == {
        **{k: v for k, v in meta.items() if k != "include_audio"}, "include_audio": False,
        "transformer_cache_quantize": "mxfp8-blocks"}

    # a rebuild that fails at its second shard: the old metadata is gone already
    calls = {"n": 0}
    real_write = tc.write_safetensors

    def failing_write(path, items, **kw):
        calls["n"] += 1
        if calls["n"] == 2:
            raise OSError("disk full")
        return real_write(path, items, **kw)

    monkeypatch.setattr(tc, "write_safetensors", failing_write)
    with pytest.raises(OSError, match="disk full"):
        tc.build_transformer_cache(ckpt, cache, include_audio=True, device="cpu", shard_limit_bytes=1 << 16)
    assert not meta_path.exists()
    assert tc.read_cache_metadata(cache) is None
