"""Text-connector weight loading on the host: every tensor of a synthetic
stock checkpoint lands in its fused / permuted place."""

import numpy as np
import pytest
import torch

import _cache_fixture as fx
import _connector_fixture as cf


def _make(tmp_path, rng, layers=2):
    T = cf.connector_tensors(rng, hidden_dim=64, num_gemma_layers=3, video_dim=128, video_heads=2, audio_dim=64,
                             audio_heads=2, layers=layers, registers=16)
    T["model.diffusion_model.transformer_blocks.0.attn1.to_q.weight"] = np.zeros((2, 2), np.float32)  # not ours
    p = tmp_path / "ckpt.safetensors"
    fx.write_safetensors(p, [(k, "BF16", v) for k, v in T.items()])
    return T, p


def _model(layers=2):
    from ltx_amd.model.text_encoder.encoder import create_av_text_connector_v2

    return create_av_text_connector_v2(hidden_dim=64, num_gemma_layers=3, video_inner_dim=128, audio_inner_dim=64,
                                       video_connector_heads=2, video_connector_head_dim=64,
                                       audio_connector_heads=2, audio_connector_head_dim=32,
                                       connector_layers=layers, num_registers=16, device="cpu", init="empty")


def test_connector_weights_land_in_place(tmp_path, rng):
    from ltx_amd.loader.text_connector import load_av_text_connector_weights

    T, p = _make(tmp_path, rng)
    m = _model()
    n = load_av_text_connector_weights(m, p)
    assert n == len(T) - 1
    fe = m.feature_extractor
    w = T["text_embedding_projection.video_aggregate_embed.weight"]  # columns d*L + l
    got = fe.video_aggregate_embed.w.float().numpy()                  # columns l*D + d
    for l in range(3):
        for d in (0, 17, 63):
            np.testing.assert_array_equal(got[:, l * 64 + d], w[:, d * 3 + l])
    np.testing.assert_array_equal(fe.audio_aggregate_embed.bias.numpy(),
                                  T["text_embedding_projection.audio_aggregate_embed.bias"])
    for mod, c in (("video", m.embeddings_connector), ("audio", m.audio_embeddings_connector)):
        pre = f"model.diffusion_model.{mod}_embeddings_connector."
        np.testing.assert_array_equal(c.learnable_registers.float().numpy(), T[pre + "learnable_registers"])
        for i, blk in enumerate(c.transformer_1d_blocks):
            b = f"{pre}transformer_1d_blocks.{i}."
            q = np.concatenate([T[f"{b}attn1.{x}.weight"] for x in ("to_q", "to_k", "to_v", "to_gate_logits")])
            np.testing.assert_array_equal(blk.attn1.proj_q.w.float().numpy(), q)
            qb = np.concatenate([T[f"{b}attn1.{x}.bias"] for x in ("to_q", "to_k", "to_v", "to_gate_logits")])
            np.testing.assert_array_equal(blk.attn1.proj_q.bias.numpy(), qb)
            np.testing.assert_array_equal(blk.attn1.to_out.w.float().numpy(), T[f"{b}attn1.to_out.0.weight"])
            np.testing.assert_array_equal(blk.attn1.q_norm.numpy(), T[f"{b}attn1.q_norm.weight"])
            np.testing.assert_array_equal(blk.attn1.k_norm.numpy(), T[f"{b}attn1.k_norm.weight"])
            np.testing.assert_array_equal(blk.ff.project_in.w.float().numpy(), T[f"{b}ff.net.0.proj.weight"])
            np.testing.assert_array_equal(blk.ff.project_out.bias.numpy(), T[f"{b}ff.net.2.bias"])


def test_connector_weights_missing_and_extra(tmp_path, rng):
    from ltx_amd.loader.text_connector import load_av_text_connector_weights

    T, p = _make(tmp_path, rng, layers=2)
    with pytest.raises(ValueError, match="no place in the connector"):
        load_av_text_connector_weights(_model(layers=1), p)  # block 1 tensors have no place
    with pytest.raises(ValueError, match="missing"):
        load_av_text_connector_weights(_model(layers=3), p)
