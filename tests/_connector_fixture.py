"""Synthetic LTX-2.3 text-connector / text-projection tensors under the stock
checkpoint's names (model/text_encoder/encoder.py:147-222, :409-434), written
from the reference's loader tables independently of the product's loader."""

from __future__ import annotations

import numpy as np

from oracle.bf16 import bf16r


def connector_tensors(rng, *, hidden_dim, num_gemma_layers, video_dim, video_heads, audio_dim, audio_heads, layers,
                      registers=128):
    """{checkpoint key: float32 array of bf16 values}; aggregate weights in the
    reference's column order (feature index d * num_gemma_layers + l)."""
    out = {}
    flat = hidden_dim * num_gemma_layers

    def put(key, shape, std):
        out[key] = bf16r((rng.standard_normal(shape) * std).astype(np.float32))

    for name, dim in (("video_aggregate_embed", video_dim), ("audio_aggregate_embed", audio_dim)):
        put(f"text_embedding_projection.{name}.weight", (dim, flat), 1.0 / np.sqrt(flat))
        put(f"text_embedding_projection.{name}.bias", (dim,), 0.05)
    for mod, dim, heads in (("video", video_dim, video_heads), ("audio", audio_dim, audio_heads)):
        pre = f"model.diffusion_model.{mod}_embeddings_connector."
        out[pre + "learnable_registers"] = bf16r(rng.uniform(-1, 1, (registers, dim)).astype(np.float32))
        for i in range(layers):
            b = f"{pre}transformer_1d_blocks.{i}."
            for p, n in (("to_q", dim), ("to_k", dim), ("to_v", dim), ("to_gate_logits", heads)):
                put(f"{b}attn1.{p}.weight", (n, dim), 1.0 / np.sqrt(dim))
                put(f"{b}attn1.{p}.bias", (n,), 0.05)
            put(f"{b}attn1.to_out.0.weight", (dim, dim), 1.0 / np.sqrt(dim))
            put(f"{b}attn1.to_out.0.bias", (dim,), 0.05)
            out[f"{b}attn1.q_norm.weight"] = bf16r((1 + 0.2 * rng.standard_normal(dim)).astype(np.float32))
            out[f"{b}attn1.k_norm.weight"] = bf16r((1 + 0.2 * rng.standard_normal(dim)).astype(np.float32))
            put(f"{b}ff.net.0.proj.weight", (4 * dim, dim), 1.0 / np.sqrt(dim))
            put(f"{b}ff.net.0.proj.bias", (4 * dim,), 0.05)
            put(f"{b}ff.net.2.weight", (dim, 4 * dim), 1.0 / np.sqrt(4 * dim))
            put(f"{b}ff.net.2.bias", (dim,), 0.05)
    return out


def oracle_connector_weights(T: dict, mod: str, layers: int):
    """Oracle-form (``oracle.connector.connector``) weights of one modality."""
    import torch

    pre = f"model.diffusion_model.{mod}_embeddings_connector."
    g = lambda k: torch.from_numpy(T[k])  # noqa: E731
    blocks = []
    for i in range(layers):
        b = f"{pre}transformer_1d_blocks.{i}."
        a = {}
        for p in ("to_q", "to_k", "to_v", "to_gate_logits"):
            a[p], a[p + "_b"] = g(f"{b}attn1.{p}.weight"), g(f"{b}attn1.{p}.bias")
        a["to_out"], a["to_out_b"] = g(f"{b}attn1.to_out.0.weight"), g(f"{b}attn1.to_out.0.bias")
        a["q_norm"], a["k_norm"] = g(f"{b}attn1.q_norm.weight"), g(f"{b}attn1.k_norm.weight")
        ff = {"w1": g(f"{b}ff.net.0.proj.weight"), "b1": g(f"{b}ff.net.0.proj.bias"),
              "w2": g(f"{b}ff.net.2.weight"), "b2": g(f"{b}ff.net.2.bias")}
        blocks.append({"attn1": a, "ff": ff})
    return {"registers": g(pre + "learnable_registers"), "blocks": blocks}
