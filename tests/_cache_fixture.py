"""Synthetic LTX-2.3 transformer weights under the reference's names, written
as the reference's files: stock PyTorch checkpoints (bf16 or FP8 E4M3 with
``weight_scale``) and transformer caches (plain / ``__layout__`` /
``__quant__`` MXFP8, single file or shards).

The parameter names and shapes are written out here from the reference's
module definitions (model/transformer/model.py:637-705,
transformer.py:192-284, attention.py:403-418, feed_forward.py:37-62,
timestep_embedding.py:95-184), independently of the product's loader, and the
PyTorch names from the checkpoint layout (``to_out.0``, ``ff.net.0.proj``,
``ff.net.2``, prefix ``model.diffusion_model.``, weight_converter.py:10-52).

Values are not Gaussian weights but are chosen to make every mapping mistake
visible: every tensor has its own distribution, biases and RMSNorm weights are
non-trivial, and MXFP8 codes/scales are drawn directly (random E4M3 codes of
moderate exponent, scales around 2^-log2(sqrt K)).
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

from oracle import quant as oq
from oracle.bf16 import bf16r

AUDIO_DIM, AUDIO_HEADS = 2048, 32  # the LTX-2.3 audio stream (32 heads x 64)
PATCH_CHANNELS = 128


def linear_shapes(num_layers: int, vd: int, heads: int, ctx: int, audio: bool, ad: int = AUDIO_DIM,
                  ah: int = AUDIO_HEADS) -> dict[str, tuple[int, int]]:
    """Module path -> (out, in) of every Linear of the transformer."""
    out: dict[str, tuple[int, int]] = {}

    def attn(prefix, q, kv, inner, h):
        out[f"{prefix}.to_q"] = (inner, q)
        out[f"{prefix}.to_k"] = (inner, kv)
        out[f"{prefix}.to_v"] = (inner, kv)
        out[f"{prefix}.to_gate_logits"] = (h, q)
        out[f"{prefix}.to_out"] = (q, inner)

    for i in range(num_layers):
        b = f"transformer_blocks.{i}"
        attn(f"{b}.attn1", vd, vd, vd, heads)
        attn(f"{b}.attn2", vd, ctx, vd, heads)
        out[f"{b}.ff.project_in.proj"] = (4 * vd, vd)
        out[f"{b}.ff.project_out"] = (vd, 4 * vd)
        if audio:
            attn(f"{b}.audio_attn1", ad, ad, ad, ah)
            attn(f"{b}.audio_attn2", ad, ad, ad, ah)
            out[f"{b}.audio_ff.project_in.proj"] = (4 * ad, ad)
            out[f"{b}.audio_ff.project_out"] = (ad, 4 * ad)
            attn(f"{b}.audio_to_video_attn", vd, ad, ad, ah)
            attn(f"{b}.video_to_audio_attn", ad, vd, ad, ah)
    out["patchify_proj"] = (vd, PATCH_CHANNELS)
    out["proj_out"] = (PATCH_CHANNELS, vd)
    mlps = [("adaln_single", vd, 9), ("prompt_adaln_single", vd, 2)]
    if audio:
        out["audio_patchify_proj"] = (ad, PATCH_CHANNELS)
        out["audio_proj_out"] = (PATCH_CHANNELS, ad)
        mlps += [("av_ca_video_scale_shift_adaln_single", vd, 4), ("av_ca_a2v_gate_adaln_single", vd, 1),
                 ("audio_adaln_single", ad, 9), ("audio_prompt_adaln_single", ad, 2),
                 ("av_ca_audio_scale_shift_adaln_single", ad, 4), ("av_ca_v2a_gate_adaln_single", ad, 1)]
    for name, d, n in mlps:
        out[f"{name}.emb.timestep_embedder.linear_1"] = (d, 256)
        out[f"{name}.emb.timestep_embedder.linear_2"] = (d, d)
        out[f"{name}.linear"] = (n * d, d)
    return out


def vector_shapes(num_layers: int, vd: int, audio: bool, ad: int = AUDIO_DIM) -> dict[str, tuple[int, ...]]:
    """Module path -> shape of the non-Linear parameters (tables, RMSNorm)."""
    out: dict[str, tuple[int, ...]] = {"scale_shift_table": (2, vd)}
    if audio:
        out["audio_scale_shift_table"] = (2, ad)
    for i in range(num_layers):
        b = f"transformer_blocks.{i}"
        out[f"{b}.scale_shift_table"] = (9, vd)
        out[f"{b}.prompt_scale_shift_table"] = (2, vd)
        attns = [("attn1", vd), ("attn2", vd)]
        if audio:
            out[f"{b}.audio_scale_shift_table"] = (9, ad)
            out[f"{b}.audio_prompt_scale_shift_table"] = (2, ad)
            out[f"{b}.scale_shift_table_a2v_ca_video"] = (5, vd)
            out[f"{b}.scale_shift_table_a2v_ca_audio"] = (5, ad)
            attns += [("audio_attn1", ad), ("audio_attn2", ad), ("audio_to_video_attn", ad),
                      ("video_to_audio_attn", ad)]
        for a, inner in attns:
            out[f"{b}.{a}.q_norm.weight"] = (inner,)
            out[f"{b}.{a}.k_norm.weight"] = (inner,)
    return out


def is_block_linear(base: str) -> bool:
    return base.startswith("transformer_blocks.")


def random_codes(rng, shape) -> np.ndarray:
    """E4M3 codes with exponent field 4..10 (|v| in [2^-3, 15]), random sign
    and mantissa; no NaN code."""
    e = rng.integers(4, 11, size=shape, dtype=np.uint8)
    m = rng.integers(0, 8, size=shape, dtype=np.uint8)
    s = rng.integers(0, 2, size=shape, dtype=np.uint8)
    return (s << 7) | (e << 3) | m


_E4M3 = oq.e4m3_decode_table()


def decode_mxfp8(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """``oracle.quant.mxfp8_dequantize`` in float32 arithmetic (the scale is a
    power of two, so the product is exact and has the E4M3 code's 4
    significant bits: no bf16 rounding happens); for large weights."""
    n, k = codes.shape
    f = np.ldexp(np.float32(1.0), scales.astype(np.int32) - 127).astype(np.float32)
    out = _E4M3[codes].reshape(n, k // 32, 32) * f[..., None]
    out = out.reshape(n, k)
    ref = oq.mxfp8_dequantize(codes[:4], scales[:4])  # spot check against the oracle's decode
    assert np.array_equal(out[:4], ref)
    return out


def synthetic_weights(num_layers: int, vd: int, heads: int, ctx: int, audio: bool, *, seed: int = 0,
                      mxfp8_blocks: bool = False, ad: int = AUDIO_DIM, ah: int = AUDIO_HEADS) -> dict:
    """{"linears": {base: {"w": f32 bf16 values (N, K) or None, "codes",
    "scales" (mxfp8), "b": f32 (N)}}, "vectors": {path: f32}}.

    With ``mxfp8_blocks`` the block linears get MXFP8 codes (N, K) and
    scales (N, K/32) and ``w`` holds their decoded values."""
    import torch

    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)

    def normal_bf16(shape, std):  # bf16 values as float32 (torch: fast for the 10^8-element MLP weights)
        return (torch.randn(shape, generator=gen) * std).bfloat16().float().numpy()

    lin = {}
    for base, (n, k) in linear_shapes(num_layers, vd, heads, ctx, audio, ad, ah).items():
        rec: dict = {"b": bf16r((rng.standard_normal(n) * 0.05).astype(np.float32))}
        if mxfp8_blocks and is_block_linear(base):
            codes = random_codes(rng, (n, k))
            base_exp = 127 - 3 - int(round(np.log2(np.sqrt(k))))
            scales = (base_exp + rng.integers(-1, 2, size=(n, k // 32))).astype(np.uint8)
            rec.update(codes=codes, scales=scales, w=decode_mxfp8(codes, scales))
        else:
            rec["w"] = normal_bf16((n, k), 1.0 / np.sqrt(k))
        lin[base] = rec
    vec = {}
    for path, shape in vector_shapes(num_layers, vd, audio, ad).items():
        if path.endswith("norm.weight"):
            v = 1.0 + 0.2 * rng.standard_normal(shape)
        else:
            v = 0.05 * rng.standard_normal(shape)
        vec[path] = bf16r(v.astype(np.float32))
    return {"linears": lin, "vectors": vec}


# -- writers -------------------------------------------------------------------
def _bf16_bits(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def write_safetensors(path: Path, items: list[tuple[str, str, np.ndarray]]) -> None:
    """``(key, safetensors dtype, array)``; BF16 arrays given as float32 values."""
    header, blobs, off = {}, [], 0
    for key, dt, arr in items:
        data = _bf16_bits(arr) if dt == "BF16" else np.ascontiguousarray(arr)
        blob = data.tobytes()
        header[key] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(blob)]}
        blobs.append(blob)
        off += len(blob)
    hb = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for blob in blobs:
            f.write(blob)


def _pack_u32(codes: np.ndarray) -> np.ndarray:
    """MLX packing of 8-bit codes: 4 per uint32 word, code j in bits [8j, 8j+8)
    (row blocks, to bound the temporaries of large weights)."""
    n = codes.shape[0]
    out = np.empty((n, codes.shape[1] // 4), dtype="<u4")
    for r in range(0, n, 1024):
        c = codes[r:r + 1024].astype(np.uint32).reshape(min(1024, n - r), -1, 4)
        out[r:r + 1024] = c[..., 0] | (c[..., 1] << 8) | (c[..., 2] << 16) | (c[..., 3] << 24)
    return out


def cache_items(W: dict, *, mode: str = "off", layout: tuple[str, ...] = ()) -> list[tuple[str, str, np.ndarray]]:
    """Reference cache entries.  ``mode``: "off" | "mxfp8-blocks" |
    "mxfp8-blocks-pretranspose" (block linears must carry codes for the
    mxfp8 modes; the pretranspose variant re-quantises W^T with the oracle
    encoder).  ``layout``: module paths stored as ``__layout__.<p>.weight_t``."""
    items = []
    for base, rec in W["linears"].items():
        items.append((f"{base}.bias", "BF16", rec["b"]))
        if mode != "off" and is_block_linear(base):
            if mode == "mxfp8-blocks":
                codes, scales = rec["codes"], rec["scales"]
            else:
                codes, scales = oq.mxfp8_quantize(rec["w"].T.copy())
            items.append((f"__quant__.{base}.weight", "U32", _pack_u32(codes)))
            items.append((f"__quant__.{base}.scales", "U8", scales))
        elif base in layout:
            items.append((f"__layout__.{base}.weight_t", "BF16", rec["w"].T.copy()))
        else:
            items.append((f"{base}.weight", "BF16", rec["w"]))
    for path, v in W["vectors"].items():
        items.append((path, "BF16", v))
    return items


def write_cache(cache_file: Path, items, *, shards: int = 1, metadata: dict | None = None) -> None:
    """Single ``transformer.safetensors`` or ``shards`` files
    ``transformer-NNNNN.safetensors`` beside it, plus ``metadata.json``."""
    cache_file = Path(cache_file)
    cache_file.parent.mkdir(parents=True, exist_ok=True)
    if shards <= 1:
        write_safetensors(cache_file, items)
    else:
        per = -(-len(items) // shards)
        for s in range(shards):
            write_safetensors(cache_file.with_name(f"{cache_file.stem}-{s:05d}{cache_file.suffix}"),
                              items[s * per:(s + 1) * per])
    if metadata is not None:
        (cache_file.parent / "metadata.json").write_text(json.dumps(metadata))


def pytorch_name(path: str) -> str:
    """Checkpoint key of a module path (the inverse of the reference's renames)."""
    p = path.replace(".to_out.", ".to_out.0.")
    p = p.replace("audio_ff.project_in.proj.", "audio_ff.net.0.proj.").replace("audio_ff.project_out.",
                                                                               "audio_ff.net.2.")
    if ".ff.project_in.proj." in p and ".audio_ff." not in p:
        p = p.replace(".ff.project_in.proj.", ".ff.net.0.proj.")
    if ".ff.project_out." in p and ".audio_ff." not in p:
        p = p.replace(".ff.project_out.", ".ff.net.2.")
    return "model.diffusion_model." + p


def checkpoint_items(W: dict, *, fp8: bool = False, rng_seed: int = 1, extra: bool = True):
    """A stock checkpoint.  With ``fp8`` the block linears are E4M3 codes with
    a per-tensor ``weight_scale`` (+ an ``input_scale`` to drop) and ``W`` is
    updated with the decoded values the loader must produce."""
    rng = np.random.default_rng(rng_seed)
    items = []
    for base, rec in W["linears"].items():
        key = pytorch_name(base + ".weight")
        if fp8 and is_block_linear(base):
            codes = random_codes(rng, rec["w"].shape)
            scale = np.float32(2.0 ** -6 * (1 + rng.random()))
            items.append((key, "F8_E4M3", codes))
            items.append((key + "_scale", "F32", np.array([scale], np.float32)))
            items.append((key[: -len(".weight")] + ".input_scale", "F32", np.array([0.5], np.float32)))
            rec["w"] = oq.fp8_checkpoint_dequant(codes, scale, out="bf16")
        else:
            items.append((key, "BF16", rec["w"]))
        items.append((pytorch_name(base + ".bias"), "BF16", rec["b"]))
    for path, v in W["vectors"].items():
        items.append((pytorch_name(path), "BF16", v))
    if extra:  # tensors that are not the transformer's
        items.append(("vae.decoder.conv_in.weight", "BF16", np.ones((4, 4), np.float32)))
        items.append(("model.diffusion_model.video_embeddings_connector.proj.weight", "BF16",
                      np.ones((8, 8), np.float32)))
    return items


def check_against_named(model, W):
    """Every resident tensor equals the named tensor it came from (decoded
    per its resident format; biases and tables as fp32)."""
    from _weights import block_weights, mlp_weights

    lin, vec = W["linears"], W["vectors"]
    for i, blk in enumerate(model.transformer_blocks):
        for name, a in block_weights(blk).items():
            pre = f"transformer_blocks.{i}.{name}"
            if name.endswith("ff"):
                np.testing.assert_array_equal(a["w1"].numpy(), lin[f"{pre}.project_in.proj"]["w"])
                np.testing.assert_array_equal(a["b1"].numpy(), lin[f"{pre}.project_in.proj"]["b"])
                np.testing.assert_array_equal(a["w2"].numpy(), lin[f"{pre}.project_out"]["w"])
                np.testing.assert_array_equal(a["b2"].numpy(), lin[f"{pre}.project_out"]["b"])
                continue
            for p in ("to_q", "to_k", "to_v", "to_gate_logits", "to_out"):
                np.testing.assert_array_equal(a[p].numpy(), lin[f"{pre}.{p}"]["w"], err_msg=f"{pre}.{p}")
                np.testing.assert_array_equal(a[p + "_b"].numpy(), lin[f"{pre}.{p}"]["b"], err_msg=f"{pre}.{p}")
            np.testing.assert_array_equal(a["q_norm"].numpy(), vec[f"{pre}.q_norm.weight"])
            np.testing.assert_array_equal(a["k_norm"].numpy(), vec[f"{pre}.k_norm.weight"])
        t = blk.video_tables.cpu().numpy()
        np.testing.assert_array_equal(t[0:9], vec[f"transformer_blocks.{i}.scale_shift_table"])
        np.testing.assert_array_equal(t[9:11], vec[f"transformer_blocks.{i}.prompt_scale_shift_table"])
        if model.audio_config is not None:
            np.testing.assert_array_equal(t[11:16], vec[f"transformer_blocks.{i}.scale_shift_table_a2v_ca_video"])
            a = blk.audio_tables.cpu().numpy()
            np.testing.assert_array_equal(a[0:9], vec[f"transformer_blocks.{i}.audio_scale_shift_table"])
            np.testing.assert_array_equal(a[9:11], vec[f"transformer_blocks.{i}.audio_prompt_scale_shift_table"])
            np.testing.assert_array_equal(a[11:16], vec[f"transformer_blocks.{i}.scale_shift_table_a2v_ca_audio"])
    tops = [("patchify_proj", model.patchify_proj), ("proj_out", model.proj_out)]
    mlps = ["adaln_single", "prompt_adaln_single"]
    if model.audio_config is not None:
        tops += [("audio_patchify_proj", model.audio_patchify_proj), ("audio_proj_out", model.audio_proj_out)]
        mlps += ["av_ca_video_scale_shift_adaln_single", "av_ca_a2v_gate_adaln_single", "audio_adaln_single",
                 "audio_prompt_adaln_single", "av_ca_audio_scale_shift_adaln_single", "av_ca_v2a_gate_adaln_single"]
        np.testing.assert_array_equal(model.audio_scale_shift_table.cpu().numpy(), vec["audio_scale_shift_table"])
    for name, lw in tops:
        np.testing.assert_array_equal(lw.w.float().cpu().numpy(), lin[name]["w"])
        np.testing.assert_array_equal(lw.bias.cpu().numpy(), lin[name]["b"])
    np.testing.assert_array_equal(model.scale_shift_table.cpu().numpy(), vec["scale_shift_table"])
    for name in mlps:
        m = mlp_weights(getattr(model, name))
        for k, path in (("w1", "emb.timestep_embedder.linear_1"), ("w2", "emb.timestep_embedder.linear_2"),
                        ("w", "linear")):
            np.testing.assert_array_equal(m[k].numpy(), lin[f"{name}.{path}"]["w"], err_msg=f"{name}.{path}")
            np.testing.assert_array_equal(m["b" + k[1:]].numpy(), lin[f"{name}.{path}"]["b"])
