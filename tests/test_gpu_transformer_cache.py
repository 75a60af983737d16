"""Checkpoint / transformer-cache loading through the HIP decoders and
encoders, and a denoise step of a model loaded from a reference-format cache.

* ``mxfp8-blocks-pretranspose`` caches (W^T quantised along N) decode exactly
  to bf16 and keep the quantised-linear arithmetic;
* FP8 E4M3 stock checkpoints (per-tensor ``weight_scale``) decode bit-exactly
  to the oracle's values; resident re-quantisation to MXFP8 / int8 gives the
  oracle encoders' codes;
* ``build_transformer_cache`` from a stock checkpoint, loaded back, equals the
  direct load (bf16, MXFP8, pretransposed MXFP8);
* end to end: an LTX-2.3 AV model at full width (1 block) loaded from a
  synthetic ``mxfp8-blocks`` cache with non-trivial biases, RMSNorm weights,
  tables and AdaLN MLPs runs one distilled step; the oracle runs the same step
  from the NAMED tensors of the cache (not from the loaded model), so any
  misplaced projection, norm, table or bias fails the cosine gate.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _cache_fixture as fx
from _util import cos_sim
from oracle import block as ob
from oracle import quant as oq
from oracle import rope as orope

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMALL = dict(vd=256, heads=32, ctx=192, ad=256, ah=32)  # 32 heads: gate rows quantise along N in groups of 32


def _small_model(layers=1, audio=True, fmt="bf16"):
    from ltx_amd.model.transformer.model import LTXModel

    return LTXModel(num_layers=layers, num_attention_heads=32, attention_head_dim=8, cross_attention_dim=192,
                    weight_format=fmt, audio=audio, init="empty", audio_attention_heads=32,
                    audio_attention_head_dim=8)


def _small_W(layers=1, audio=True, seed=0, mxfp8=False):
    s = SMALL
    return fx.synthetic_weights(layers, s["vd"], s["heads"], s["ctx"], audio, seed=seed, mxfp8_blocks=mxfp8,
                                ad=s["ad"], ah=s["ah"])


def _fused_parts(blk, i):
    """(LinearWeight, [named parts]) of every fused projection of block i."""
    out = []
    for name in ("attn1", "audio_attn1"):
        a = getattr(blk, name)
        out.append((a.proj_q, [f"transformer_blocks.{i}.{name}.{p}" for p in ("to_q", "to_k", "to_v",
                                                                          "to_gate_logits")]))
    for name in ("attn2", "audio_attn2", "audio_to_video_attn", "video_to_audio_attn"):
        a = getattr(blk, name)
        out.append((a.proj_q, [f"transformer_blocks.{i}.{name}.{p}" for p in ("to_q", "to_gate_logits")]))
        out.append((a.proj_kv, [f"transformer_blocks.{i}.{name}.{p}" for p in ("to_k", "to_v")]))
    for name in ("attn1", "attn2", "audio_attn1", "audio_attn2", "audio_to_video_attn", "video_to_audio_attn"):
        out.append((getattr(blk, name).to_out, [f"transformer_blocks.{i}.{name}.to_out"]))
    for ff in ("ff", "audio_ff"):
        f = getattr(blk, ff)
        out.append((f.project_in, [f"transformer_blocks.{i}.{ff}.project_in.proj"]))
        out.append((f.project_out, [f"transformer_blocks.{i}.{ff}.project_out"]))
    return out


def test_pretransposed_mxfp8_cache_decodes_exactly(tmp_path):
    from ltx_amd.kernels import gemm
    from ltx_amd.loader import load_transformer_cache

    print("pretranspose cache, small widths", flush=True)
    W = _small_W(seed=1)
    cache = tmp_path / "transformer.safetensors"
    items = fx.cache_items(W, mode="mxfp8-blocks-pretranspose")
    fx.write_cache(cache, items, shards=2, metadata={"transformer_cache_quantize": "mxfp8-blocks-pretranspose"})
    model = _small_model()
    load_transformer_cache(model, cache)
    blk = model.transformer_blocks[0]
    for lw, parts in _fused_parts(blk, 0):
        assert lw.kind == "bf16" and lw.qlinear
        want = np.concatenate([oq.mxfp8_dequantize(*oq.mxfp8_quantize(W["linears"][p]["w"].T.copy())).T
                               for p in parts])
        np.testing.assert_array_equal(gemm.dequantize(lw).float().cpu().numpy(), want, err_msg=parts[0])
        np.testing.assert_array_equal(lw.bias.cpu().numpy(), np.concatenate([W["linears"][p]["b"] for p in parts]))


def test_fp8_checkpoint_install_and_requantise(tmp_path):
    from ltx_amd.loader import load_transformer_weights

    print("fp8 checkpoint, small widths", flush=True)
    W = _small_W(seed=2)
    p = tmp_path / "ltx-fp8.safetensors"
    fx.write_safetensors(p, fx.checkpoint_items(W, fp8=True))  # W now holds the decoded values
    model = _small_model()
    load_transformer_weights(model, p)
    fx.check_against_named(model, W)
    assert all(w.kind == "bf16" and not w.qlinear for w in model.transformer_blocks[0].linear_weights())
    for fmt in ("mxfp8", "int8"):
        m = _small_model(fmt=fmt)
        load_transformer_weights(m, p, weight_format=fmt)
        for lw, parts in _fused_parts(m.transformer_blocks[0], 0):
            assert lw.kind == fmt and lw.qlinear == (fmt == "mxfp8")
            enc = [(oq.mxfp8_quantize if fmt == "mxfp8" else oq.int8_quantize)(W["linears"][q]["w"]) for q in parts]
            np.testing.assert_array_equal(lw.w.cpu().numpy().view(np.uint8),
                                          np.concatenate([e[0] for e in enc]).view(np.uint8), err_msg=parts[0])
            np.testing.assert_array_equal(lw.scale.cpu().numpy(), np.concatenate([e[1] for e in enc]))
        assert m.patchify_proj.kind == "bf16"


@pytest.mark.parametrize("mode", ["off", "mxfp8-blocks", "mxfp8-blocks-pretranspose"])
def test_build_cache_round_trip(tmp_path, mode):
    """Stock FP8 checkpoint -> build_transformer_cache -> load equals the
    direct load in the matching resident format."""
    from ltx_amd.loader import build_transformer_cache, load_transformer_cache, load_transformer_weights

    print(f"build cache mode={mode}", flush=True)
    W = _small_W(seed=3)
    p = tmp_path / "ltx.safetensors"
    fx.write_safetensors(p, fx.checkpoint_items(W, fp8=True))
    cache = tmp_path / "cache" / "transformer.safetensors"
    res = build_transformer_cache(p, cache, include_audio=True, transformer_cache_quantize=mode,
                                  shard_limit_bytes=1 << 20)
    assert res.loaded_count == len(W["linears"]) * 2 + len(W["vectors"])
    from ltx_amd.loader.transformer_cache import existing_cache_shards
    assert len(existing_cache_shards(cache)) > 1
    from_cache = _small_model(fmt="mxfp8" if mode == "mxfp8-blocks" else "bf16")
    load_transformer_cache(from_cache, cache)  # the mode comes from metadata.json
    if mode == "off":
        fx.check_against_named(from_cache, W)
        return
    direct = _small_model(fmt="mxfp8")
    load_transformer_weights(direct, p, weight_format="mxfp8")
    for (a, parts), (b, _) in zip(_fused_parts(from_cache.transformer_blocks[0], 0),
                                  _fused_parts(direct.transformer_blocks[0], 0)):
        assert a.qlinear and b.qlinear
        if mode == "mxfp8-blocks":
            assert torch.equal(a.w, b.w) and torch.equal(a.scale, b.scale), parts[0]
        else:
            want = np.concatenate([oq.mxfp8_dequantize(*oq.mxfp8_quantize(W["linears"][q]["w"].T.copy())).T
                                   for q in parts])
            np.testing.assert_array_equal(a.w.float().cpu().numpy(), want, err_msg=parts[0])
        assert torch.equal(a.bias, b.bias)


# -- end to end ----------------------------------------------------------------
def _oracle_weights(W, layers, qlinear_blocks):
    """Oracle-form weights straight from the named tensors."""
    lin, vec = W["linears"], W["vectors"]
    T = torch.from_numpy

    def lw(base):
        return T(lin[base]["w"]), T(lin[base]["b"])

    def mlp(name):
        d = {}
        for k, path in (("1", "emb.timestep_embedder.linear_1"), ("2", "emb.timestep_embedder.linear_2"),
                        ("", "linear")):
            d["w" + k], d["b" + k] = lw(f"{name}.{path}")
        return d

    blocks = []
    for i in range(layers):
        B = {}
        for a in ("attn1", "attn2", "audio_attn1", "audio_attn2", "audio_to_video_attn", "video_to_audio_attn"):
            pre = f"transformer_blocks.{i}.{a}"
            d = {}
            for p in ("to_q", "to_k", "to_v", "to_gate_logits", "to_out"):
                d[p], d[p + "_b"] = lw(f"{pre}.{p}")
                d[p + "_qlinear"] = qlinear_blocks
            d["q_norm"], d["k_norm"] = T(vec[f"{pre}.q_norm.weight"]), T(vec[f"{pre}.k_norm.weight"])
            B[a] = d
        for f in ("ff", "audio_ff"):
            pre = f"transformer_blocks.{i}.{f}"
            w1, b1 = lw(f"{pre}.project_in.proj")
            w2, b2 = lw(f"{pre}.project_out")
            B[f] = {"w1": w1, "b1": b1, "w2": w2, "b2": b2, "w1_qlinear": qlinear_blocks,
                    "w2_qlinear": qlinear_blocks}
        blocks.append(B)

    def tables(i, names):
        return T(np.concatenate([vec[f"transformer_blocks.{i}.{n}"] for n in names]))

    return {
        "patchify": lw("patchify_proj"), "audio_patchify": lw("audio_patchify_proj"),
        "mlps_v": [mlp(n) for n in ("adaln_single", "prompt_adaln_single", "av_ca_video_scale_shift_adaln_single",
                                    "av_ca_a2v_gate_adaln_single")],
        "mlps_a": [mlp(n) for n in ("audio_adaln_single", "audio_prompt_adaln_single",
                                    "av_ca_audio_scale_shift_adaln_single", "av_ca_v2a_gate_adaln_single")],
        "tables_v": torch.stack([tables(i, ("scale_shift_table", "prompt_scale_shift_table",
                                            "scale_shift_table_a2v_ca_video")) for i in range(layers)]),
        "tables_a": torch.stack([tables(i, ("audio_scale_shift_table", "audio_prompt_scale_shift_table",
                                            "scale_shift_table_a2v_ca_audio")) for i in range(layers)]),
        "blocks": blocks,
        "sst_out_v": T(vec["scale_shift_table"]), "proj_out_v": lw("proj_out"),
        "sst_out_a": T(vec["audio_scale_shift_table"]), "proj_out_a": lw("audio_proj_out"),
    }


def test_model_loaded_from_mxfp8_cache_matches_oracle_step(tmp_path):
    from ltx_amd.loader import load_transformer_cache
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.pipeline import DenoiseState, denoise_step

    print("end to end: full-width 1-block mxfp8-blocks cache", flush=True)
    W = fx.synthetic_weights(1, 4096, 32, 4096, True, seed=11, mxfp8_blocks=True)
    cache = tmp_path / "transformer.safetensors"
    fx.write_cache(cache, fx.cache_items(W, mode="mxfp8-blocks"), shards=2,
                   metadata={"transformer_cache_quantize": "mxfp8-blocks"})
    model = LTXModel(num_layers=1, weight_format="mxfp8", init="empty")
    loaded, _, quant = load_transformer_cache(model, cache)
    print(f"loaded {loaded} tensors ({quant} quantised)", flush=True)
    state = DenoiseState(model, height=128, width=192, frames=9, text_tokens=16, audio_frames=12, seed=5)
    vpos, apos = state.video_positions, state.audio_positions
    pes = tuple(tuple(torch.from_numpy(a) for a in p) for p in (
        orope.rope_tables(vpos, 4096, 32, orope.VIDEO_MAX_POS),
        orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS)))
    vlat, alat = state.video_latent.float().cpu(), state.audio_latent.float().cpu()
    vctx, actx = state.video_context.float().cpu(), state.audio_context.float().cpu()
    denoise_step(model, state, 0)
    torch.cuda.synchronize()
    MW = _oracle_weights(W, 1, qlinear_blocks=True)
    sig = state.sigmas
    ov, oa = ob.model_step(MW, vlat, alat, vctx, actx, sig[0], sig[1], pes)
    gv, ga = state.video_latent.float().cpu(), state.audio_latent.float().cpu()
    cv, ca = cos_sim(gv.numpy(), ov.numpy()), cos_sim(ga.numpy(), oa.numpy())
    # the step's change (x_next - x), which carries the velocity, must match too
    dv = cos_sim((gv - vlat).numpy(), (ov - vlat).numpy())
    da = cos_sim((ga - alat).numpy(), (oa - alat).numpy())
    print(f"video cos {cv:.6f} (delta {dv:.6f})  audio cos {ca:.6f} (delta {da:.6f})", flush=True)
    assert cv >= 0.999 and ca >= 0.999
    assert dv >= 0.999 and da >= 0.999
