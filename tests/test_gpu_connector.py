"""Text conditioning on the GPU: the Gemma feature normalisation kernel
against the oracle, and the connectors / full encode_from_hidden_states of a
model loaded from a synthetic stock checkpoint against the oracle run from the
checkpoint's named tensors (model/text_encoder/connector.py,
feature_extractor.py, encoder.py:80-122)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _cache_fixture as fx
import _connector_fixture as cf
from _util import cos_sim, max_rel_err, ulp_diff_bf16
from oracle import block as ob
from oracle import connector as oc
from oracle import rope as orope
from oracle.bf16 import bf16r

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("L,T", [(3, 37), (49, 4)])
def test_gemma_features_kernel(L, T):
    from ltx_amd import _lib

    print(f"gemma features L={L} T={T}", flush=True)
    rng = np.random.default_rng(L * 100 + T)
    D = 3840
    h = bf16r(rng.standard_normal((L, T, D)).astype(np.float32) * rng.uniform(0.1, 30, (L, T, 1)).astype(np.float32))
    mask = (rng.random(T) > 0.3).astype(np.int32)
    mask[0] = 1
    hd = torch.from_numpy(h).to(DEV).bfloat16()
    md = torch.from_numpy(mask).to(DEV)
    sv, sa = oc.bf16_value(oc.aggregate_scale(4096, D)), oc.bf16_value(oc.aggregate_scale(2048, D))
    fv = torch.empty((T, L * D), dtype=torch.bfloat16, device=DEV)
    fa = torch.empty_like(fv)
    _lib.call("ltx_gemma_features_bf16", hd.data_ptr(), L, T, D, T * D, D, md.data_ptr(), oc.bf16_value(1e-6), sv,
              sa, fv.data_ptr(), fa.data_ptr(), L * D, _lib.stream_of(hd))
    torch.cuda.synchronize()
    for got, s in ((fv, oc.aggregate_scale(4096, D)), (fa, oc.aggregate_scale(2048, D))):
        ref = oc.gemma_features(h, mask, s)
        g = got.float().cpu().numpy()
        ulps = ulp_diff_bf16(g, ref)
        # the fp32 sum of squares is summed in another order than the oracle's:
        # a row whose mean lands on a bf16 rounding boundary may differ by an ulp
        rows_exact = (ulps.reshape(T, L, D).max(-1) == 0).mean()
        print(f"  exact rows {rows_exact:.4f}, max ulp {ulps.max()}", flush=True)
        assert rows_exact >= 0.97 and ulps.max() <= 2
        assert not g[mask == 0].any()


def _write_ckpt(tmp_path, T):
    p = tmp_path / "ltx-text.safetensors"
    fx.write_safetensors(p, [(k, "BF16", v) for k, v in T.items()])
    return p


def test_connectors_match_oracle(tmp_path):
    """Full-width connectors (video 32x128, audio 32x64), 2 layers, 256 input
    tokens extended by registers to 1024.  Gate: the block gate (normwise max
    relative error 1e-2) per stacked layer, cosine >= 0.9999."""
    from ltx_amd.loader.text_connector import load_av_text_connector_weights
    from ltx_amd.model.text_encoder.encoder import create_av_text_connector_v2

    print("connectors full width, 2 layers", flush=True)
    rng = np.random.default_rng(7)
    layers = 2
    T = cf.connector_tensors(rng, hidden_dim=64, num_gemma_layers=1, video_dim=4096, video_heads=32,
                             audio_dim=2048, audio_heads=32, layers=layers)
    m = create_av_text_connector_v2(hidden_dim=64, num_gemma_layers=1, connector_layers=layers, init="empty")
    load_av_text_connector_weights(m, _write_ckpt(tmp_path, T))
    for mod, c, dim in (("video", m.embeddings_connector, 4096), ("audio", m.audio_embeddings_connector, 2048)):
        x = bf16r(rng.standard_normal((256, dim)).astype(np.float32))
        out, mask = c(torch.from_numpy(x).to(DEV).bfloat16()[None])
        torch.cuda.synchronize()
        assert out.shape == (1, 1024, dim) and not mask.any()
        idx = np.arange(1024, dtype=np.float32)
        pe = tuple(torch.from_numpy(a) for a in orope.rope_tables(np.stack([idx, idx], -1)[None, None], dim, 32, [1]))
        # the product's RoPE tables equal the oracle's bit for bit
        assert all(torch.equal(g.cpu(), o) for g, o in zip(c.rope(1024), pe))
        ref = oc.connector(cf.oracle_connector_weights(T, mod, layers), torch.from_numpy(x), pe, heads=32)
        got = out[0].float().cpu().numpy()
        err, cs = max_rel_err(got, ref.numpy()), cos_sim(got, ref.numpy())
        print(f"  {mod}: max_rel_err={err:.3e} cos={cs:.6f}", flush=True)
        # the bf16 gate of one block (1e-2 normwise) per stacked layer
        assert err <= 1e-2 * layers and cs >= 0.9999


def test_encode_from_hidden_states_matches_oracle(tmp_path):
    """Feature extractor (4 Gemma layers of 3840, 64 tokens with left padding)
    + 1-layer connectors, against the oracle composed from the named tensors."""
    from ltx_amd.loader.text_connector import load_av_text_connector_weights
    from ltx_amd.model.text_encoder.encoder import create_av_text_connector_v2

    print("encode_from_hidden_states", flush=True)
    rng = np.random.default_rng(9)
    Lg, D, Tt = 4, 3840, 64
    T = cf.connector_tensors(rng, hidden_dim=D, num_gemma_layers=Lg, video_dim=4096, video_heads=32,
                             audio_dim=2048, audio_heads=32, layers=1)
    m = create_av_text_connector_v2(hidden_dim=D, num_gemma_layers=Lg, connector_layers=1, init="empty")
    load_av_text_connector_weights(m, _write_ckpt(tmp_path, T))
    hidden = bf16r(rng.standard_normal((Lg, Tt, D)).astype(np.float32) * 3)
    mask = np.ones(Tt, np.int32)
    mask[:10] = 0  # left padding
    out = m.encode_from_hidden_states([torch.from_numpy(hidden[l]).to(DEV).bfloat16()[None] for l in range(Lg)],
                                      torch.from_numpy(mask)[None].to(DEV))
    torch.cuda.synchronize()
    assert out.video_encoding.shape == (1, 1024, 4096) and out.audio_encoding.shape == (1, 1024, 2048)
    assert out.attention_mask.shape == (1, 1024) and bool(out.attention_mask.all())
    idx = np.arange(1024, dtype=np.float32)
    for mod, dim, enc in (("video", 4096, out.video_encoding), ("audio", 2048, out.audio_encoding)):
        w = torch.from_numpy(T[f"text_embedding_projection.{mod}_aggregate_embed.weight"])
        b = torch.from_numpy(T[f"text_embedding_projection.{mod}_aggregate_embed.bias"])
        feats = oc.gemma_features(hidden, mask, oc.aggregate_scale(dim, D))  # layer-major
        # the reference's column order is d*L + l: permute the features to it
        feats_ref = torch.from_numpy(feats.reshape(Tt, Lg, D).transpose(0, 2, 1).reshape(Tt, D * Lg).copy())
        x = ob.linear(feats_ref, w, b)
        pe = tuple(torch.from_numpy(a) for a in orope.rope_tables(np.stack([idx, idx], -1)[None, None], dim, 32, [1]))
        ref = oc.connector(cf.oracle_connector_weights(T, mod, 1), x, pe, heads=32)
        got = enc[0].float().cpu().numpy()
        err, cs = max_rel_err(got, ref.numpy()), cos_sim(got, ref.numpy())
        print(f"  {mod}: max_rel_err={err:.3e} cos={cs:.6f}", flush=True)
        # 1e-2 per stage: the bf16 projection and one connector layer
        assert err <= 2e-2 and cs >= 0.9999
