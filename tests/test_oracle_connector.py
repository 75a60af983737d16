"""Pin the text-conditioning oracle (oracle/connector.py) and the connector's
host logic; CPU only."""

import numpy as np
import torch

from oracle import block as ob
from oracle import connector as oc
from oracle.bf16 import bf16r


def test_features_mask_scale_and_unit_rms(rng):
    L, T, D = 3, 7, 3840
    h = bf16r(rng.standard_normal((L, T, D)).astype(np.float32) * 5)
    mask = np.array([0, 1, 1, 0, 1, 1, 1])
    s = oc.aggregate_scale(4096, 3840)
    assert oc.bf16_value(s) == 1.03125 and oc.bf16_value(oc.aggregate_scale(2048, 3840)) == 0.73046875
    f = oc.gemma_features(h, mask, s)
    assert f.shape == (T, L * D)
    assert not f[[0, 3]].any()  # padding tokens are zero
    unscaled = oc.gemma_features(h, None, 1.0).reshape(T, L, D)
    ms = (unscaled.astype(np.float64) ** 2).mean(-1)
    assert np.all(np.abs(ms - 1.0) < 0.02)  # bf16 rounding of mean and rsqrt
    # layer-major: columns l*D .. (l+1)*D are layer l of the token
    one = oc.gemma_features(h[1:2], None, 1.0)
    np.testing.assert_array_equal(unscaled[:, 1, :], one)


def test_register_extension():
    regs = torch.arange(128 * 4, dtype=torch.float32).reshape(128, 4)
    x = -torch.ones(256, 4)
    y = oc.extend_with_registers(x, regs)
    assert y.shape == (1024, 4)
    assert torch.equal(y[:256], x)
    assert torch.equal(y[256], regs[0]) and torch.equal(y[1023], regs[127]) and torch.equal(y[300], regs[300 % 128])
    assert oc.extend_with_registers(torch.zeros(1100, 4), regs).shape == (1152, 4)
    assert oc.extend_with_registers(torch.zeros(1024, 4), regs).shape == (1024, 4)


def test_block_with_zero_output_projections_is_identity():
    g = torch.Generator().manual_seed(0)
    d, heads, dh = 128, 2, 64

    def lin(n, k, zero=False):
        w = torch.zeros(n, k) if zero else ob.bf(torch.randn(n, k, generator=g) * 0.1)
        return w, torch.zeros(n)

    a = {}
    for nm, (n, k) in {"to_q": (d, d), "to_k": (d, d), "to_v": (d, d), "to_gate_logits": (heads, d)}.items():
        a[nm], a[nm + "_b"] = lin(n, k)
    a["to_out"], a["to_out_b"] = lin(d, d, zero=True)
    a["q_norm"] = a["k_norm"] = torch.ones(d)
    ff = {}
    ff["w1"], ff["b1"] = lin(4 * d, d)
    ff["w2"], ff["b2"] = lin(d, 4 * d, zero=True)
    x = ob.bf(torch.randn(16, d, generator=g))
    y = oc.block1d({"attn1": a, "ff": ff}, x, None, heads)
    assert torch.equal(y, x)


def test_connector_lengths_and_host_register_extension():
    from ltx_amd.model.text_encoder.connector import Embeddings1DConnector

    c = Embeddings1DConnector(64, 2, num_layers=1, device="cpu", init="empty")
    c.learnable_registers = torch.arange(128 * 128, dtype=torch.float32).reshape(128, 128).bfloat16()
    assert [c.extended_length(t) for t in (1, 256, 1024, 1025, 1100)] == [1024, 1024, 1024, 1152, 1152]
    x = torch.zeros(300, 128, dtype=torch.bfloat16)
    y = c.append_learnable_registers(x)
    ref = oc.extend_with_registers(x.float(), c.learnable_registers.float())
    assert torch.equal(y.float(), ref)
