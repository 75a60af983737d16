"""Pin the weight-format oracle (E4M3, MXFP8, int8) and the GEMM oracle."""

import numpy as np
import pytest
import torch

from oracle import quant as oq
from oracle.bf16 import bf16r


def test_e4m3_table_matches_torch_and_known_answer():
    table = oq.e4m3_decode_table()
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(table)
    assert nan.sum() == 2 and np.isnan(codes[nan]).all()
    np.testing.assert_array_equal(table[~nan], codes[~nan])
    # reference known answer: byte 0x38 -> 1.0; x weight_scale 2.0 -> 2.0
    # (tests/test_transformer_cache.py:64-95)
    assert table[0x38] == 1.0 and table[0x38] * np.float32(2.0) == 2.0
    assert table[0x7E] == 448.0 and table[0x01] == 2.0 ** -9


def test_e4m3_encode_brute_force(rng):
    table = oq.e4m3_decode_table().astype(np.float64)
    finite = ~np.isnan(table)
    vals = np.concatenate([
        rng.standard_normal(4000) * np.exp2(rng.uniform(-12, 9, 4000)),
        table[finite],                                     # exact codes
        (table[finite][:-1] + table[finite][1:]) / 2.0,     # midpoints (ties)
        np.array([500.0, -1e6, 449.0, 464.0, 470.0]),
    ])
    codes = oq.e4m3_encode(vals)
    got = table[codes]
    for v, g, c in zip(vals, got, codes):
        a = min(abs(v), 448.0)
        cand = table[:0x7F]
        d = np.abs(cand - a)
        best = np.flatnonzero(d == d.min())
        want = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
        assert (c & 0x7F) == want, (v, c, want)
        assert (v < 0) == bool(c & 0x80) or a == 0


def test_torch_cast_agrees_inside_range(rng):
    # torch's float8_e4m3fn cast is RNE; inside +-448 it must agree exactly
    v = (rng.standard_normal(20000) * 40).clip(-448, 448).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(oq.e4m3_encode(v), ref)


def test_mxfp8_scale_rule_and_roundtrip(rng):
    W = bf16r(rng.standard_normal((8, 256)).astype(np.float32) * 0.02)
    codes, scales = oq.mxfp8_quantize(W)
    deq = oq.mxfp8_dequantize(codes, scales)
    blocks = np.abs(W.reshape(8, 8, 32)).max(-1)
    X = scales.astype(np.int64) - 127
    # 2^(X+8) <= amax < 2^(X+9): the block max lands in the top binade
    assert np.all(np.exp2(X + 8.0) <= blocks) and np.all(blocks < np.exp2(X + 9.0))
    # error: at most half a step of the top binade (2^(X+8) * 2^-4), except
    # that OCP's scale lets amax/2^X reach [448, 512), which saturates to 448
    err = np.abs(deq - W).reshape(8, 8, 32).max(-1)
    bound = np.maximum(np.exp2(X + 8.0 - 4.0), blocks - 448.0 * np.exp2(X))
    assert np.all(err <= bound + 1e-30)
    # a block whose values are exactly representable round-trips exactly
    exact = np.zeros((1, 32), np.float32)
    exact[0, :8] = [1.0, -2.0, 0.5, 448.0, -0.015625, 3.0, 0.0, 256.0]
    c, s = oq.mxfp8_quantize(exact)
    np.testing.assert_array_equal(oq.mxfp8_dequantize(c, s), exact)
    assert s[0, 0] == 127  # amax 448 -> X = 8 - 8 = 0
    # zero block
    c, s = oq.mxfp8_quantize(np.zeros((1, 32), np.float32))
    assert s[0, 0] == 0 and not c.any()


def test_int8_brute_force(rng):
    W = bf16r(rng.standard_normal((16, 64)).astype(np.float32) * 0.02)
    W[3] = 0.0
    q, s = oq.int8_quantize(W)
    assert s[3] == 0 and not q[3].any()
    assert np.all(np.abs(q) <= 127) and np.all(np.abs(q).max(-1)[s > 0] == 127)
    for r in range(16):
        if s[r] == 0:
            continue
        t = W[r].astype(np.float64) / float(s[r])  # exact quotient
        # q is one of the two integers around w/s, the nearest one unless the
        # quotient is within fp32 division error of a half-way point
        assert np.all((q[r] == np.floor(t)) | (q[r] == np.ceil(t)))
        frac = np.abs(t - np.floor(t))
        clear = np.abs(frac - 0.5) > 1e-5
        assert np.all(q[r][clear] == np.round(t[clear]))
    deq = oq.int8_dequantize(q, s)
    np.testing.assert_array_equal(deq, bf16r((q.astype(np.float32) * s[:, None]).astype(np.float32)))


@pytest.mark.parametrize("epi", ["bias", "gelu", "sigmoid2", "residual", "residual_round"])
def test_linear_oracle_against_float64_loops(rng, epi):
    x = bf16r(rng.standard_normal((5, 64)).astype(np.float32))
    W = bf16r(rng.standard_normal((24, 64)).astype(np.float32) * 0.1)
    b = rng.standard_normal(24).astype(np.float32)
    res = bf16r(rng.standard_normal((5, 24)).astype(np.float32))
    g = rng.standard_normal(24).astype(np.float32)
    out = oq.linear(x, W, b, epilogue=epi, residual=res, gate=g, exact=True)
    for i in range(5):
        for j in range(24):
            acc = sum(float(x[i, k]) * float(W[j, k]) for k in range(64)) + float(b[j])
            y = float(bf16r(np.float32(acc)))
            if epi == "gelu":
                import math
                y = 0.5 * y * (1 + math.tanh(math.sqrt(2 / math.pi) * (y + 0.044715 * y ** 3)))
            elif epi == "sigmoid2":
                import math
                y = 2.0 * float(bf16r(np.float32(1 / (1 + math.exp(-y)))))
            elif epi == "residual":
                y = float(res[i, j]) + float(g[j]) * y
            elif epi == "residual_round":
                y = float(res[i, j]) + float(bf16r(np.float32(float(g[j]) * y)))
            assert out[i, j] == bf16r(np.float32(y)), (i, j)


def test_linear_oracle_quantized_linear_form_matches_torch_bf16_add(rng):
    """nn.QuantizedLinear's ``quantized_matmul(x, w) + bias``: the product is a
    bf16 tensor and the bias add is a bf16 add (transformer_cache.py:177-193).
    torch's bfloat16 add rounds the same way, so it checks the form."""
    x = bf16r(rng.standard_normal((16, 64)).astype(np.float32))
    W = bf16r(rng.standard_normal((40, 64)).astype(np.float32) * 0.1)
    b = bf16r(rng.standard_normal(40).astype(np.float32))
    out = oq.linear(x, W, b, exact=True, round_then_bias=True)
    prod = torch.from_numpy(x).double() @ torch.from_numpy(W).double().T
    ref = (prod.float().bfloat16() + torch.from_numpy(b).bfloat16()).float().numpy()
    np.testing.assert_array_equal(out, ref)
    # and it differs from the single-rounding addmm form somewhere
    single = oq.linear(x, W, b, exact=True)
    assert (single != out).any()
