"""Pin the attention oracle: brute-force float64 loops and softmax invariants."""

import math

import numpy as np

from oracle.attention import attention
from oracle.bf16 import bf16r


def test_against_bruteforce_loops(rng):
    heads, dh, tq, tk = 2, 8, 5, 7
    q = bf16r(rng.standard_normal((tq, heads * dh)).astype(np.float32))
    k = bf16r(rng.standard_normal((tk, heads * dh)).astype(np.float32))
    v = bf16r(rng.standard_normal((tk, heads * dh)).astype(np.float32))
    g = bf16r(rng.uniform(0, 2, (tq, heads)).astype(np.float32))
    out = attention(q, k, v, heads, gate=g, exact=True)
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        for i in range(tq):
            s = [sum(float(q[i, sl][c]) * float(k[j, sl][c]) for c in range(dh)) / math.sqrt(dh) for j in range(tk)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            o = [sum(w[j] * float(v[j, sl][c]) for j in range(tk)) / z for c in range(dh)]
            ref = bf16r(bf16r(np.array(o, np.float32)) * g[i, h])
            np.testing.assert_array_equal(out[i, sl], ref)


def test_identical_keys_average_values(rng):
    heads, dh, tq, tk = 1, 16, 3, 9
    q = bf16r(rng.standard_normal((tq, dh)).astype(np.float32))
    k = np.tile(bf16r(rng.standard_normal((1, dh)).astype(np.float32)), (tk, 1))
    v = bf16r(rng.standard_normal((tk, dh)).astype(np.float32))
    out = attention(q, k, v, heads, exact=True)
    np.testing.assert_array_equal(out, np.tile(bf16r(v.astype(np.float64).mean(0).astype(np.float32)), (tq, 1)))


def test_dominant_key_selects_its_value(rng):
    dh, tk = 16, 6
    q = np.zeros((1, dh), np.float32)
    q[0, 0] = 64.0
    k = np.zeros((tk, dh), np.float32)
    k[3, 0] = 64.0  # score 64*64/4 = 1024 vs 0 elsewhere
    v = bf16r(rng.standard_normal((tk, dh)).astype(np.float32))
    out = attention(q, k, v, 1, exact=True)
    np.testing.assert_array_equal(out[0], v[3])
