"""GPU parity of the one-launch few-row GEMM (ltx_gemm_rows_*).

* In-GEMM dequantisation: bit-exact, shown with A = [I 0] / [0 I] row blocks
  over two splits (each output is one product 1.0 * w' plus exact zeros, and
  the split sum adds exact zeros), for every weight format.
* Every epilogue x format on the audio stream's shapes (68 and 121 rows, the
  fused QKV + gate columns) against the fp32-accumulating oracle: normwise
  max relative error <= 1e-2, cosine >= 0.9999, >= 85 % of outputs
  bit-identical; and against the single-pass tile kernel.
* The split sum is deterministic: repeated calls, interleaved with other
  launches, give identical bits; the ticket counters are left at zero.
* A captured HIP graph of the calls replays to the eager result.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import bf16_from_torch, cos_sim, max_rel_err, ulp_diff_bf16
from oracle import quant as oq
from oracle.bf16 import bf16r

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPIS = ["bias", "gelu", "sigmoid2", "residual", "residual_round"]


def _bf(rng, shape, scale=1.0):
    return bf16r(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


def _t(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def _decoded(kind, W):
    if kind == "bf16":
        return W
    if kind == "int8":
        return oq.int8_dequantize(*oq.int8_quantize(W))
    return oq.mxfp8_dequantize(*oq.mxfp8_quantize(W))


def _codes(gemm):
    return {"bias": gemm.EPI_BIAS, "gelu": gemm.EPI_GELU, "sigmoid2": gemm.EPI_SIGMOID2,
            "residual": gemm.EPI_RESIDUAL, "residual_round": gemm.EPI_RESIDUAL_ROUND}


@pytest.mark.parametrize("kind", ["bf16", "int8", "mxfp8"])
@pytest.mark.parametrize("N", [256, 520])
def test_rows_identity_returns_decoded_weight(kind, N):
    """x = [I 0] and [0 I] (128 rows each, K = 256) over two splits of 128:
    C = x @ W'^T is the decoded weight's left / right half, transposed."""
    from ltx_amd.kernels import gemm

    rng = np.random.default_rng(N + len(kind))
    K = 256
    W = bf16r(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.02))
    W[1] = 0.0
    W[2, :64] = bf16r(np.linspace(-3, 3, 64, dtype=np.float32))
    W[5] = bf16r(np.logspace(-6, 2, K, dtype=np.float32) * np.sign(rng.standard_normal(K)).astype(np.float32))
    wt = gemm.make_weight(_t(W), kind=kind)
    deq = bf16_from_torch(gemm.dequantize(wt))
    eye = torch.eye(128, dtype=torch.bfloat16, device=DEV)
    zero = torch.zeros((128, 128), dtype=torch.bfloat16, device=DEV)
    for half, x in enumerate((torch.cat([eye, zero], 1), torch.cat([zero, eye], 1))):
        print(f"rows identity {kind} N={N} half={half}", flush=True)
        out = gemm.linear_rows(x.contiguous(), wt, splits=2 if kind != "bf16" else 4)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bf16_from_torch(out), deq[:, 128 * half:128 * (half + 1)].T)


@pytest.mark.parametrize("kind", ["bf16", "int8", "mxfp8"])
@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("M,K,N", [(68, 2048, 6176), (68, 8192, 2048), (121, 2048, 8192), (1, 4096, 1024),
                                   (100, 2048, 2080), (33, 1024, 520)])
def test_rows_epilogues(kind, epi, M, K, N):
    """Every epilogue with a non-zero bias (the quantised-linear rounding for
    MXFP8), the head-gate columns of a fused projection for the bias form, in
    place on the residual for the gated forms; automatic split count."""
    from ltx_amd.kernels import gemm

    print(f"rows {kind} {epi} M={M} K={K} N={N} splits={gemm.rows_splits(M, N, K, kind)}", flush=True)
    rng = np.random.default_rng(M + K + N + len(epi))
    x = _bf(rng, (M, K))
    W = _bf(rng, (N, K), 0.02)
    b = bf16r(rng.standard_normal(N).astype(np.float32) * 0.1)
    res = _bf(rng, (M, N))
    g = rng.standard_normal(N).astype(np.float32) * 0.5
    wt = gemm.make_weight(_t(W), _t(b, torch.float32), kind=kind)
    sig = N - 32 if epi == "bias" else None
    code = _codes(gemm)[epi]

    def run(rows):
        if epi.startswith("residual"):
            rt = _t(res)
            if rows:
                o = gemm.linear_rows(_t(x), wt, epilogue=code, out=rt, residual=rt, gate=_t(g, torch.float32))
                assert o.data_ptr() == rt.data_ptr()
                return o
            return gemm.linear(_t(x), wt, epilogue=code, out=rt, residual=rt, gate=_t(g, torch.float32), splits=1)
        if rows:
            return gemm.linear_rows(_t(x), wt, epilogue=code, sigmoid_from=sig)
        return gemm.linear(_t(x), wt, epilogue=code, sigmoid_from=sig, splits=1)

    got, single = bf16_from_torch(run(True)), bf16_from_torch(run(False))
    torch.cuda.synchronize()
    ref = oq.linear(x, _decoded(kind, W), b, epilogue=epi, residual=res, gate=g, round_then_bias=kind == "mxfp8")
    if sig is not None:
        ref[:, sig:] = oq.linear(x, _decoded(kind, W), b, epilogue="sigmoid2",
                                 round_then_bias=kind == "mxfp8")[:, sig:]
    assert max_rel_err(got, ref) <= 1e-2
    assert cos_sim(got, ref) >= 0.9999
    assert (ulp_diff_bf16(got, ref) == 0).mean() >= 0.85
    assert (ulp_diff_bf16(got, single) == 0).mean() >= 0.85


@pytest.mark.parametrize("kind", ["bf16", "mxfp8"])
def test_rows_deterministic_and_counters_zero(kind):
    """The split sum runs in split order in whichever workgroup finishes last:
    the same call gives the same bits every time (here interleaved with other
    products on the same stream, and on a second stream), for every split
    count; the ticket counters end at zero."""
    from ltx_amd.kernels import gemm

    rng = np.random.default_rng(7)
    M, K, N = 68, 8192, 2048
    x, W = _t(_bf(rng, (M, K))), _t(_bf(rng, (N, K), 0.02))
    wt = gemm.make_weight(W, kind=kind)
    other = gemm.make_weight(_t(_bf(rng, (6176, 2048), 0.02)), kind=kind)
    xo = _t(_bf(rng, (M, 2048)))
    for s in (1, 2, 8, 16, 32):
        print(f"rows determinism {kind} splits={s}", flush=True)
        first = gemm.linear_rows(x, wt, splits=s).clone()
        for _ in range(3):
            gemm.linear_rows(xo, other)
            again = gemm.linear_rows(x, wt, splits=s)
            torch.cuda.synchronize()
            assert torch.equal(first, again)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        a = gemm.linear_rows(x, wt, splits=16)
    b = gemm.linear_rows(xo, other)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(a, gemm.linear_rows(x, wt, splits=16))
    assert torch.equal(b, gemm.linear_rows(xo, other))
    torch.cuda.synchronize()
    for buf in gemm._rows_counters.values():
        assert int(buf.abs().sum().item()) == 0


def test_rows_graph_replay_matches_eager():
    """A few-row product with a gated residual epilogue captured in a HIP graph
    (its counters zeroed by a fill kernel inside the graph when the capture
    stream has no cached array) replays to the eager bits, three times, with
    eager work of the same kernel between the replays."""
    from ltx_amd.kernels import gemm

    rng = np.random.default_rng(11)
    M, K, N = 68, 2048, 8192
    wt = gemm.make_weight(_t(_bf(rng, (N, K), 0.02)), _t(rng.standard_normal(N).astype(np.float32) * 0.1,
                                                           torch.float32), kind="mxfp8")
    w2 = gemm.make_weight(_t(_bf(rng, (2048, N), 0.02)), kind="mxfp8")
    x = _t(_bf(rng, (M, K)))
    res0 = _t(_bf(rng, (M, 2048)))
    gt = _t(rng.standard_normal(2048).astype(np.float32) * 0.5, torch.float32)

    def step(res):
        h = gemm.linear(x, wt, epilogue=gemm.EPI_GELU)
        return gemm.linear(h, w2, epilogue=gemm.EPI_RESIDUAL, out=res, residual=res, gate=gt)

    res = res0.clone()
    eager = step(res).clone()
    res_g = res0.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(res0.clone())  # warm-up on the capture stream's neighbour
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        step(res_g)
    for rep in range(3):
        print(f"rows graph replay {rep}", flush=True)
        res_g.copy_(res0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(res_g, eager)
        other = res0.clone()
        step(other)  # eager calls of the same kernels between replays
        torch.cuda.synchronize()
        assert torch.equal(other, eager)


def test_rows_rejects_bad_splits():
    from ltx_amd._lib import LtxKernelError
    from ltx_amd.kernels import gemm

    wt = gemm.make_weight(torch.zeros((64, 2048), dtype=torch.bfloat16, device=DEV), kind="mxfp8")
    x = torch.zeros((4, 2048), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(LtxKernelError):
        gemm.linear_rows(x, wt, splits=32)  # 2048 % (128 * 32) != 0 for 8-bit weights
    with pytest.raises(LtxKernelError):
        gemm.linear_rows(x, wt, splits=3)   # 2048 % (128 * 3) != 0
