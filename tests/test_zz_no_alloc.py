"""The no-allocation split-KV attention entry point against the one that
takes a caller workspace, through the C ABI.

``ltx_flash_attn_splitkv_noalloc_bf16`` runs the same kernels with the
partials in the library's fixed per-GPU scratch, so its output must equal
``ltx_flash_attn_splitkv_bf16``'s bit for bit -- on two calls in a row, the
second smaller, so stale partials of the first call would show.  A request
above the scratch limit is refused before anything is enqueued.
"""

from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(tq, tk, H, dh, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = (torch.randn((tq, H * dh), generator=g) * 2).to(torch.bfloat16).to(DEV)
    k = (torch.randn((tk, H * dh), generator=g) * 2).to(torch.bfloat16).to(DEV)
    v = torch.randn((tk, H * dh), generator=g).to(torch.bfloat16).to(DEV)
    gate = (torch.rand((tq, H), generator=g) * 2).to(torch.bfloat16).to(DEV)
    return q, k, v, gate


def _run_pair(tq, tk, H, dh, splits, seed):
    from ltx_amd import _lib
    from ltx_amd.kernels import attention as A

    q, k, v, gate = _inputs(tq, tk, H, dh, seed)
    vt = A.transpose_v(v, H)
    tkp = vt.shape[-1]
    scale = 1.0 / math.sqrt(dh)
    s = _lib.stream_of(q)
    ref = torch.full((tq, H * dh), float("nan"), dtype=torch.bfloat16, device=DEV)
    got = torch.full_like(ref, float("nan"))
    nbytes = _lib.lib().ltx_attn_splitkv_workspace_bytes(tq, H, dh, splits)
    assert 0 < nbytes <= _lib.ATTN_NOALLOC_SCRATCH_BYTES
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    print(f"no-alloc split-KV Tq={tq} Tk={tk} H={H} dh={dh} splits={splits}", flush=True)
    _lib.call("ltx_flash_attn_splitkv_bf16", q.data_ptr(), H * dh, k.data_ptr(), H * dh, vt.data_ptr(), tkp,
              ref.data_ptr(), H * dh, gate.data_ptr(), H, tq, tk, H, dh, scale, splits, ws.data_ptr(), nbytes, s)
    _lib.call("ltx_flash_attn_splitkv_noalloc_bf16", q.data_ptr(), H * dh, k.data_ptr(), H * dh, vt.data_ptr(),
              tkp, got.data_ptr(), H * dh, gate.data_ptr(), H, tq, tk, H, dh, scale, splits, s)
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_split_kv_equals_workspace_entry_point_on_two_calls():
    # the 121-frame audio queries over 6144 video keys, then the 68-frame ones
    # over 3456 (a smaller request: the first call's partials stay behind)
    for tq, tk, H, dh, splits, seed in ((121, 6144, 32, 64, 16, 1), (68, 3456, 32, 64, 16, 2)):
        ref, got = _run_pair(tq, tk, H, dh, splits, seed)
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (tq, tk, splits)


def test_noalloc_split_kv_refuses_requests_above_the_scratch_limit():
    from ltx_amd import _lib

    tq, tk, H, dh, splits = 1024, 4096, 32, 128, 64  # 1 GiB of partials
    need = _lib.lib().ltx_attn_splitkv_workspace_bytes(tq, H, dh, splits)
    assert need > _lib.ATTN_NOALLOC_SCRATCH_BYTES
    q, k, v, gate = _inputs(tq, 64, H, dh, 3)  # only pointers are passed; nothing runs
    out = torch.empty_like(q)
    status = _lib.lib().ltx_flash_attn_splitkv_noalloc_bf16(
        q.data_ptr(), H * dh, k.data_ptr(), H * dh, v.data_ptr(), tk, out.data_ptr(), H * dh, gate.data_ptr(), H,
        tq, tk, H, dh, 1.0 / math.sqrt(dh), splits, _lib.stream_of(q))
    assert status == _lib.ERR_SCRATCH_LIMIT
    assert "scratch" in _lib.lib().ltx_status_string(status).decode()
    # an invalid split count is refused too
    assert _lib.lib().ltx_flash_attn_splitkv_noalloc_bf16(
        q.data_ptr(), H * dh, k.data_ptr(), H * dh, v.data_ptr(), 64, out.data_ptr(), H * dh, gate.data_ptr(), H,
        8, 64, H, dh, 1.0 / math.sqrt(dh), 0, _lib.stream_of(q)) == -1


def test_noalloc_split_kv_replays_from_a_graph():
    """Once the first call on the device has resolved the scratch address
    (outside capture), the entry point enqueues only its two kernels: a HIP
    graph holding it replays bit-identically to the workspace entry point,
    with eager work between the replays reusing the same scratch."""
    from ltx_amd import _lib
    from ltx_amd.kernels import attention as A

    tq, tk, H, dh, splits = 68, 3456, 32, 64, 16
    ref, _ = _run_pair(tq, tk, H, dh, splits, 4)  # resolves the address outside capture
    q, k, v, gate = _inputs(tq, tk, H, dh, 4)
    vt = A.transpose_v(v, H)
    tkp = vt.shape[-1]
    out = torch.full((tq, H * dh), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("no-alloc split-KV under graph capture", flush=True)
    with torch.cuda.graph(graph):
        _lib.call("ltx_flash_attn_splitkv_noalloc_bf16", q.data_ptr(), H * dh, k.data_ptr(), H * dh,
                  vt.data_ptr(), tkp, out.data_ptr(), H * dh, gate.data_ptr(), H, tq, tk, H, dh,
                  1.0 / math.sqrt(dh), splits, _lib.stream_of(q))
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
        # eager work on the same scratch between replays (another problem size)
        _run_pair(121, 6144, 32, 64, 16, 10 + i)
