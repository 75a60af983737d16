"""Host-side logic of bench.py: the one-GPU guard, the step's algorithmic
flop count and the HBM-traffic record it reports (no GPU needed)."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]


def test_step_flops_closed_form():
    """48 blocks at 3456 video + 68 audio + 256 text tokens: 101.0 TFLOP.
    Spot-check the composition: a video-only one-block step is the six
    projection GEMM groups plus self and text attention plus the output
    head, written out here from the block's shapes."""
    total = bench.step_flops(3456, 68, 256, 48)
    assert total == pytest.approx(101.01e12, rel=1e-3)
    tv, s, d, h = 3456, 256, 4096, 32
    gemm = (2 * tv * d * (3 * d + h) + 2 * tv * d * d          # self-attention QKV + gate, out
            + 2 * tv * d * (d + h) + 2 * s * d * 2 * d + 2 * tv * d * d  # text attention Q + gate, KV, out
            + 2 * tv * d * 4 * d * 2)                          # feed-forward up and down
    attn = 4 * tv * tv * d + 4 * tv * s * d
    head = 2 * tv * 128 * d * 2                                # patchify in, projection out
    assert bench.step_flops(tv, 0, s, 1) == pytest.approx(gemm + attn + head, rel=1e-12)
    # linear in the block count beyond the per-step head
    assert bench.step_flops(tv, 68, s, 2) - bench.step_flops(tv, 68, s, 1) == pytest.approx(
        bench.step_flops(tv, 68, s, 1) - bench.step_flops(tv, 68, s, 0), rel=1e-12)


def test_traffic_record_is_consistent():
    """The bytes the bench reports are the counter values scaled by the copy
    calibration recorded next to them."""
    rec = json.loads((ROOT / "profiles" / "gemm_ff_up_hbm_traffic.json").read_text())
    for r in rec["launches"]:
        expect = r["fetch_size_kib"] * 1024 * r["fetch_scale"] + r["write_size_kib"] * 1024 * r["write_scale"]
        assert r["hbm_bytes"] == pytest.approx(expect, abs=1024)
        assert bench.measured_traffic(r["kernel"], r["weights"]) == r["hbm_bytes"]
        assert r["hbm_bytes"] > r["algorithmic_bytes"]
    assert bench.measured_traffic("no such kernel", "mxfp8") is None


def test_launch_stamps_pair_the_chosen_launches():
    """The stamp recorder brackets exactly the launches `select` chooses, in
    per-graph slot ranges, and turns stamp pairs into durations."""
    import torch

    st = bench.LaunchStamps(torch, 2, lambda info, k: "ff_up" if info[0] == "ff_up" else None, device="cpu")
    written = []

    def fake_stamp(addr):  # records the slot a stamp kernel would write
        written.append(addr)
        base = st.slots.data_ptr()
        idx = (addr - base) // 8
        st.slots.view(-1)[idx] = 1000 * (len(written))

    st._stamp = fake_stamp
    launches = [("qkv",), ("ff_up",), ("out",), ("ff_up",)]
    for k in range(2):
        st.k = k
        for info in launches:
            st.hook("pre", info)
            st.hook("post", info)
    assert st.count == [2, 2]
    row = st.slots.shape[1] * 8
    base = st.slots.data_ptr()
    # graph k's pairs at slots 0..3 of its row, pre before post
    assert written == [base + k * row + o for k in range(2) for o in (0, 8, 16, 24)]
    d = st.durations_ms(rate=1000.0)  # 1000 ticks per ms
    assert d == [1.0, 1.0, 1.0, 1.0]
    assert [lab for lab, _, _ in st.records(rate=1000.0)] == ["ff_up"] * 4


def test_gemm_classes_of_the_step_shapes():
    """Every GEMM shape of the 768x512x65 AV block maps to its class, and the
    per-class summary is flops over stamped durations."""
    from ltx_amd.kernels import gemm

    tv, ta, s = 3456, 68, 256
    B, R, G = gemm.EPI_BIAS, gemm.EPI_RESIDUAL, gemm.EPI_GELU
    cases = {("mxfp8", tv, 16384, 4096, G): "ff_up", ("mxfp8", tv, 4096, 16384, R): "ff_down",
             ("mxfp8", tv, 3 * 4096 + 32, 4096, B): "qkv", ("mxfp8", tv, 4096, 4096, R): "out",
             ("mxfp8", tv, 4096, 4096, B): "v2a_kv", ("mxfp8", tv, 4096 + 32, 4096, B): "text_q",
             ("mxfp8", tv, 2048 + 32, 4096, B): "a2v_q", ("mxfp8", tv, 4096, 2048, R): "a2v_out",
             ("mxfp8", ta, 3 * 2048 + 32, 2048, B): "audio", ("mxfp8", s, 8192, 4096, B): "context_kv"}
    for info, want in cases.items():
        assert bench.gemm_class(info, tv, ta, s) == want, info
    # each class is stamped in exactly one step graph (FF up in all of them)
    stamped = [c for group in bench.GEMM_CLASS_GRAPHS for c in group]
    assert len(stamped) == len(set(stamped)) and set(stamped) | {"ff_up"} == set(cases.values())
    recs = [(c, info, 0.5) for info, c in cases.items() if c in bench.VIDEO_STREAM_CLASSES]
    summ = bench.gemm_class_summary(recs + [("ff_up", ("mxfp8", tv, 16384, 4096, G), 0.25)])
    fl = 2.0 * tv * 16384 * 4096
    assert summ["ff_up"]["launches"] == 2 and summ["ff_up"]["avg_us"] == 375.0
    assert summ["ff_up"]["tflops"] == pytest.approx(2 * fl / 0.75e-3 / 1e12, abs=0.1)
    vs = summ["video_stream"]
    # one launch of each class per block, two of the 4096 x 4096 output projections
    assert vs["us_per_block"] == pytest.approx(375.0 + 500.0 * 5 + 2 * 500.0, abs=0.1)
    assert vs["frac_bf16_peak"] == pytest.approx(vs["tflops"] / bench.PEAK_BF16_TFLOPS, abs=1e-3)
