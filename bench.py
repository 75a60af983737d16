"""Benchmark: ms per distilled audio+video DiT denoise step on one MI355X.

Workload (default): the LTX-2.3 22B-shape transformer, 48 blocks resident in
HBM with random-init weights ~N(0, 0.02) stored as MXFP8 (E4M3 codes + E8M0
scale per 32 along K; --weights bf16|int8 for the other formats), one
denoise step at
768x512x65 -> 3456 video tokens (latent 9x16x24), 68 audio tokens and 256
text tokens per modality, eight distilled sigmas cycled.  A "step" is one
full transformer forward (preprocess, 48 blocks, output heads) plus the fused
X0/Euler update.  Inputs are resident before timing starts.

Prints ONE JSON line.  Besides ms/step and tokens/s it carries:
  roofline      the dominant kernel (video FF up-projection GEMM, M=3456,
                K=4096, N=16384, GELU epilogue): algorithmic flops per launch /
                its average launch time inside the timed replays of the
                step graphs, from device clock stamps (ltx_device_clock_stamp)
                captured right before and after every such launch on its
                stream (HIP events cannot be recorded inside graphs on ROCm;
                the timed graphs carry these 96 tiny stamp kernels per step);
                ``traffic`` = HBM bytes per launch from the rocprofv3
                FETCH_SIZE / WRITE_SIZE summary committed in profiles/ for
                this kernel and weight format (null when none matches);
  gemm_classes  the step's GEMMs by class (video QKV + gate, the two 4096 x
                4096 output projections, FF down, text query, A2V query and
                output, V2A key/value on the video tokens, the text contexts'
                key/value, the audio stream's few-row GEMMs), each class timed
                in one of the eight timed step graphs by the same device
                clock stamps as the roofline kernel: launches, average us,
                algorithmic flops / launch time and its fraction of the bf16
                MFMA peak (the audio stream's and the contexts' launches run
                beside the video stream's, sharing the chip);
  attention     the flash-attention calls of the block alone (video self at
                3456 and 6144 tokens, the 3456 x 256 text cross-attention,
                A2V 3456 x 68 and split-KV V2A 68 x 3456), each replayed from
                a HIP graph: us, TFLOP/s and fraction of the bf16 peak
                (4 Tq Tk H dh flops);
  mx_opt_in     the opt-in MX path (MXFP8 activations on the scaled fp8
                MFMA; not the reference's arithmetic): ms per step with the
                same model, the FF-up launch in those step graphs against the
                5 PFLOP/s fp8 peak, and the big products alone;
  video_only    the same 48-block step with the audio modality disabled (no
                audio stream, no A2V / V2A), same box, graph replay, and
                av_minus_video_ms = the headline minus it: what the audio
                stream costs the step;
  gemm_shapes   the block's projection shapes at M=3456 (Q/K/V/out 4096x4096
                x4, FF up 4096->16384, FF down 16384->4096) in int8 W8A16,
                MXFP8 and bf16 weights (the library's automatic kernel
                choice), each launch replayed from a HIP graph: ms, TFLOP/s
                and fraction of the bf16 MFMA peak (the MFMAs are bf16);
  fused_ops     HBM GB/s of the row kernels (AdaLN, gated add, QK-norm +
                RoPE) at the reference's test shape (T=14640, C=4096), at the
                step's 3456 video rows (768x512x65) and at 1296 rows
                (512x288x65), inputs and outputs rotating through >= 1.5 GB
                (no Infinity-Cache reuse), launches replayed from a HIP graph
                (kernel time, not host dispatch);
  clip_768x512x121  ms per step of the same 48-block model at 768x512x121
                (6144 video + 121 audio + 256 text tokens), the eight
                distilled steps replayed as HIP graphs;
  guided_step   ms per step of the CFG/STG guided loop (positive, negative
                prompt and STG-perturbed passes stacked into one forward;
                CFG-star and STG guidance; Euler), each step a HIP graph;
  per_block     one bf16 video block and one AV block at 768x512x65, AdaLN
                rows from the timestep MLPs at sigma 0.5, graph replay;
  cpu_baseline  the oracle (CPU restatement of the reference block) timed on
                this host for one AV block at the same shapes (1 warmup + 5
                timed runs; mean and p50), x48.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ltx-2-mlx_amd"))

METRIC = "ms per DiT denoise step (1 GPU, 768x512x65); fused-op HBM GB/s; GEMM MFMA %"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBPS = 8000.0


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=16)
    # the GPU clock ramps up over the first ~1-2 s of sustained matrix load;
    # 16 warmup steps (~2 s) put the timed steps at the steady clock
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--height", type=int, default=512)
    ap.add_argument("--width", type=int, default=768)
    ap.add_argument("--frames", type=int, default=65)
    ap.add_argument("--audio-tokens", type=int, default=None)
    ap.add_argument("--text-tokens", type=int, default=256)
    ap.add_argument("--weights", choices=["bf16", "int8", "mxfp8"], default="mxfp8")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of HIP graph replay")
    ap.add_argument("--kernel-steps", type=int, default=2, help="eager steps for the dominant-kernel timing")
    ap.add_argument("--guided-steps", type=int, default=3,
                    help="also time this many CFG-star + STG guided steps (3 passes each, eager); 0 skips")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fused-bench", action="store_true")
    ap.add_argument("--no-clip-768x512x121", action="store_true", help="skip the 768x512x121 leg")
    ap.add_argument("--no-gemm-shapes", action="store_true", help="skip the per-shape GEMM leg")
    ap.add_argument("--no-attention-leg", action="store_true", help="skip the attention-call leg")
    ap.add_argument("--no-video-only", action="store_true", help="skip the video-only step leg")
    ap.add_argument("--no-mx", action="store_true", help="skip the opt-in MXFP8-activation leg")
    ap.add_argument("--no-class-stamps", action="store_true",
                    help="stamp only the FF-up launches in the timed graphs (no per-class GEMM timing)")
    ap.add_argument("--cpu-runs", type=int, default=5, help="timed oracle block runs after one warmup")
    ap.add_argument("--counter-workload",
                    choices=["ff-up", "ff-up-vs-library", "copy", "fused-ops", "attention", "audio-rows"],
                    default=None,
                    help="run only a short workload for rocprofv3 --pmc passes and exit: the video FF "
                         "up-projection GEMM (4 launches, --weights format), the three row kernels (adaln, "
                         "gated add, QK-norm + RoPE; 4 cache-cold launches each), the video self-attention at "
                         "3456 and 6144 tokens and the 3456 x 256 text cross-attention (4 launches each, 32 "
                         "heads of 128, gated), the audio stream's four 68-row MXFP8 products (4 launches each "
                         "on distinct weights, automatic split-K path then the one-launch few-row kernel) or a "
                         "1 GiB device copy (3 launches, the FETCH_SIZE / WRITE_SIZE calibration)")
    ap.add_argument("--counter-tile", choices=["auto", "256", "g8"], default="auto",
                    help="tile choice of the ff-up counter workload: the library's automatic choice (the "
                         "8-wave kernel for every format at this shape), the 4-wave 256x256 kernel, or the "
                         "8-wave kernel")
    return ap.parse_args(argv)


def counter_workload(kind: str, weights: str, tile_name: str = "auto") -> None:
    import torch

    from ltx_amd.kernels import gemm

    tile = {"auto": gemm.TILE_AUTO, "256": gemm.TILE_256, "g8": gemm.TILE_G8}[tile_name]

    if kind == "fused-ops":
        # each row kernel 4 times on cache-cold rotating buffers (counter
        # runs), at T = 14640 and then at the step's 3456 video rows
        for T in (14640, 3456):
            _, launchers = fused_op_launchers(torch, T=T)
            for name, fn, _ in launchers:
                for i in range(4):
                    fn(i)
            del launchers
    elif kind == "attention":
        from ltx_amd.kernels.attention import flash_attention

        g = torch.Generator(device="cuda").manual_seed(0)
        for tq, tk in ((3456, 3456), (6144, 6144), (3456, 256)):
            q = torch.randn((tq, 4096), generator=g, device="cuda").bfloat16()
            k = torch.randn((tk, 4096), generator=g, device="cuda").bfloat16()
            v = torch.randn((tk, 4096), generator=g, device="cuda").bfloat16()
            gate = (torch.rand((tq, 32), generator=g, device="cuda") * 2).bfloat16()
            out = torch.empty((tq, 4096), dtype=torch.bfloat16, device="cuda")
            for _ in range(4):
                flash_attention(q, k, v, 32, gate=gate, out=out)
    elif kind == "audio-rows":
        # the audio stream's four 68-row products (QKV + head gates, out, FF up,
        # FF down; MXFP8 weights), each on four weight copies so every launch
        # reads its weights from HBM as in the step: first through the
        # library's automatic path (split-K tile kernel + epilogue kernel),
        # then through the one-launch few-row kernel
        g = torch.Generator(device="cuda").manual_seed(0)
        shapes = ((2048, 6176, gemm.EPI_BIAS), (2048, 2048, gemm.EPI_RESIDUAL), (2048, 8192, gemm.EPI_GELU),
                  (8192, 2048, gemm.EPI_RESIDUAL))
        for rows in (False, True):
            for K, N, epi in shapes:
                x = torch.randn((68, K), generator=g, device="cuda").bfloat16()
                res = torch.randn((68, N), generator=g, device="cuda").bfloat16()
                gate = torch.randn(N, generator=g, device="cuda")
                wts = [gemm.make_weight((torch.randn((N, K), generator=g, device="cuda") * 0.02).bfloat16(),
                                        torch.zeros(N, device="cuda"), kind="mxfp8") for _ in range(4)]
                kw = dict(out=res, residual=res, gate=gate) if epi == gemm.EPI_RESIDUAL else {}
                for wt in wts:
                    if rows:
                        gemm.linear_rows(x, wt, epilogue=epi, **kw)
                    else:
                        gemm.linear(x, wt, epilogue=epi, **kw)
    elif kind == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
    elif kind == "ff-up-vs-library":
        # the FF up-projection shape through the vendor library (hipBLASLt,
        # plain bf16 linear) and through this library's bf16 and MXFP8 GEMMs
        # (bias epilogue; the --counter-tile choice)
        g = torch.Generator(device="cuda").manual_seed(0)
        x = torch.randn((3456, 4096), generator=g, device="cuda").bfloat16()
        w = (torch.randn((16384, 4096), generator=g, device="cuda") * 0.02).bfloat16()
        b = torch.zeros(16384, device="cuda")
        wb, wm = gemm.make_weight(w, b, kind="bf16"), gemm.make_weight(w, b, kind="mxfp8")
        for _ in range(3):
            torch.nn.functional.linear(x, w)
            gemm.linear(x, wb, tile=gemm.TILE_256 if tile == gemm.TILE_G8 else tile)
            gemm.linear(x, wm, tile=tile)
    else:
        g = torch.Generator(device="cuda").manual_seed(0)
        x = torch.randn((3456, 4096), generator=g, device="cuda").bfloat16()
        w = (torch.randn((16384, 4096), generator=g, device="cuda") * 0.02).bfloat16()
        wt = gemm.make_weight(w, torch.zeros(16384, device="cuda"), kind=weights)
        out = torch.empty((3456, 16384), dtype=torch.bfloat16, device="cuda")
        for _ in range(4):
            gemm.linear(x, wt, epilogue=gemm.EPI_GELU, out=out, tile=tile)
    torch.cuda.synchronize()
    print(f"counter workload {kind} ({weights}, tile {tile_name}) done", flush=True)


def step_flops(tv: int, ta: int, s: int, layers: int) -> float:
    """Algorithmic flops of one step (GEMMs 2MNK + attention 4*Tq*Tk*H*dh)."""
    vd, ad, hv, ha = 4096, 2048, 32, 32
    g = 0.0
    g += 2 * tv * vd * (3 * vd + hv) + 2 * tv * vd * vd           # attn1 qkv+gate, out
    g += 2 * tv * vd * (vd + hv) + 2 * s * vd * 2 * vd + 2 * tv * vd * vd  # attn2
    g += 2 * tv * vd * 4 * vd * 2                                  # ff
    if ta:
        g += 2 * ta * ad * (3 * ad + ha) + 2 * ta * ad * ad
        g += 2 * ta * ad * (ad + ha) + 2 * s * ad * 2 * ad + 2 * ta * ad * ad
        g += 2 * ta * ad * 4 * ad * 2
        g += 2 * tv * vd * (ad + ha) + 2 * ta * ad * 2 * ad + 2 * tv * ad * vd   # a2v
        g += 2 * ta * ad * (ad + ha) + 2 * tv * vd * 2 * ad + 2 * ta * ad * ad   # v2a
    a = 4 * tv * tv * vd + 4 * tv * s * vd
    if ta:
        a += 4 * ta * ta * ad + 4 * ta * s * ad + 4 * tv * ta * ad * 2
    return layers * (g + a) + 2 * tv * 128 * vd * 2 + 2 * ta * 128 * ad * 2


def measured_traffic(kernel: str, weights: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (profiles/gemm_ff_up_hbm_traffic.json), or None."""
    path = ROOT / "profiles" / "gemm_ff_up_hbm_traffic.json"
    try:
        rec = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    for r in rec.get("launches", []):
        if r.get("kernel") == kernel and r.get("weights") == weights:
            return r.get("hbm_bytes")
    return None


def fused_op_launchers(torch, T=14640, C=4096, heads=32):
    """The three HBM-bound row kernels at (T, C) on preallocated buffers that
    rotate through >= 1.5 GB per operand, so no operand is served from the
    256 MB last-level cache.  QK-norm + RoPE works in place on the Q and K
    columns of a fused (T, 3C) projection output (the block's layout) with
    the shared (T, C/2) fp32 cos / sin tables.  Returns (nbuf, [(name,
    launch(i), algorithmic bytes per launch)])."""
    from ltx_amd.kernels.fused_ops import adaln_rows, gated_add_rows
    from ltx_amd.kernels.rope_ops import qknorm_rope_

    nbytes = T * C * 2
    nbuf = max(3, math.ceil(1.5e9 / nbytes))
    xs = [torch.randn((T, C), device="cuda").bfloat16() for _ in range(nbuf)]
    bs = [torch.randn((T, C), device="cuda").bfloat16() for _ in range(nbuf)]
    outs = [torch.empty((T, C), device="cuda", dtype=torch.bfloat16) for _ in range(nbuf)]
    scale = torch.randn(C, device="cuda") * 0.1
    shift = torch.randn(C, device="cuda") * 0.1
    gate = torch.randn(C, device="cuda") * 0.5
    nq = max(3, math.ceil(1.5e9 / (T * (3 * C * 2 + C * 4))))
    qkv = [torch.randn((T, 3 * C), device="cuda").bfloat16() for _ in range(nq)]
    tabs = [(torch.rand((T, C // 2), device="cuda") * 2 - 1, torch.rand((T, C // 2), device="cuda") * 2 - 1)
            for _ in range(nq)]
    wq = torch.rand(C, device="cuda") + 0.5
    wk = torch.rand(C, device="cuda") + 0.5
    return nbuf, [
        ("adaln_norm_fused", lambda i: adaln_rows(xs[i % nbuf], C, scale, shift, outs[(i + 1) % nbuf],
                                                  C, T, C, 1e-6, 0),
         2 * nbytes + 2 * C * 4),
        ("gated_add_fused", lambda i: gated_add_rows(xs[i % nbuf], C, bs[i % nbuf], C, gate,
                                                     outs[(i + 1) % nbuf], C, T, C, 0),
         3 * nbytes + C * 4),
        ("qknorm_rope", lambda i: qknorm_rope_(qkv[i % nq][:, :C], wq, tabs[i % nq], qkv[i % nq][:, C:2 * C], wk,
                                               tabs[i % nq], heads),
         4 * nbytes + 2 * T * (C // 2) * 4 + 2 * C * 4),
    ]


def fused_op_bandwidth(torch, T=14640, C=4096):
    """HBM GB/s of the row kernels (fused_op_launchers), each replayed from a
    HIP graph, best of three replays."""
    nbuf, launchers = fused_op_launchers(torch, T, C)
    res = {}
    for name, fn, algo in launchers:
        for i in range(nbuf):
            fn(i)
        torch.cuda.synchronize()
        # replayed from a HIP graph so host dispatch does not pace the short kernels
        iters = max(8 * nbuf, 256)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(iters):
                fn(i % nbuf)
        g.replay()
        torch.cuda.synchronize()
        t = float("inf")
        for _ in range(3):  # best of three replays
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            g.replay()
            e.record()
            torch.cuda.synchronize()
            t = min(t, s.elapsed_time(e) / iters * 1e-3)
        del g
        res[name] = {"us": round(t * 1e6, 2), "GB/s": round(algo / t / 1e9, 1),
                     "frac_hbm_peak": round(algo / t / 1e9 / PEAK_HBM_GBPS, 3), "bytes": algo}
    del launchers
    return res


def cpu_baseline(tv: int, ta: int, s: int, layers: int, grid, runs: int = 5):
    """Oracle AV block at full shapes on the host (one warmup, then ``runs``
    timed runs), x layers."""
    import torch

    from oracle import block as ob
    from oracle import rope as orope

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)

    def rnd(*shape, std=0.02):
        return ob.bf(torch.randn(shape, generator=g) * std)

    def attn(qd, kd, heads, dh):
        inner = heads * dh
        return {"to_q": rnd(inner, qd), "to_q_b": torch.zeros(inner), "to_k": rnd(inner, kd),
                "to_k_b": torch.zeros(inner), "to_v": rnd(inner, kd), "to_v_b": torch.zeros(inner),
                "to_gate_logits": rnd(heads, qd), "to_gate_logits_b": torch.zeros(heads),
                "to_out": rnd(qd, inner), "to_out_b": torch.zeros(qd), "q_norm": torch.ones(inner),
                "k_norm": torch.ones(inner)}

    def ff(d):
        return {"w1": rnd(4 * d, d), "b1": torch.zeros(4 * d), "w2": rnd(d, 4 * d), "b2": torch.zeros(d)}

    W = {"attn1": attn(4096, 4096, 32, 128), "attn2": attn(4096, 4096, 32, 128), "ff": ff(4096),
         "audio_attn1": attn(2048, 2048, 32, 64), "audio_attn2": attn(2048, 2048, 32, 64), "audio_ff": ff(2048),
         "audio_to_video_attn": attn(4096, 2048, 32, 64), "video_to_audio_attn": attn(2048, 4096, 32, 64)}
    vpos = orope.video_positions(*grid, fps=24.0)
    apos = orope.audio_positions(ta)
    pes = [tuple(torch.from_numpy(a) for a in p) for p in (
        orope.rope_tables(vpos, 4096, 32, orope.VIDEO_MAX_POS),
        orope.rope_tables(vpos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos, 2048, 32, orope.AUDIO_MAX_POS),
        orope.rope_tables(apos[:, 0:1], 2048, 32, orope.AUDIO_MAX_POS))]
    vx, ax = rnd(tv, 4096, std=1.0), rnd(ta, 2048, std=1.0)
    vctx, actx = rnd(s, 4096, std=1.0), rnd(s, 2048, std=1.0)
    vada, aada = torch.randn(16, 4096, generator=g) * 0.05, torch.randn(16, 2048, generator=g) * 0.05
    ob.block(W, vx, ax, vada, aada, vctx, actx, *pes)  # warmup
    times = []
    for _ in range(max(1, runs)):
        t0 = time.perf_counter()
        ob.block(W, vx, ax, vada, aada, vctx, actx, *pes)
        times.append(time.perf_counter() - t0)
    mean, p50 = sum(times) / len(times), sorted(times)[len(times) // 2]
    return {"value": round(mean * layers * 1e3, 1), "unit": "ms/step", "cores": threads, "kind": "port",
            "p50": round(p50 * layers * 1e3, 1), "runs": len(times),
            "sample": f"one AV block (oracle, torch-CPU fp32 with the reference's bf16 roundings) at "
                      f"{tv} video + {ta} audio + {s} text tokens: 1 warmup + {len(times)} timed runs "
                      f"(mean {mean:.2f} s, p50 {p50:.2f} s per block), x{layers} blocks; the reference's own "
                      f"MLX CPU backend is not installable here"}


def gemm_step_profile(run_step, steps, tv, torch, prefill=None):
    """Time every GEMM launch of ``steps`` eager steps with events recorded on
    its own stream around the launch (the ``--no-graph`` fallback: the events
    include host gaps whenever the host enqueues slower than the device
    runs).  ``prefill`` is queued first.  Returns (FF-up launch durations in
    ms, per-stream summary, host enqueue ms per eager step)."""
    from ltx_amd.kernels import gemm

    recs = []
    main = torch.cuda.current_stream().cuda_stream

    def hook(phase, info):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        if phase == "pre":
            recs.append([info, torch.cuda.current_stream().cuda_stream, e, None])
        else:
            recs[-1][3] = e

    torch.cuda.synchronize()
    if prefill is not None:
        prefill()
    gemm.LAUNCH_HOOK = hook
    try:
        t0 = time.perf_counter()
        for i in range(steps):
            run_step(i)
        host_ms = (time.perf_counter() - t0) / steps * 1e3
        torch.cuda.synchronize()
    finally:
        gemm.LAUNCH_HOOK = None
    ff_up, groups = [], {}
    for (kind, m, n, k, epi), stream, pre, post in recs:
        ms = pre.elapsed_time(post)
        if epi == gemm.EPI_GELU and m == tv and k == 4096:
            ff_up.append(ms)
        g = groups.setdefault("video_stream" if stream == main else "audio_stream", [0, 0.0, 0.0])
        g[0] += 1
        g[1] += 2.0 * m * n * k
        g[2] += ms
    summary = {}
    tot = [0, 0.0, 0.0]
    for name, (cnt, fl, ms) in groups.items():
        tot = [tot[0] + cnt, tot[1] + fl, tot[2] + ms]
        summary[name] = {"launches_per_step": cnt // steps, "gflop_per_step": round(fl / steps / 1e9, 1),
                         "ms_per_step": round(ms / steps, 3),
                         "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                         "frac_bf16_peak": round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    summary["all"] = {"gflop_per_step": round(tot[1] / steps / 1e9, 1), "ms_per_step": round(tot[2] / steps, 3),
                      "tflops": round(tot[1] / (tot[2] * 1e-3) / 1e12, 1),
                      "frac_bf16_peak": round(tot[1] / (tot[2] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    return ff_up, summary, host_ms


# GEMM classes of the step, by launch shape (kind, M, N, K, epilogue) at
# 4096-wide video and 2048-wide audio streams
def gemm_class(info, tv: int, ta: int, s: int):
    from ltx_amd.kernels import gemm

    _, m, n, k, epi = info
    resid = epi in (gemm.EPI_RESIDUAL, gemm.EPI_RESIDUAL_ROUND)
    if m == tv:
        if k == 4096 and n == 16384:
            return "ff_up"
        if k == 16384:
            return "ff_down"
        if k == 4096 and n == 3 * 4096 + 32:
            return "qkv"
        if k == 4096 and n == 4096:
            return "out" if resid else "v2a_kv"
        if k == 4096 and n == 4096 + 32:
            return "text_q"
        if k == 4096 and n == 2048 + 32:
            return "a2v_q"
        if k == 2048 and n == 4096:
            return "a2v_out"
        return None
    if m == ta:
        return "audio"
    if m == s:
        return "context_kv"
    return None


# which classes besides FF up the step graph k carries stamps for: one group
# per graph, so each timed graph holds few extra stamp kernels
GEMM_CLASS_GRAPHS = (("qkv",), ("out",), ("ff_down",), ("text_q", "context_kv"), ("a2v_q", "a2v_out"),
                     ("v2a_kv",), ("audio",), ())
VIDEO_STREAM_CLASSES = ("ff_up", "ff_down", "qkv", "out", "text_q", "a2v_q", "a2v_out")


class LaunchStamps:
    """Device clock stamps around chosen GEMM launches inside captured HIP
    graphs.  While ``capturing(k)`` is active, every launch for which
    ``select(info, k)`` returns a label gets a stamp kernel
    (ltx_device_clock_stamp) right before and right after it on its stream,
    writing into slot range k; each replay of that graph overwrites the range,
    so after the timed replays it holds the last replay of every graph.  The
    counter's rate comes from two stamps around a host sleep."""

    CAP = 1024  # stamped launches per graph

    def __init__(self, torch, graphs: int, select, device: str = "cuda"):
        self.torch, self.select = torch, select
        self.slots = torch.zeros((graphs, 2 * self.CAP), dtype=torch.int64, device=device)
        self.count = [0] * graphs
        self.labels = [[] for _ in range(graphs)]
        self.k, self.on = None, False

    def _stamp(self, addr):
        from ltx_amd import _lib

        _lib.call("ltx_device_clock_stamp", addr, self.torch.cuda.current_stream().cuda_stream)

    def hook(self, phase, info):
        k = self.k
        if phase == "pre":
            label = self.select(info, k)
            self.on = label is not None
            if self.on:
                if self.count[k] >= self.CAP:
                    raise RuntimeError("too many stamped launches in one graph")
                self.labels[k].append((label, info))
                self._stamp(self.slots[k].data_ptr() + 16 * self.count[k])
        elif self.on:
            self._stamp(self.slots[k].data_ptr() + 16 * self.count[k] + 8)
            self.count[k] += 1
            self.on = False

    def capturing(self, k):
        import contextlib

        from ltx_amd.kernels import gemm

        @contextlib.contextmanager
        def ctx():
            self.k = k
            gemm.LAUNCH_HOOK = self.hook
            try:
                yield
            finally:
                gemm.LAUNCH_HOOK = None
                self.k = None

        return ctx()

    def ticks_per_ms(self) -> float:
        from ltx_amd import _lib

        torch = self.torch
        r = torch.zeros(2, dtype=torch.int64, device="cuda")
        s = torch.cuda.current_stream().cuda_stream
        _lib.call("ltx_device_clock_stamp", r.data_ptr(), s)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        time.sleep(0.25)
        _lib.call("ltx_device_clock_stamp", r.data_ptr() + 8, s)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        v = r.tolist()
        return (v[1] - v[0]) / ((t1 - t0) * 1e3)

    def durations_ms(self, rate=None, label=None) -> list:
        """Stamped launch durations (ms), all or those of one label."""
        return [d for lab, _, d in self.records(rate) if label is None or lab == label]

    def records(self, rate=None) -> list:
        """(label, launch info, duration ms) of every stamped launch."""
        rate = self.ticks_per_ms() if rate is None else rate
        v = self.slots.tolist()
        out = []
        for k, n in enumerate(self.count):
            out += [(self.labels[k][i][0], self.labels[k][i][1], (v[k][2 * i + 1] - v[k][2 * i]) / rate)
                    for i in range(n)]
        return out


def gemm_class_summary(records) -> dict:
    """Per GEMM class: launches, average us, algorithmic TFLOP/s and fraction
    of the bf16 peak over the stamped launches; ``video_stream`` combines
    the video-stream classes (flops over summed durations of one launch of
    each kind per block, i.e. weighted by how often the step runs them)."""
    acc = {}
    for label, (_, m, n, k, _), ms in records:
        a = acc.setdefault(label, [0, 0.0, 0.0])
        a[0] += 1
        a[1] += 2.0 * m * n * k
        a[2] += ms
    res = {}
    for label, (cnt, fl, ms) in sorted(acc.items()):
        res[label] = {"launches": cnt, "avg_us": round(ms / cnt * 1e3, 1),
                      "gflop_per_launch": round(fl / cnt / 1e9, 2),
                      "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                      "frac_bf16_peak": round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    per_block = {"ff_up": 1, "ff_down": 1, "qkv": 1, "out": 2, "text_q": 1, "a2v_q": 1, "a2v_out": 1}
    if all(c in res for c in per_block):
        fl = sum(res[c]["gflop_per_launch"] * per_block[c] for c in per_block)
        us = sum(res[c]["avg_us"] * per_block[c] for c in per_block)
        res["video_stream"] = {"us_per_block": round(us, 1), "gflop_per_block": round(fl, 1),
                               "tflops": round(fl / us * 1e3, 1),
                               "frac_bf16_peak": round(fl / us * 1e3 / PEAK_BF16_TFLOPS, 4)}
    return res


def gemm_shapes(torch, fmt: str, m: int = 3456, tile=None) -> dict:
    """The block's projection GEMMs at M rows in one weight format: each shape
    launched 10 times from a HIP graph, best of three replays.  ``tile``
    forces a kernel (gemm.TILE_*) instead of the automatic choice."""
    from ltx_amd.kernels import gemm

    tile = gemm.TILE_AUTO if tile is None else tile

    g = torch.Generator(device="cuda").manual_seed(0)
    shapes = (("qkv_out_4096x4096", 4096, 4096, 4), ("ff_up_4096x16384", 4096, 16384, 1),
              ("ff_down_16384x4096", 16384, 4096, 1))
    res, tot_ms, tot_fl = {}, 0.0, 0.0
    for name, k, n, count in shapes:
        x = torch.randn((m, k), generator=g, device="cuda").bfloat16()
        w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).bfloat16()
        wt = gemm.make_weight(w, torch.zeros(n, device="cuda"), kind=fmt)
        out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        gemm.linear(x, wt, out=out, tile=tile)
        torch.cuda.synchronize()
        iters = 10
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(iters):
                gemm.linear(x, wt, out=out, tile=tile)
        graph.replay()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) / iters)
        fl = 2.0 * m * n * k
        res[name] = {"ms": round(best, 4), "tflops": round(fl / (best * 1e-3) / 1e12, 1),
                     "frac_bf16_peak": round(fl / (best * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), "per_block": count}
        tot_ms += best * count
        tot_fl += fl * count
        del graph, x, w, wt, out
    res["block_total"] = {"ms": round(tot_ms, 4), "gflop": round(tot_fl / 1e9, 1),
                          "tflops": round(tot_fl / (tot_ms * 1e-3) / 1e12, 1),
                          "frac_bf16_peak": round(tot_fl / (tot_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    return res


def attention_leg(torch, replays: int = 20) -> dict:
    """The block's flash-attention calls alone, gated, 32 heads: video self at
    3456 and 6144 tokens (dh 128), the 3456 x 256 text cross-attention, A2V
    (3456 queries over 68 audio keys, dh 64) and V2A (68 over 3456, split-KV
    as dispatched).  Each call replayed ``replays`` times from a HIP graph,
    best of three replays."""
    from ltx_amd.kernels.attention import flash_attention

    g = torch.Generator(device="cuda").manual_seed(0)
    res = {}
    for name, tq, tk, dh in (("self_3456", 3456, 3456, 128), ("self_6144", 6144, 6144, 128),
                             ("text_3456x256", 3456, 256, 128), ("a2v_3456x68", 3456, 68, 64),
                             ("v2a_68x3456", 68, 3456, 64)):
        d = 32 * dh
        q = torch.randn((tq, d), generator=g, device="cuda").bfloat16()
        k = torch.randn((tk, d), generator=g, device="cuda").bfloat16()
        v = torch.randn((tk, d), generator=g, device="cuda").bfloat16()
        gate = (torch.rand((tq, 32), generator=g, device="cuda") * 2).bfloat16()
        out = torch.empty((tq, d), dtype=torch.bfloat16, device="cuda")
        flash_attention(q, k, v, 32, gate=gate, out=out)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(replays):
                flash_attention(q, k, v, 32, gate=gate, out=out)
        graph.replay()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) / replays)
        fl = 4.0 * tq * tk * d
        res[name] = {"us": round(best * 1e3, 1), "tflops": round(fl / (best * 1e-3) / 1e12, 1),
                     "frac_bf16_peak": round(fl / (best * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                     "gflop": round(fl / 1e9, 2)}
        del graph, q, k, v, gate, out
    return res


def video_only_leg(args, torch, s: int, steps_timed: int = 16) -> dict:
    """The same 48-block step with the audio modality disabled: no audio
    stream, no A2V / V2A sub-layers, video text cross-attention and FF
    unchanged; the eight distilled steps as HIP graphs, one warm-up pass of
    each, then ``steps_timed`` steps."""
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.pipeline import DenoiseState, denoise_step

    model = LTXModel(num_layers=args.layers, weight_format=args.weights, seed=0, audio=False)
    st = DenoiseState(model, args.height, args.width, args.frames, text_tokens=s, seed=0)
    pes = model.rope(st.video_positions, None)
    nsig = len(st.sigmas) - 1
    denoise_step(model, st, 0, pes)
    torch.cuda.synchronize()
    pool = torch.cuda.graph_pool_handle()
    graphs = []
    for i in range(nsig):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            denoise_step(model, st, i, pes)
        graphs.append(g)
    for _ in range(2):
        for i in range(nsig):
            graphs[i].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps_timed):
        graphs[i % nsig].replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps_timed * 1e3
    tv = st.video_tokens
    fl = step_flops(tv, 0, s, args.layers)
    del graphs, model, st
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 3), "steps": steps_timed, "timing": "hip-graph replay",
            "workload": f"{args.layers}-block video-only denoise step at {args.width}x{args.height}x{args.frames}",
            "video_tokens": tv, "text_tokens": s, "step_tflop": round(fl / 1e12, 2),
            "step_tflops_achieved": round(fl / (ms * 1e-3) / 1e12, 1)}


PEAK_FP8_TFLOPS = 5000.0


def mx_opt_in_leg(model, state, pes, torch, tv: int, ta: int, s: int, steps_timed: int = 16) -> dict:
    """The opt-in MX path (gemm.MX_ACTIVATIONS): the same model and step with
    every large MXFP8 product on the scaled fp8 MFMA, activations quantised to
    MXFP8 (the FF hidden rows by the up-projection's epilogue, the other
    inputs by the row quantiser); eight step graphs captured anew, 16 warm-up
    and ``steps_timed`` timed replays, FF-up launches stamped as in the
    headline.  Plus the block's three big products alone (graph replay of 10
    launches, best of three): quantised-input GEMM time against the 5 PFLOP/s
    dense fp8 peak."""
    from ltx_amd.kernels import gemm
    from ltx_amd.pipeline import denoise_step

    nsig = len(state.sigmas) - 1
    stamps = LaunchStamps(torch, nsig, lambda info, k: "ff_up" if gemm_class(info, tv, ta, s) == "ff_up" else None)
    gemm.MX_ACTIVATIONS = True
    try:
        denoise_step(model, state, 0, pes)
        torch.cuda.synchronize()
        pool = torch.cuda.graph_pool_handle()
        graphs = []
        for i in range(nsig):
            g = torch.cuda.CUDAGraph()
            with stamps.capturing(i), torch.cuda.graph(g, pool=pool):
                denoise_step(model, state, i, pes)
            graphs.append(g)
    finally:
        gemm.MX_ACTIVATIONS = False
    for i in range(16):
        graphs[i % nsig].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps_timed):
        graphs[i % nsig].replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps_timed * 1e3
    durs = stamps.durations_ms()
    del graphs
    fl = 2.0 * tv * 4096 * 16384
    k_ms = sum(durs) / len(durs)
    res = {"ms_per_step": round(ms, 3), "steps": steps_timed, "timing": "hip-graph replay",
           "tokens_per_s": round((tv + ta) / (ms * 1e-3), 1),
           "ff_up_in_step": {"launch_us": round(k_ms * 1e3, 1), "launches_timed": len(durs),
                             "tflops": round(fl / (k_ms * 1e-3) / 1e12, 1),
                             "frac_fp8_peak": round(fl / (k_ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)},
           "arithmetic": "MXFP8 activations x MXFP8 weights (scaled fp8 MFMA); the reference keeps bf16 "
                         "activations -- opt-in, not the parity path"}
    g = torch.Generator(device="cuda").manual_seed(0)
    shapes = {}
    for name, m, k, n in (("ff_up_4096x16384", tv, 4096, 16384), ("ff_down_16384x4096", tv, 16384, 4096),
                          ("qkv_4096x12320", tv, 4096, 3 * 4096 + 32)):
        x = torch.randn((m, k), generator=g, device="cuda").bfloat16()
        wt = gemm.make_weight((torch.randn((n, k), generator=g, device="cuda") * 0.02).bfloat16(),
                              torch.zeros(n, device="cuda"), kind="mxfp8")
        codes, scales = gemm.quantize_rows_mxfp8(x)
        out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        for label, fn in (("gemm", lambda: gemm.linear_mx(codes, scales, wt, out=out)),
                          ("row_quantiser", lambda: gemm.quantize_rows_mxfp8(x, codes, scales))):
            fn()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(10):
                    fn()
            graph.replay()
            torch.cuda.synchronize()
            best = float("inf")
            for _ in range(3):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                graph.replay()
                b.record()
                torch.cuda.synchronize()
                best = min(best, a.elapsed_time(b) / 10)
            del graph
            if label == "gemm":
                fl = 2.0 * m * n * k
                shapes[name] = {"us": round(best * 1e3, 1), "tflops": round(fl / (best * 1e-3) / 1e12, 1),
                                "frac_fp8_peak": round(fl / (best * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)}
            else:
                shapes[name]["row_quantiser_us"] = round(best * 1e3, 1)
        del x, wt, codes, scales, out
    res["gemm_alone"] = shapes
    return res


def clip_768x512x121_leg(model, torch, steps_timed: int = 16) -> dict:
    """ms per step at 768x512x121: 6144 video + 121 audio + 256 text tokens,
    the eight distilled steps captured as HIP graphs, one full warmup pass,
    then ``steps_timed`` steps."""
    from ltx_amd.pipeline import DenoiseState, denoise_step

    st = DenoiseState(model, 512, 768, 121, text_tokens=256, audio_frames=121, seed=0)
    pes = model.rope(st.video_positions, st.audio_positions)
    nsig = len(st.sigmas) - 1
    denoise_step(model, st, 0, pes)
    torch.cuda.synchronize()
    pool = torch.cuda.graph_pool_handle()
    graphs = []
    for i in range(nsig):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            denoise_step(model, st, i, pes)
        graphs.append(g)
    for i in range(nsig):
        graphs[i].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps_timed):
        graphs[i % nsig].replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps_timed * 1e3
    finite = bool(torch.isfinite(st.video_latent.float()).all() and torch.isfinite(st.audio_latent.float()).all())
    del graphs
    tv, ta = st.video_tokens, st.audio_tokens
    fl = step_flops(tv, ta, 256, model.num_layers)
    return {"ms_per_step": round(ms, 3), "steps": steps_timed, "timing": "hip-graph replay",
            "workload": f"{model.num_layers}-block AV denoise step at 768x512x121",
            "video_tokens": tv, "audio_tokens": ta, "text_tokens": 256,
            "tokens_per_s": round((tv + ta) / (ms * 1e-3), 1), "step_tflop": round(fl / 1e12, 2),
            "step_tflops_achieved": round(fl / (ms * 1e-3) / 1e12, 1), "latents_finite": finite}


def per_block_leg(torch, args, ta: int, s: int, replays: int = 20) -> dict:
    """One transformer block at 768x512x65, bf16 weights ~N(0, 0.02), AdaLN
    rows from the model's timestep MLPs at sigma = 0.5: the video-only block
    (3456 video + 256 text tokens) and the joint AV block (+ 68 audio
    tokens, audio on its second stream).  Each block call is captured as a
    HIP graph and replayed; ms per block call, best of three runs."""
    from ltx_amd import _lib
    from ltx_amd.kernels import gemm
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.model.transformer.transformer import ADA_ROWS, TransformerArgs
    from ltx_amd.pipeline import DenoiseState

    res = {}
    for name, audio in (("video_block_bf16", False), ("av_block_bf16", True)):
        m = LTXModel(num_layers=1, weight_format="bf16", seed=3, audio=audio)
        st = DenoiseState(m, args.height, args.width, args.frames, text_tokens=s,
                          audio_frames=ta if audio else 0, seed=3)
        vpe, vxpe, ape, axpe = m.rope(st.video_positions, st.audio_positions if audio else None)
        sig = torch.full((1,), 0.5, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream
        vx = gemm.linear(st.video_latent, m.patchify_proj)
        m._timestep_rows(sig, sig, video=True)
        _lib.call("ltx_broadcast_add_f32", m.video_tables.data_ptr(), m._temb_v.data_ptr(), m._ada_v.data_ptr(),
                  1, ADA_ROWS * m.video_dim, stream)
        video = TransformerArgs(x=vx, context=st.video_context, timesteps=m._temb_v[:9],
                                positional_embeddings=vpe, cross_positional_embeddings=vxpe)
        audio_args = None
        block = m.transformer_blocks[0]
        block.ada_rows_video = m._ada_v[0]
        if audio:
            ax = gemm.linear(st.audio_latent, m.audio_patchify_proj)
            m._timestep_rows(sig, sig, video=False)
            _lib.call("ltx_broadcast_add_f32", m.audio_tables.data_ptr(), m._temb_a.data_ptr(), m._ada_a.data_ptr(),
                      1, ADA_ROWS * m.audio_dim, stream)
            audio_args = TransformerArgs(x=ax, context=st.audio_context, timesteps=m._temb_a[:9],
                                         positional_embeddings=ape, cross_positional_embeddings=axpe)
            block.ada_rows_audio = m._ada_a[0]
            block.audio_stream = torch.cuda.Stream()
        def call():
            block(video, audio_args)
            if block.audio_stream is not None:  # join the audio stream (the model does after its last block)
                torch.cuda.current_stream().wait_stream(block.audio_stream)

        call()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call()
        g.replay()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            t0 = time.perf_counter()
            for _ in range(replays):
                g.replay()
            torch.cuda.synchronize()
            best = min(best, (time.perf_counter() - t0) / replays * 1e3)
        res[name] = {"ms": round(best, 3), "video_tokens": st.video_tokens, "audio_tokens": st.audio_tokens,
                     "text_tokens": s, "weights": "bf16", "sigma": 0.5, "timing": "hip-graph replay"}
        del g, m, st, block
        torch.cuda.empty_cache()
    return res


def guided_step_ms(model, args, ta: int, s: int) -> dict:
    """ms per guided step of the CFG/STG loop (av_pipeline.py:625-757): the
    positive, negative-prompt and STG-perturbed transformer passes stacked
    into one forward, CFG-star guidance (video 3.0, audio 7.0), STG (scale
    1.0, video self-attention skipped in every block), Euler; shifted LTX-2
    sigma schedule.  Each step is captured as a HIP graph once; a generation
    replays them (warm-up generation first, then the timed one)."""
    import torch

    from ltx_amd.components.guiders import CFGStarRescalingGuider, STGGuider
    from ltx_amd.components.perturbations import create_batched_stg_config
    from ltx_amd.components.schedulers import LTX2Scheduler
    from ltx_amd.pipeline import CfgAvLoop, DenoiseState

    kw = dict(video_guider=CFGStarRescalingGuider(3.0), audio_guider=CFGStarRescalingGuider(7.0),
              stg_guider=STGGuider(1.0), stg_perturbations=create_batched_stg_config(1, blocks=None))
    print(f"# guided loop: capture + warmup + {args.guided_steps} steps", file=sys.stderr, flush=True)
    st = DenoiseState(model, args.height, args.width, args.frames, text_tokens=s, audio_frames=ta, seed=1,
                      sigmas=LTX2Scheduler().execute(steps=args.guided_steps))
    noise = (st.video_latent.clone(), st.audio_latent.clone())
    loop = CfgAvLoop(model, st, **kw).capture()

    def generation():
        st.video_latent.copy_(noise[0])
        st.audio_latent.copy_(noise[1])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loop.run()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    generation()
    wall = generation()
    finite = bool(torch.isfinite(st.video_latent.float()).all().item())
    del loop
    return {"ms_per_step": round(wall / args.guided_steps * 1e3, 3), "passes_per_step": 3,
            "passes": "stacked (one forward per step, M = 3 x tokens)", "steps": args.guided_steps,
            "timing": "hip-graph replay", "latents_finite": finite,
            "loop": "CfgAvLoop: CFG-star video 3.0 / audio 7.0 + STG 1.0 (all blocks), LTX2Scheduler sigmas"}


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: the denoise step runs whole on one MI355X (all 48 blocks' "
                                   "weights resident in its HBM) and is not sharded across GPUs", "n_gpus": args.gpus}))
        return 2
    if args.counter_workload:
        counter_workload(args.counter_workload, args.weights, args.counter_tile)
        return 0
    import torch

    from ltx_amd.components.patchifiers import audio_latent_frames, video_latent_grid
    from ltx_amd.kernels import gemm
    from ltx_amd.model.transformer.model import LTXModel
    from ltx_amd.pipeline import DenoiseState, denoise_step

    torch.backends.cuda.matmul.allow_tf32 = False
    grid = video_latent_grid(args.height, args.width, args.frames)
    tv = grid[0] * grid[1] * grid[2]
    ta = audio_latent_frames(args.frames) if args.audio_tokens is None else args.audio_tokens
    s = args.text_tokens
    print(f"# building {args.layers}-block model ({args.weights}) ...", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    model = LTXModel(num_layers=args.layers, weight_format=args.weights, seed=0)
    state = DenoiseState(model, args.height, args.width, args.frames, text_tokens=s, audio_frames=ta, seed=0)
    pes = model.rope(state.video_positions, state.audio_positions)
    torch.cuda.synchronize()
    print(f"# built in {time.perf_counter() - t0:.1f} s; weights {model.weight_bytes() / 1e9:.1f} GB",
          file=sys.stderr, flush=True)
    nsig = len(state.sigmas) - 1

    def run_step(i):
        denoise_step(model, state, i % nsig, pes)

    # warmup (eager), then optional graph capture of the 8 distinct steps
    run_step(0)
    torch.cuda.synchronize()
    graphs = None
    from ltx_amd.kernels import gemm as _gemm

    # the dominant kernel's launches (video FF up) get device clock stamps
    # inside the captured step graphs, so its duration is read from the timed
    # replays themselves; graph k also stamps the GEMM classes of
    # GEMM_CLASS_GRAPHS[k]
    def select(info, k):
        c = gemm_class(info, tv, ta, s)
        if c == "ff_up" or (not args.no_class_stamps and c in GEMM_CLASS_GRAPHS[k % len(GEMM_CLASS_GRAPHS)]):
            return c
        return None

    stamps = LaunchStamps(torch, nsig, select)
    if not args.no_graph:
        graphs = []
        pool = torch.cuda.graph_pool_handle()
        for i in range(nsig):
            g = torch.cuda.CUDAGraph()
            with stamps.capturing(i), torch.cuda.graph(g, pool=pool):
                run_step(i)
            graphs.append(g)
        torch.cuda.synchronize()
    do = (lambda i: graphs[i % nsig].replay()) if graphs else run_step
    for i in range(args.warmup):
        do(i)
    torch.cuda.synchronize()
    print(f"# warmup done; timing {args.steps} steps ({'graph' if graphs else 'eager'})", file=sys.stderr, flush=True)
    t_start = time.perf_counter()
    for i in range(args.steps):
        do(i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    ms = wall / args.steps * 1e3

    # dominant kernel (FF up-projection GEMM) and the GEMM classes: their
    # stamps in the last timed replay of each step graph (eager: stream
    # events, below)
    records = stamps.records() if graphs else []
    durs = [d for lab, _, d in records if lab == "ff_up"]
    timing = "device clock stamps around each launch in the timed HIP-graph replays (last replay of each step graph)"
    gemm_classes = gemm_class_summary(records) if records else None
    if not durs:
        durs, _, _ = gemm_step_profile(run_step, args.kernel_steps, tv, torch)
        timing = "stream events around each launch in eager steps"
    k_ms = sum(durs) / len(durs)
    k_flop = 2.0 * tv * 4096 * 16384
    achieved = k_flop / (k_ms * 1e-3) / 1e12
    # the kernel the automatic tile choice runs for this shape: the 8-wave
    # kernel for every weight format, its 256-row tiles for the first rows and
    # (when that shortens the partial last round, e.g. rows 3072-3455 of the
    # 3456-token step) 128-row tiles for the rest in a second launch; a launch
    # here is the product, i.e. both launches
    kname = f"gemm8_kernel<{args.weights},GELU>"
    roofline = {"bound": "mfma", "kernel": f"{kname} (video FF up, M={tv} K=4096 N=16384; bf16 MFMA; "
                                           "the automatic row split into 256- and 128-row tiles)",
                "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(kname, args.weights),
                "launch_us": round(k_ms * 1e3, 1), "launches_timed": len(durs),
                "launch_timing": timing,
                "algorithmic_flop_per_launch": k_flop}
    flops = step_flops(tv, ta, s, args.layers)
    out = {
        "metric": METRIC, "value": round(ms, 3), "unit": "ms/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init weights ~N(0,0.02), Gaussian latents and text context",
        "config": {"workload": f"48-block LTX-2.3 AV denoise step at {args.width}x{args.height}x{args.frames}"
                               if args.layers == 48 else f"{args.layers}-block AV denoise step",
                   "video_tokens": tv, "audio_tokens": ta, "text_tokens": s, "blocks": args.layers,
                   "weights": args.weights, "timing": "hip-graph replay, FF-up launches bracketed by device clock stamps" if graphs else "eager"},
        "tokens_per_s": round((tv + ta) / (ms * 1e-3), 1),
        "step_tflop": round(flops / 1e12, 2), "step_tflops_achieved": round(flops / (ms * 1e-3) / 1e12, 1),
        "ff_up_mfma_pct": round(100 * achieved / PEAK_BF16_TFLOPS, 1),
        "roofline": roofline,
        "gemm_classes": gemm_classes,
    }
    if gemm_classes and "video_stream" in gemm_classes:
        out["video_stream_gemm_mfma_pct"] = round(100 * gemm_classes["video_stream"]["frac_bf16_peak"], 1)
    del graphs
    if args.weights == "mxfp8" and not args.no_mx:
        print("# opt-in MX path: step graphs with MXFP8 activations", file=sys.stderr, flush=True)
        out["mx_opt_in"] = mx_opt_in_leg(model, state, pes, torch, tv, ta, s)
    if not args.no_clip_768x512x121 and args.layers == 48:
        print("# 768x512x121: 48-block MXFP8 step graphs", file=sys.stderr, flush=True)
        out["clip_768x512x121"] = clip_768x512x121_leg(model, torch)
    if args.guided_steps > 0:
        out["guided_step"] = guided_step_ms(model, args, ta, s)
    del model, state
    torch.cuda.empty_cache()
    if not args.no_video_only and ta:
        print("# video-only step graphs", file=sys.stderr, flush=True)
        out["video_only"] = video_only_leg(args, torch, s)
        out["av_minus_video_ms"] = round(ms - out["video_only"]["ms_per_step"], 3)
    if not args.no_attention_leg:
        print("# attention calls", file=sys.stderr, flush=True)
        out["attention"] = attention_leg(torch)
    if not args.no_gemm_shapes:
        print("# one block (bf16): video and AV", file=sys.stderr, flush=True)
        out["per_block"] = per_block_leg(torch, args, ta, s)
    if not args.no_gemm_shapes:
        print("# projection GEMM shapes at M=3456", file=sys.stderr, flush=True)
        out["gemm_shapes"] = {fmt: gemm_shapes(torch, fmt) for fmt in ("int8", "mxfp8", "bf16")}
    if not args.no_fused_bench:
        print("# fused ops", file=sys.stderr, flush=True)
        out["fused_ops"] = fused_op_bandwidth(torch)
        out["fused_ops"]["T3456_768x512x65"] = fused_op_bandwidth(torch, T=3456)
        out["fused_ops"]["T1296_512x288x65"] = fused_op_bandwidth(torch, T=1296)
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(ROOT))
        print("# cpu baseline (oracle block on host cores) ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(tv, ta, s, args.layers, grid, runs=args.cpu_runs)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
