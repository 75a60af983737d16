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
                its average launch time from stream events around every such
                launch in eager steps run right after the timed region (the
                timed region replays HIP graphs, which take no events);
                ``traffic`` = HBM bytes per launch from the rocprofv3
                FETCH_SIZE / WRITE_SIZE summary committed in profiles/ for
                this kernel and weight format (null when none matches);
  fused_ops     HBM GB/s of adaln_norm_fused / gated_add_fused at the
                reference's test shape (T=14640, C=4096) over a >512 MB buffer
                rotation (no Infinity-Cache reuse), launches replayed from a
                HIP graph (kernel time, not host dispatch);
  guided_step   ms per step of the CFG/STG guided loop (three transformer
                passes: positive, negative prompt, STG-perturbed; CFG-star and
                STG guidance; Euler), eager launches;
  cpu_baseline  the oracle (CPU restatement of the reference block) timed on
                this host for one AV block at the same shapes, x48.
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
    ap.add_argument("--counter-workload", choices=["ff-up", "ff-up-vs-library", "copy"], default=None,
                    help="run only a short workload for rocprofv3 --pmc passes and exit: the video FF "
                         "up-projection GEMM (4 launches, --weights format) or a 1 GiB device copy (3 "
                         "launches, the FETCH_SIZE / WRITE_SIZE calibration)")
    return ap.parse_args(argv)


def counter_workload(kind: str, weights: str) -> None:
    import torch

    from ltx_amd.kernels import gemm

    if kind == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
    elif kind == "ff-up-vs-library":
        # the FF up-projection shape through the vendor library (hipBLASLt,
        # plain bf16 linear) and through this library's bf16 and MXFP8 GEMMs
        g = torch.Generator(device="cuda").manual_seed(0)
        x = torch.randn((3456, 4096), generator=g, device="cuda").bfloat16()
        w = (torch.randn((16384, 4096), generator=g, device="cuda") * 0.02).bfloat16()
        b = torch.zeros(16384, device="cuda")
        wb, wm = gemm.make_weight(w, b, kind="bf16"), gemm.make_weight(w, b, kind="mxfp8")
        for _ in range(3):
            torch.nn.functional.linear(x, w)
            gemm.linear(x, wb, tile=gemm.TILE_256)
            gemm.linear(x, wm, tile=gemm.TILE_256)
    else:
        g = torch.Generator(device="cuda").manual_seed(0)
        x = torch.randn((3456, 4096), generator=g, device="cuda").bfloat16()
        w = (torch.randn((16384, 4096), generator=g, device="cuda") * 0.02).bfloat16()
        wt = gemm.make_weight(w, torch.zeros(16384, device="cuda"), kind=weights)
        out = torch.empty((3456, 16384), dtype=torch.bfloat16, device="cuda")
        for _ in range(4):
            gemm.linear(x, wt, epilogue=gemm.EPI_GELU, out=out)
    torch.cuda.synchronize()
    print(f"counter workload {kind} ({weights}) done", flush=True)


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


def fused_op_bandwidth(torch):
    """adaln / gated_add HBM GB/s at T=14640, C=4096: the kernels launched
    through their row-view launchers on preallocated buffers, inputs and
    outputs each rotating through >= 1.5 GB so neither operand can be served
    from the 256 MB last-level cache."""
    from ltx_amd.kernels.fused_ops import adaln_rows, gated_add_rows

    T, C = 14640, 4096
    nbytes = T * C * 2
    nbuf = max(2, math.ceil(1.5e9 / nbytes))
    xs = [torch.randn((T, C), device="cuda").bfloat16() for _ in range(nbuf)]
    bs = [torch.randn((T, C), device="cuda").bfloat16() for _ in range(nbuf)]
    outs = [torch.empty((T, C), device="cuda", dtype=torch.bfloat16) for _ in range(nbuf)]
    scale = torch.randn(C, device="cuda") * 0.1
    shift = torch.randn(C, device="cuda") * 0.1
    gate = torch.randn(C, device="cuda") * 0.5
    res = {}
    for name, fn, algo in (("adaln_norm_fused", lambda i: adaln_rows(xs[i], C, scale, shift, outs[(i + 1) % nbuf],
                                                                      C, T, C, 1e-6, 0),
                            2 * nbytes + 2 * C * 4),
                           ("gated_add_fused", lambda i: gated_add_rows(xs[i], C, bs[i], C, gate, outs[(i + 1) % nbuf],
                                                                        C, T, C, 0),
                            3 * nbytes + C * 4)):
        for i in range(nbuf):
            fn(i)
        torch.cuda.synchronize()
        # replayed from a HIP graph so host dispatch does not pace the ~45 us kernels
        iters = 8 * nbuf
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
    del xs, bs, outs
    return res


def cpu_baseline(tv: int, ta: int, s: int, layers: int, grid):
    """Oracle AV block at full shapes on the host, x layers."""
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
    t0 = time.perf_counter()
    ob.block(W, vx, ax, vada, aada, vctx, actx, *pes)
    dt = time.perf_counter() - t0
    return {"value": round(dt * layers * 1e3, 1), "unit": "ms/step", "cores": threads, "kind": "port",
            "sample": f"one AV block (oracle, torch-CPU fp32 with the reference's bf16 roundings) at "
                      f"{tv} video + {ta} audio + {s} text tokens, timed once ({dt:.2f} s) and x{layers} blocks; "
                      f"the reference's own MLX CPU backend is not installable here"}


def guided_step_ms(model, args, ta: int, s: int) -> dict:
    """ms per guided step of the CFG/STG loop (av_pipeline.py:625-757): the
    positive, negative-prompt and STG-perturbed transformer passes, CFG-star
    guidance (video 3.0, audio 7.0), STG (scale 1.0, video self-attention
    skipped in every block), Euler; shifted LTX-2 sigma schedule; eager."""
    import torch

    from ltx_amd.components.guiders import CFGStarRescalingGuider, STGGuider
    from ltx_amd.components.perturbations import create_batched_stg_config
    from ltx_amd.components.schedulers import LTX2Scheduler
    from ltx_amd.pipeline import DenoiseState, denoise_cfg_av

    kw = dict(video_guider=CFGStarRescalingGuider(3.0), audio_guider=CFGStarRescalingGuider(7.0),
              stg_guider=STGGuider(1.0), stg_perturbations=create_batched_stg_config(1, blocks=None))

    def run(steps):
        st = DenoiseState(model, args.height, args.width, args.frames, text_tokens=s, audio_frames=ta, seed=1,
                          sigmas=LTX2Scheduler().execute(steps=steps))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        denoise_cfg_av(model, st, **kw)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    print(f"# guided loop: warmup + {args.guided_steps} steps", file=sys.stderr, flush=True)
    run(2)  # the shifted schedule needs two steps for finite sigmas
    wall = run(args.guided_steps)
    return {"ms_per_step": round(wall / args.guided_steps * 1e3, 3), "passes_per_step": 3,
            "steps": args.guided_steps, "timing": "eager",
            "loop": "denoise_cfg_av: CFG-star video 3.0 / audio 7.0 + STG 1.0 (all blocks), LTX2Scheduler sigmas"}


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; the denoise step does not shard across GPUs "
                                   "here (see DESIGN.md for the sharding design)", "n_gpus": args.gpus}))
        return 2
    if args.counter_workload:
        counter_workload(args.counter_workload, args.weights)
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
    if not args.no_graph:
        graphs = []
        pool = torch.cuda.graph_pool_handle()
        for i in range(nsig):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
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

    # dominant kernel: FF up-projection GEMM, timed with stream events in eager steps
    ev = []

    def hook(phase, info):
        kind, m, n, k, epi = info
        if epi == gemm.EPI_GELU and m == tv and k == 4096:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            ev.append(e)

    gemm.LAUNCH_HOOK = hook
    try:
        for i in range(args.kernel_steps):
            run_step(i)
        torch.cuda.synchronize()
    finally:
        gemm.LAUNCH_HOOK = None
    durs = [ev[j].elapsed_time(ev[j + 1]) for j in range(0, len(ev), 2)]
    k_ms = sum(durs) / len(durs)
    k_flop = 2.0 * tv * 4096 * 16384
    achieved = k_flop / (k_ms * 1e-3) / 1e12
    kname = f"gemm_kernel<256,256,{args.weights},GELU>"
    roofline = {"bound": "mfma", "kernel": f"{kname} (video FF up, M={tv} K=4096 N=16384; bf16 MFMA)",
                "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(kname, args.weights),
                "launch_us": round(k_ms * 1e3, 1), "launches_timed": len(durs),
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
                   "weights": args.weights, "timing": "hip-graph replay" if graphs else "eager"},
        "tokens_per_s": round((tv + ta) / (ms * 1e-3), 1),
        "step_tflop": round(flops / 1e12, 2), "step_tflops_achieved": round(flops / (ms * 1e-3) / 1e12, 1),
        "gemm_mfma_pct": round(100 * achieved / PEAK_BF16_TFLOPS, 1),
        "roofline": roofline,
    }
    if not args.no_fused_bench or args.guided_steps > 0:
        del graphs
    if args.guided_steps > 0:
        out["guided_step"] = guided_step_ms(model, args, ta, s)
    if not args.no_fused_bench:
        out["fused_ops"] = fused_op_bandwidth(torch)
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(ROOT))
        print("# cpu baseline (oracle block on host cores) ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(tv, ta, s, args.layers, grid)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
