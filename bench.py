#!/usr/bin/env python3
"""Benchmark of the MI355X tensor-op path (BASELINE.json metric), one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--quick]

Headline (``value``): BASELINE config 2 -- fp16 GEMM + bias, M = N = 4096, K = 4100, split-K 4,
B stored [N][K] (the reference's default layout), A, B ~ N(0,1)/sqrt(K), bias ~ U[-0.5, 0.5),
fp32 accumulate, fp16 out. A step is one run of the path (split-K GEMM + reduce) over resident
inputs; three input copies rotate so the 256 MB Infinity Cache cannot serve repeats. The K timed
steps are submitted as one HIP graph (the reference encodes its duplicatedCount dispatches into one
command buffer the same way); ``eager_ms_per_step`` times the same K steps launched one by one.
``value`` = 2*M*N*K / (wall time per step), in TFLOP/s.

``roofline`` describes the dominant kernel of the headline step: achieved = algorithmic FLOPs per
launch / that kernel's average duration (HIP events on the stream it runs on), peak = MI355X's
published dense fp16 MFMA rate (2.5 PFLOP/s). ``traffic`` comes from the committed rocprofv3
--pmc FETCH_SIZE / WRITE_SIZE measurement of the same kernel (profiles/traffic.json) when present.

``cpu_baseline``: the CPU oracle (C restatement of matmul.swift:498-510, fp32 sequential
accumulation, OpenMP over rows) timed on this host on a bounded row sample of the same GEMM.

``configs``: every other BASELINE configuration measured the same way (split-K 1 variant of
config 2, the bf16 decode GEMM in GB/s, conv2d / conv3d, flash attention fwd both masks), plus the
attention backward at the config 5 shape, attention forward and backward with 8 grouped K/V heads
at that shape, the OIDHW -> DHWIO convolution-weight re-layout (GB/s) and the reference's own
default GEMM run (M=32, N=3072, K=80000, split-K 30; GB/s).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2500.0  # MI355X published dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_steps(dev, plan, arg_sets, warmup, steps):
    """Exactly `steps` runs, submitted as one HIP graph (the reference's duplicatedCount
    dispatches in one command buffer, matmul.swift:447-449) after `warmup` untimed runs, timed by
    wall clock between device syncs. The same `steps` runs launched one call at a time are timed
    the same way and reported alongside (eager). Per-kernel averages come from HIP events
    (mtk_profile) in a separate pass."""
    g_warm = plan.graph(arg_sets, warmup) if warmup > 0 else None
    g = plan.graph(arg_sets, steps)
    try:
        if g_warm is not None:
            g_warm.launch()
        dev.sync()
        t0 = time.perf_counter()
        g.launch()
        dev.sync()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    finally:
        g.close()
        if g_warm is not None:
            g_warm.close()
    t0 = time.perf_counter()
    for i in range(steps):
        plan.launch(arg_sets[i % len(arg_sets)])
    dev.sync()
    eager_ms = (time.perf_counter() - t0) * 1e3 / steps
    prof = plan.profile(arg_sets, warmup=1, iters=steps)
    return wall_ms, eager_ms, prof


def gemm_case(dev, mtk, inputs, M, N, K, dtype, split_k, seeds, dists, copies=3, tile=0, split_mode="auto"):
    plan = mtk.GemmPlan(dev, M, N, K, trans_b=True, dtype=dtype, has_bias=True, split_k=split_k, tile=tile,
                        split_mode=split_mode)
    C = dev.empty(M * N * 2)
    ws = dev.empty(plan.workspace_bytes) if plan.workspace_bytes else None
    sets = []
    for c in range(copies):
        A = dists[0](inputs, seeds[0] + 100 * c, (M, K), dtype)
        B = dists[1](inputs, seeds[1] + 100 * c, (N, K), dtype)
        bias = dists[2](inputs, seeds[2] + 100 * c, (N,), dtype)
        sets.append(plan.args(dev.upload(A), dev.upload(B), dev.upload(bias), C, ws))
    return plan, sets


def summarize(name, plan, timing, bound, key=None):
    """One configuration's line. Kernel rates use the sum of the plan's per-step kernel times (every
    kernel of a multi-kernel plan, each averaged over the profiled launches), so they cover the
    whole step's work. HIP event pairs around a launch add a few microseconds of their own, so when
    that sum exceeds the graph's wall time per step (short kernels), the graph time is used."""
    wall_ms, eager_ms, prof = timing
    flops, byts = plan.work()
    kern = max(prof["kernels"].items(), key=lambda kv: kv[1])
    events_ms = sum(prof["kernels"].values())
    kernel_ms, source = (events_ms, "HIP events, sum over the plan's kernels") if events_ms <= wall_ms else (
        wall_ms, "graph wall time per step (the event-timed sum exceeds it)")
    out = {"workload": name, "plan": plan.describe(), "ms_per_step": wall_ms, "eager_ms_per_step": eager_ms,
           "tflops": flops / (wall_ms * 1e-3) / 1e12, "pct_mfma_peak": 100 * flops / (wall_ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS,
           "kernels_ms": prof["kernels"], "kernels_total_ms": kernel_ms, "kernel_time_source": source,
           "dominant_kernel": kern[0], "traffic": traffic_for(f"{kern[0]}@{key}") if key else None}
    if bound == "hbm":
        out["gbs"] = byts / (wall_ms * 1e-3) / 1e9
        out["pct_hbm_peak"] = 100 * out["gbs"] / PEAK_HBM_GBS
        out["kernel_gbs"] = byts / (kernel_ms * 1e-3) / 1e9
    else:
        out["kernel_tflops"] = flops / (kernel_ms * 1e-3) / 1e12
    return out


def host_threads():
    """Host threads for the CPU baselines: every CPU this process may run on, capped by
    OMP_NUM_THREADS when the environment sets it (the GPU box sets it to its CPU share per GPU)."""
    cpus = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return (min(cpus, int(env)) if env.isdigit() and int(env) > 0 else cpus), cpus


def cpu_baseline(target_s=10.0):
    """Oracle GEMM (config 2 shape) on a growing row sample until ~target_s of CPU work."""
    import oracle

    threads, cpus = host_threads()
    M, N, K = 4096, 4096, 4100
    B = oracle.normal(2, (N, K), 0, 1 / np.sqrt(K))
    bias = oracle.uniform(3, (N,), -0.5, 0.5)
    rows, el, reps = 16, 0.0, 1
    while True:
        A = oracle.normal(1, (rows, K), 0, 1 / np.sqrt(K))
        t0 = time.perf_counter()
        oracle.gemm(A, B, bias, trans_b=True, threads=threads)
        el = time.perf_counter() - t0
        if el >= target_s or rows >= M:
            break
        rows = min(M, rows * 2 if el < target_s / 4 else int(rows * target_s / max(el, 1e-3)) + 1)
    if el < target_s:  # whole GEMM done in less than the target: repeat it for a stable time
        reps = max(1, int(target_s / max(el, 1e-3)))
        t0 = time.perf_counter()
        for _ in range(reps):
            oracle.gemm(A, B, bias, trans_b=True, threads=threads)
        el = (time.perf_counter() - t0) / reps
    tflops = 2.0 * rows * N * K / el / 1e12
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": tflops, "unit": "TFLOP/s", "cores": threads, "host_cpus": cpus,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "kind": "port",
            "sample": f"oracle_gemm (fp32 sequential accumulate, matmul.swift:498-510) on {rows} of the 4096 rows "
                      f"of config 2 (M=N=4096, K=4100, bias), {el:.2f} s per run averaged over {reps} run(s), "
                      f"{threads} threads ({cpus} CPUs in this process's affinity, OMP_NUM_THREADS="
                      f"{os.environ.get('OMP_NUM_THREADS')}) of {cpu}"}


def cpu_baselines_other(target_s=3.0):
    """The CPU oracle on bounded samples of the other MFMA-bound configurations:
    attention (config 5, Network.swift:134-179 / 286-311 restated) on a block of query rows of
    every (b, h), conv2d (config 4a, ConvolutionShared.swift:4994-5026) on a block of output rows.
    Each sample grows until it takes about target_s seconds; TFLOP/s counts the sampled work."""
    import oracle

    threads, _ = host_threads()
    out = {}
    Q = oracle.normal(10, (2, 4096, 32, 128))
    K = oracle.normal(11, (2, 4096, 32, 128))
    V = oracle.normal(12, (2, 4096, 32, 128))
    rows = 4
    while True:
        t0 = time.perf_counter()
        oracle.attention(Q, K, V, rows=(0, rows), threads=threads)
        el = time.perf_counter() - t0
        if el >= target_s or rows >= 4096:
            break
        rows = min(4096, max(rows * 2, int(rows * target_s / max(el, 1e-3)) + 1))
    out["config5_attn"] = {"value": 4.0 * 2 * 32 * rows * 4096 * 128 / el / 1e12, "unit": "TFLOP/s", "cores": threads,
                           "kind": "port", "sample": f"oracle_attention on query rows 0..{rows - 1} of every (b, h) "
                                                     f"of config 5 (non-causal), {el:.2f} s"}
    dims = oracle.ConvDims.conv2d(N=8, H=128, W=128, C=256, O=256, PT=1, PB=1, PL=1, PR=1)
    x = oracle.uniform(7, dims.x_shape(), -1, 1)
    w = oracle.uniform(8, dims.w_shape(), -1, 1)
    b = oracle.uniform(9, (dims.O,), -1, 1)
    nrows = 2
    total = dims.N * dims.OH
    while True:
        t0 = time.perf_counter()
        oracle.conv(dims, x, w, b, rows=(0, nrows), threads=threads)
        el = time.perf_counter() - t0
        if el >= target_s or nrows >= total:
            break
        nrows = min(total, max(nrows * 2, int(nrows * target_s / max(el, 1e-3)) + 1))
    out["config4a_conv2d"] = {"value": 2.0 * nrows * dims.OW * dims.O * 9 * dims.C / el / 1e12, "unit": "TFLOP/s",
                              "cores": threads, "kind": "port",
                              "sample": f"oracle_conv on output rows 0..{nrows - 1} (of {total}) of config 4a, {el:.2f} s"}
    return out


def traffic_for(key):
    """HBM bytes per launch of kernel@workload from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    measurement (profiles/traffic.json, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return t.get(key, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Under a sustained MFMA load the card runs its first launches fast, then pulls its clock down
    # for a few milliseconds and settles in between (headline kernel: 164-171 us, then 205-225 us,
    # then 177-189 us per launch); the default warm-up reaches the settled state before anything
    # is timed. --warmup / --steps time exactly what they ask for.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only (no other configs)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="", help="comma-separated prefixes of the other configs' keys to measure "
                                               "(default: all); the headline always runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the tensor-op path on a single MI355X and has no "
              f"multi-GPU mode (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import example_matmul_metal4_amd as mtk
    from example_matmul_metal4_amd import inputs

    dev = mtk.Device(0)
    info = dev.info
    log(f"[bench] {info['name']} {info['arch']} CUs={info['compute_units']} clock={info['clock_khz']} kHz "
        f"computed dense f16 peak={info['peak_f16_tflops']:.1f} TFLOP/s")

    nrm = lambda s: (lambda inp, seed, shape, dt: inp.normal(seed, shape, 0, s, dt))
    uni = lambda lo, hi: (lambda inp, seed, shape, dt: inp.uniform(seed, shape, lo, hi, dt))

    # ---- headline: config 2
    M = N = 4096
    K = 4100
    plan, sets = gemm_case(dev, mtk, inputs, M, N, K, "f16", 4, (1, 2, 3),
                           (nrm(1 / np.sqrt(K)), nrm(1 / np.sqrt(K)), uni(-0.5, 0.5)))
    log(f"[bench] headline plan: {plan.describe()}")
    wall_ms, eager_ms, prof = time_steps(dev, plan, sets, args.warmup, args.steps)
    flops, byts = plan.work()
    value = flops / (wall_ms * 1e-3) / 1e12
    gemm_kernel = next(k for k in plan.describe().split("kernels:")[1].split() if k.startswith("mtk_gemm_"))
    kms = prof["kernels"][gemm_kernel]
    achieved = flops / (kms * 1e-3) / 1e12
    log(f"[bench] config2 split-K 4: {wall_ms:.4f} ms/step = {value:.1f} TFLOP/s (graph; eager launches "
        f"{eager_ms:.4f} ms/step); kernels {prof['kernels']}")

    line = {
        "metric": "TFLOP/s + % MFMA peak: fp16 GEMM 4096^3+bias, flash-attn fwd, conv2d, 1 GPU",
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall_ms,
        "eager_ms_per_step": eager_ms,
        "submission": f"the {args.steps} timed steps as one HIP graph (mtk_graph_*); eager_ms_per_step: same "
                      "steps launched one call at a time",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded SplitMix64: A,B ~ N(0,1)/sqrt(K), bias ~ U[-0.5,0.5)); 3 rotating input copies",
        "config": {"workload": "BASELINE config 2: fp16 GEMM C = A.B^T + bias, M=N=4096, K=4100, split-K=4, "
                               "B [N][K], fp32 accumulate, fp16 out; split-K run in-workgroup (the 4 K partitions "
                               "in sequence per output tile, fp32 partition sums parked and added in partition "
                               "order, bias last: the two-pass schedule's arithmetic, one kernel)",
                   "M": M, "N": N, "K": K, "split_k": 4, "pct_mfma_peak": 100 * value / PEAK_F16_TFLOPS},
        "roofline": {"bound": "mfma", "kernel": gemm_kernel, "achieved": achieved, "peak": PEAK_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_F16_TFLOPS, "traffic": traffic_for(f"{gemm_kernel}@config2_splitk4"),
                     "algorithmic_flops_per_launch": flops, "kernel_ms": kms},
    }

    # ---- other BASELINE configs (each its own plan, same timing method)
    if not args.quick:
        cfgs = {}
        steps = max(10, args.steps // 2)  # the other configs: half the headline's step count
        only = [o for o in args.only.split(",") if o]
        want = lambda *keys: not only or any(k.startswith(o) for k in keys for o in only)
        try:
            if want("config2_splitk1"):
                p1, s1 = gemm_case(dev, mtk, inputs, M, N, K, "f16", 1, (1, 2, 3),
                                   (nrm(1 / np.sqrt(K)), nrm(1 / np.sqrt(K)), uni(-0.5, 0.5)))
                tm = time_steps(dev, p1, s1, args.warmup, steps)
                cfgs["config2_splitk1"] = summarize("config 2 without split-K (split_k=1)", p1, tm, "mfma",
                                                    key="config2_splitk1")
            if want("config2_splitk4_two_pass"):
                p2, s2 = gemm_case(dev, mtk, inputs, M, N, K, "f16", 4, (1, 2, 3),
                                   (nrm(1 / np.sqrt(K)), nrm(1 / np.sqrt(K)), uni(-0.5, 0.5)), split_mode="two_pass")
                tm = time_steps(dev, p2, s2, args.warmup, steps)
                cfgs["config2_splitk4_two_pass"] = summarize(
                    "config 2, split-K 4 in the two-pass schedule (partition workgroups + reduce kernel)", p2, tm, "mfma",
                    key="config2_splitk4_two_pass")
            if want("config3_decode"):
                p3, s3 = gemm_case(dev, mtk, inputs, 16, 14336, 4096, "bf16", 8, (4, 5, 6),
                                   (nrm(1.0), nrm(0.02), nrm(0.02)), copies=3)
                tm = time_steps(dev, p3, s3, args.warmup, steps * 4)
                cfgs["config3_decode"] = summarize("config 3: bf16 M=16 N=14336 K=4096 split-K 8 + bias (HBM-bound)",
                                                   p3, tm, "hbm", key="config3_decode")
            if want("reference_main_large_k"):
                # the reference's own default run (matmul.swift:334): M=32, N=3072, K=80000, split-K 30;
                # HBM-bound (B is 491 MB), three rotating input copies
                p4, s4 = gemm_case(dev, mtk, inputs, 32, 3072, 80000, "f16", 30, (50, 51, 52),
                                   (nrm(1 / np.sqrt(80000)), nrm(1 / np.sqrt(80000)), uni(-0.5, 0.5)))
                tm = time_steps(dev, p4, s4, args.warmup, steps)
                cfgs["reference_main_large_k"] = summarize("reference main(): f16 M=32 N=3072 K=80000 split-K 30 + bias",
                                                           p4, tm, "hbm", key="reference_main_large_k")
            for key, dims in (("config4a_conv2d", dict(rank=2, N=8, D=1, H=128, W=128, C=256, O=256, KD=1, KH=3, KW=3,
                                                           pad_top=1, pad_bottom=1, pad_left=1, pad_right=1)),
                                  ("config4b_conv3d", dict(rank=3, N=1, D=16, H=64, W=64, C=128, O=128, KD=3, KH=3, KW=3,
                                                           pad_front=1, pad_back=1, pad_top=1, pad_bottom=1, pad_left=1,
                                                           pad_right=1))):
                    if not want(key):
                        continue
                    desc = mtk.ConvDesc(stride_d=1, stride_h=1, stride_w=1, dil_d=1, dil_h=1, dil_w=1, has_bias=1,
                                        dtype=mtk.F16, **dims)
                    pc = mtk.ConvPlan(dev, desc)
                    shape = pc.out_shape()
                    xs = (desc.N, desc.D, desc.H, desc.W, desc.C)
                    ws_ = (desc.KD, desc.KH, desc.KW, desc.C, desc.O)
                    y = dev.empty(int(np.prod(shape)) * 2)
                    sets_c = [pc.args(dev.upload(inputs.uniform(7 + 100 * c, xs, -1, 1)),
                                      dev.upload(inputs.uniform(8 + 100 * c, ws_, -1, 1)),
                                      dev.upload(inputs.uniform(9 + 100 * c, (desc.O,), -1, 1)), y) for c in range(3)]
                    tm = time_steps(dev, pc, sets_c, args.warmup, steps)
                    cfgs[key] = summarize(pc.describe().split(" kernels:")[0], pc, tm, "mfma", key=key)
                # the reference's published convolution profiles (its only published numbers, M5 iPad
                # GPU time): conv2d N1 256x256 C=O=512 3x3 at 9.71 TFLOP/s (AGENTS.md:23) and conv3d
                # N1 D3 256x256 C=O=512 3x3x3 at 9.18 TFLOP/s (AGENTS.md:49-52; largeProfileDimensions,
                # convolution3d.swift:1316-1334); no padding, stride 1; seeded U[-1,1) data
            for key, dims, m5 in (("reference_profile_conv2d", dict(rank=2, N=1, D=1, H=256, W=256, C=512, O=512, KD=1,
                                                                        KH=3, KW=3), 9.71),
                                      ("reference_profile_conv3d", dict(rank=3, N=1, D=3, H=256, W=256, C=512, O=512, KD=3,
                                                                        KH=3, KW=3), 9.18)):
                    if not want(key, "reference_profile_permute_conv3d"):
                        continue
                    desc = mtk.ConvDesc(stride_d=1, stride_h=1, stride_w=1, dil_d=1, dil_h=1, dil_w=1, has_bias=0,
                                        dtype=mtk.F16, **dims)
                    pc = mtk.ConvPlan(dev, desc)
                    shape = pc.out_shape()
                    xs = (desc.N, desc.D, desc.H, desc.W, desc.C)
                    ws_ = (desc.KD, desc.KH, desc.KW, desc.C, desc.O)
                    y = dev.empty(int(np.prod(shape)) * 2)
                    sets_c = [pc.args(dev.upload(inputs.uniform(30 + 100 * c, xs, -1, 1)),
                                      dev.upload(inputs.uniform(31 + 100 * c, ws_, -1, 1)), None, y) for c in range(3)]
                    tm = time_steps(dev, pc, sets_c, args.warmup, steps)
                    cfgs[key] = summarize(pc.describe().split(" kernels:")[0], pc, tm, "mfma", key=key)
                    cfgs[key]["reference_m5_tflops"] = m5
                    if desc.rank == 3:
                        # the reference's permute + conv3d session at this shape (AGENTS.md:49-53: 9.07
                        # TFLOP/s on M5): OIDHW weights re-laid out in the workspace by each run, then the
                        # same convolution; TFLOP/s counts the convolution's FLOPs only, as there
                        desc.weight_layout = mtk.WEIGHTS_OIDHW
                        pf = mtk.ConvPlan(dev, desc)
                        ws_f = dev.empty(pf.workspace_bytes)
                        sets_f = [pf.args(sc.x, dev.upload(inputs.uniform(31 + 100 * c, (desc.O, desc.C, desc.KD, desc.KH,
                                                                                           desc.KW), -1, 1)),
                                          None, y, ws_f) for c, sc in enumerate(sets_c)]
                        tm = time_steps(dev, pf, sets_f, args.warmup, steps)
                        s = summarize(pf.describe().split(" kernels:")[0], pf, tm, "mfma", key="reference_profile_permute_conv3d")
                        s["reference_m5_tflops"] = 9.07
                        s["overhead_vs_dhwio_pct"] = 100.0 * (tm[0] / cfgs[key]["ms_per_step"] - 1.0)
                        cfgs["reference_profile_permute_conv3d"] = s
            if want("conv_weight_permute"):
                # OIDHW -> DHWIO weight re-layout at the reference's profile shape (512 x 512, 3x3x3;
                # AGENTS.md:51), HBM-bound: 40 rotating source copies (566 MB with the destination) so the
                # 256 MB Infinity Cache cannot serve the repeats
                pp = mtk.PermutePlan(dev, 512, 512, 3, 3, 3)
                wsh = (512, 512, 3, 3, 3)
                dst = dev.empty(int(np.prod(wsh)) * 2)
                wsrc = inputs.normal(14, wsh)
                sets_p = [pp.args(dev.upload(wsrc), dst) for c in range(40)]
                tm = time_steps(dev, pp, sets_p, args.warmup, steps * 4)
                cfgs["conv_weight_permute"] = summarize("OIDHW -> DHWIO weight re-layout, O = C = 512, 3x3x3 (f16)", pp, tm,
                                                        "hbm", key="conv_weight_permute")
                cfgs["conv_weight_permute"]["reference_m5_ms"] = 3.42  # AGENTS.md:51
            for causal in (False, True):
                    if not want("config5_attn" + ("_causal" if causal else ""), "config5_attn_bwd" + ("_causal" if causal else "")):
                        continue
                    pa = mtk.AttentionPlan(dev, 2, 32, 4096, 4096, 128, causal=causal)
                    shp = (2, 4096, 32, 128)
                    o = dev.empty(int(np.prod(shp)) * 2)
                    sets_a = [pa.args(dev.upload(inputs.normal(10 + 100 * c, shp)), dev.upload(inputs.normal(11 + 100 * c, shp)),
                                      dev.upload(inputs.normal(12 + 100 * c, shp)), o) for c in range(2)]
                    tm = time_steps(dev, pa, sets_a, args.warmup, steps)
                    s = summarize(f"config 5: flash-attn fwd B=2 H=32 S=4096 D=128 {'causal' if causal else 'non-causal'}",
                                  pa, tm, "mfma", key="config5_causal" if causal else "config5")
                    s["reference_convention_tflops"] = (2 * 128 + 5) * 4096 * 4096 * 32 * 2 / (
                        2 if causal else 1) / (tm[0] * 1e-3) / 1e12
                    cfgs["config5_attn_causal" if causal else "config5_attn"] = s
                    # backward of the same shape (the reference's Network.swift gradients): O and lse from
                    # this forward, dO ~ N(0,1); FLOPs = five products of 2 S^2 D per (b, h)
                    pb = mtk.AttentionBwdPlan(dev, 2, 32, 4096, 4096, 128, causal=causal)
                    ws_b = dev.empty(pb.workspace_bytes)
                    grads = [dev.empty(int(np.prod(shp)) * 2) for _ in range(3)]
                    sets_b = []
                    for c, sa in enumerate(sets_a):
                        o_c, lse_c = dev.empty(int(np.prod(shp)) * 2), dev.empty(2 * 32 * 4096 * 4)
                        pa.run(sa.Q, sa.K, sa.V, o_c, lse_c)
                        sets_b.append(pb.args(sa.Q, sa.K, sa.V, o_c, dev.upload(inputs.normal(13 + 100 * c, shp)), lse_c,
                                              *grads, ws_b))
                    dev.sync()
                    tm = time_steps(dev, pb, sets_b, args.warmup, steps)
                    cfgs["config5_attn_bwd_causal" if causal else "config5_attn_bwd"] = summarize(
                        f"config 5 shape, flash-attn backward (dQ, dK, dV) {'causal' if causal else 'non-causal'}", pb, tm,
                        "mfma", key="config5_bwd_causal" if causal else "config5_bwd")
            if want("config5_attn_gqa8", "config5_attn_bwd_gqa8"):
                # grouped K/V heads at the config 5 shape (the reference's Hq / Hk; here Hq = 32, Hk = 8):
                # forward and backward, non-causal
                pg = mtk.AttentionPlan(dev, 2, 32, 4096, 4096, 128, H_kv=8)
                pgb = mtk.AttentionBwdPlan(dev, 2, 32, 4096, 4096, 128, H_kv=8)
                kvs = (2, 4096, 8, 128)
                sets_g, sets_gb = [], []
                ws_g = dev.empty(pgb.workspace_bytes)
                grads = [dev.empty(int(np.prod(s_)) * 2) for s_ in (shp, kvs, kvs)]
                for c in range(2):
                    q_c, k_c, v_c = (dev.upload(inputs.normal(20 + i + 100 * c, s_)) for i, s_ in enumerate((shp, kvs, kvs)))
                    o_c, lse_c = dev.empty(int(np.prod(shp)) * 2), dev.empty(2 * 32 * 4096 * 4)
                    sets_g.append(pg.args(q_c, k_c, v_c, o_c, lse_c))
                    pg.run(q_c, k_c, v_c, o_c, lse_c)
                    sets_gb.append(pgb.args(q_c, k_c, v_c, o_c, dev.upload(inputs.normal(23 + 100 * c, shp)), lse_c,
                                            *grads, ws_g))
                dev.sync()
                tm = time_steps(dev, pg, sets_g, args.warmup, steps)
                cfgs["config5_attn_gqa8"] = summarize("config 5 shape with 8 K/V heads (H=32, H_kv=8), flash-attn fwd",
                                                      pg, tm, "mfma", key="config5_gqa8")
                tm = time_steps(dev, pgb, sets_gb, args.warmup, steps)
                cfgs["config5_attn_bwd_gqa8"] = summarize(
                    "config 5 shape with 8 K/V heads (H=32, H_kv=8), flash-attn backward", pgb, tm, "mfma",
                    key="config5_bwd_gqa8")
            # other head dimensions at the config 5 shape (the reference's run(headDimension:),
            # attention.swift:398): D = 64, 256 and 512, both masks; the backward at D = 64 and 256
            for hd in (64, 256, 512):
                if not want(f"config5_attn_d{hd}"):
                    continue
                shp_d = (2, 4096, 32, hd)
                o = dev.empty(int(np.prod(shp_d)) * 2)
                sets_d = [None, None]
                for c in range(2):
                    sets_d[c] = (dev.upload(inputs.normal(10 + 100 * c, shp_d)), dev.upload(inputs.normal(11 + 100 * c, shp_d)),
                                 dev.upload(inputs.normal(12 + 100 * c, shp_d)))
                for causal in (False, True):
                    pd = mtk.AttentionPlan(dev, 2, 32, 4096, 4096, hd, causal=causal)
                    tm = time_steps(dev, pd, [pd.args(*t_, o) for t_ in sets_d], args.warmup, steps)
                    key = f"config5_attn_d{hd}" + ("_causal" if causal else "")
                    cfgs[key] = summarize(f"config 5 shape, head dimension {hd}, flash-attn fwd "
                                          f"{'causal' if causal else 'non-causal'}", pd, tm, "mfma", key=key)
                if hd > 256:  # the backward takes head dimensions up to 256
                    continue
                # the backward at this head dimension (non-causal): O and lse from the forward
                pdf = mtk.AttentionPlan(dev, 2, 32, 4096, 4096, hd)
                pdb = mtk.AttentionBwdPlan(dev, 2, 32, 4096, 4096, hd)
                ws_db = dev.empty(pdb.workspace_bytes)
                grads = [dev.empty(int(np.prod(shp_d)) * 2) for _ in range(3)]
                sets_db = []
                for c, t_ in enumerate(sets_d):
                    o_c, lse_c = dev.empty(int(np.prod(shp_d)) * 2), dev.empty(2 * 32 * 4096 * 4)
                    pdf.run(*t_, o_c, lse_c)
                    sets_db.append(pdb.args(*t_, o_c, dev.upload(inputs.normal(13 + 100 * c, shp_d)), lse_c, *grads,
                                            ws_db))
                dev.sync()
                tm = time_steps(dev, pdb, sets_db, args.warmup, steps)
                key = f"config5_attn_bwd_d{hd}"
                cfgs[key] = summarize(f"config 5 shape, head dimension {hd}, flash-attn backward (dQ, dK, dV) "
                                      "non-causal", pdb, tm, "mfma", key=key)
        except Exception as e:  # report what was measured; the headline stands on its own
            cfgs["error"] = repr(e)
        line["configs"] = cfgs
        for k, v in cfgs.items():
            if isinstance(v, dict):
                log(f"[bench] {k}: {v.get('ms_per_step', 0):.4f} ms (eager {v.get('eager_ms_per_step', 0):.4f}), "
                    f"{v.get('tflops', 0):.1f} TFLOP/s ({v.get('pct_mfma_peak', 0):.1f}% MFMA peak)"
                    + (f", {v['gbs']:.0f} GB/s" if 'gbs' in v else ""))

    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        log(f"[bench] cpu baseline: {line['cpu_baseline']}")
        if not args.quick:
            line["cpu_baselines_other"] = cpu_baselines_other()
            log(f"[bench] cpu baselines (other configs): {line['cpu_baselines_other']}")
    else:
        line["cpu_baseline"] = None
    dev.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
