"""Run one benchmark workload a fixed number of times, for profilers (rocprofv3 --kernel-trace /
--pmc). Inputs are the seeded synthetic tensors of the matching benchmark configuration, uploaded
once; only the plan's kernels run in the loop.

    python -m example_matmul_metal4_amd.profile_case gemm --split 4 --iters 20
    python -m example_matmul_metal4_amd.profile_case gemm --split 4 --mode two_pass --iters 20
    python -m example_matmul_metal4_amd.profile_case copy --iters 20   # calibration: plain copy

Cases: gemm (config 2, 4096 x 4096 x 4100 + bias, B [N][K]), gemm_nn (4096^3, B [K][N]), decode
(config 3, bf16 M=16, 3 rotating input copies), conv2d / conv3d (config 4), attn / attn_causal
(config 5), attn_bwd / attn_bwd_causal (the backward at the config 5 shape), attn_gqa8 /
attn_bwd_gqa8 (forward / backward at the config 5 shape with 8 K/V heads), permute (OIDHW -> DHWIO
weight re-layout, 512 x 512 x 3x3x3, 3 rotating source copies), copy (torch's device-to-device copy
of 256 MiB: known HBM traffic of 256 MiB read and 256 MiB written per launch, used to scale the
FETCH_SIZE / WRITE_SIZE counters).
"""
import argparse
import sys

import numpy as np


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("case", choices=["gemm", "gemm_nn", "decode", "conv2d", "conv3d", "attn", "attn_causal", "attn_bwd",
                                     "attn_bwd_causal", "attn_gqa8", "attn_bwd_gqa8", "permute", "copy"])
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--split", type=int, default=4)
    ap.add_argument("--tile", type=int, default=0)
    ap.add_argument("--mode", choices=["auto", "two_pass", "serial"], default="auto",
                    help="split-K schedule of the gemm case")
    ap.add_argument("--rows", type=int, default=0, help="query rows per workgroup of the attention cases")
    a = ap.parse_args(argv)

    if a.case == "copy":
        import torch

        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(a.iters):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy: {a.iters} x {n} bytes", flush=True)
        return 0

    import example_matmul_metal4_amd as mtk
    from example_matmul_metal4_amd import inputs

    dev = mtk.Device(0)
    try:
        if a.case == "gemm":
            M = N = 4096
            K = 4100
            plan = mtk.GemmPlan(dev, M, N, K, has_bias=True, split_k=a.split, tile=a.tile, split_mode=a.mode)
            ws = dev.empty(plan.workspace_bytes) if plan.workspace_bytes else None
            sets = [plan.args(dev.upload(inputs.normal(1, (M, K), 0, 1 / np.sqrt(K))),
                              dev.upload(inputs.normal(2, (N, K), 0, 1 / np.sqrt(K))),
                              dev.upload(inputs.uniform(3, (N,), -0.5, 0.5)), dev.empty(M * N * 2), ws)]
        elif a.case == "gemm_nn":
            M = N = K = 4096
            plan = mtk.GemmPlan(dev, M, N, K, has_bias=True, split_k=1, trans_b=False, tile=a.tile)
            sets = [plan.args(dev.upload(inputs.normal(1, (M, K), 0, 1 / np.sqrt(K))),
                              dev.upload(inputs.normal(2, (K, N), 0, 1 / np.sqrt(K))),
                              dev.upload(inputs.uniform(3, (N,), -0.5, 0.5)), dev.empty(M * N * 2), None)]
        elif a.case == "decode":
            M, N, K = 16, 14336, 4096
            plan = mtk.GemmPlan(dev, M, N, K, dtype="bf16", has_bias=True, split_k=8)
            sets = [plan.args(dev.upload(inputs.normal(4 + 100 * c, (M, K), 0, 1, "bf16")),
                              dev.upload(inputs.normal(5 + 100 * c, (N, K), 0, 0.02, "bf16")),
                              dev.upload(inputs.normal(6 + 100 * c, (N,), 0, 0.02, "bf16")), dev.empty(M * N * 2))
                    for c in range(3)]
        elif a.case in ("conv2d", "conv3d"):
            if a.case == "conv2d":
                dims = dict(rank=2, N=8, D=1, H=128, W=128, C=256, O=256, KD=1, KH=3, KW=3,
                            pad_top=1, pad_bottom=1, pad_left=1, pad_right=1)
            else:
                dims = dict(rank=3, N=1, D=16, H=64, W=64, C=128, O=128, KD=3, KH=3, KW=3, pad_front=1, pad_back=1,
                            pad_top=1, pad_bottom=1, pad_left=1, pad_right=1)
            desc = mtk.ConvDesc(stride_d=1, stride_h=1, stride_w=1, dil_d=1, dil_h=1, dil_w=1, has_bias=1,
                                dtype=mtk.F16, **dims)
            plan = mtk.ConvPlan(dev, desc)
            xs = (desc.N, desc.D, desc.H, desc.W, desc.C)
            wsh = (desc.KD, desc.KH, desc.KW, desc.C, desc.O)
            sets = [plan.args(dev.upload(inputs.uniform(7, xs, -1, 1)), dev.upload(inputs.uniform(8, wsh, -1, 1)),
                              dev.upload(inputs.uniform(9, (desc.O,), -1, 1)),
                              dev.empty(int(np.prod(plan.out_shape())) * 2))]
        elif a.case == "permute":
            wsh = (512, 512, 3, 3, 3)
            plan = mtk.PermutePlan(dev, *wsh)
            dst = dev.empty(int(np.prod(wsh)) * 2)
            sets = [plan.args(dev.upload(inputs.normal(14 + 100 * c, wsh)), dst) for c in range(3)]
        elif a.case in ("attn_gqa8", "attn_bwd_gqa8"):
            shp, kvs = (2, 4096, 32, 128), (2, 4096, 8, 128)
            fwd = mtk.AttentionPlan(dev, 2, 32, 4096, 4096, 128, H_kv=8)
            q, k, v = (dev.upload(inputs.normal(20 + i, s_)) for i, s_ in enumerate((shp, kvs, kvs)))
            o, lse = dev.empty(int(np.prod(shp)) * 2), dev.empty(2 * 32 * 4096 * 4)
            if a.case == "attn_gqa8":
                plan, sets = fwd, [fwd.args(q, k, v, o, lse)]
            else:
                fwd.run(q, k, v, o, lse)
                plan = mtk.AttentionBwdPlan(dev, 2, 32, 4096, 4096, 128, H_kv=8)
                sets = [plan.args(q, k, v, o, dev.upload(inputs.normal(23, shp)), lse,
                                  *(dev.empty(int(np.prod(s_)) * 2) for s_ in (shp, kvs, kvs)),
                                  dev.empty(plan.workspace_bytes))]
        elif a.case in ("attn_bwd", "attn_bwd_causal"):
            causal = a.case == "attn_bwd_causal"
            shp = (2, 4096, 32, 128)
            fwd = mtk.AttentionPlan(dev, 2, 32, 4096, 4096, 128, causal=causal)
            q, k, v = (dev.upload(inputs.normal(s, shp)) for s in (10, 11, 12))
            o, lse = dev.empty(int(np.prod(shp)) * 2), dev.empty(2 * 32 * 4096 * 4)
            fwd.run(q, k, v, o, lse)
            plan = mtk.AttentionBwdPlan(dev, 2, 32, 4096, 4096, 128, causal=causal)
            sets = [plan.args(q, k, v, o, dev.upload(inputs.normal(13, shp)), lse,
                              *(dev.empty(int(np.prod(shp)) * 2) for _ in range(3)), dev.empty(plan.workspace_bytes))]
        else:
            plan = mtk.AttentionPlan(dev, 2, 32, 4096, 4096, 128, causal=a.case == "attn_causal", q_rows=a.rows)
            shp = (2, 4096, 32, 128)
            sets = [plan.args(dev.upload(inputs.normal(10, shp)), dev.upload(inputs.normal(11, shp)),
                              dev.upload(inputs.normal(12, shp)), dev.empty(int(np.prod(shp)) * 2))]
        print(plan.describe(), flush=True)
        for i in range(a.iters):
            plan.launch(sets[i % len(sets)])
        dev.sync()
        print(f"{a.case}: {a.iters} runs done", flush=True)
    finally:
        dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
