"""GEMM parity over a seeded sweep of shapes that crosses every plan the library can choose.

Each case draws M, N, K, split-K, dtype and the layout of B from a fixed seed, builds the plan
through the C ABI and checks the whole output against the CPU oracle (matmul.swift:498-510) with
the acceptance of test_gemm_gpu.check (relative Frobenius <= 1e-3, element-wise dot-product bound).
The case list is fixed by the seed; the CPU test below checks that it reaches every kernel family
(decode: one or two reductions, long partitions, partial-writing; tiles: direct or register-staged,
one pass, two-pass or in-workgroup split-K), so a planner change that drops a family from the sweep
fails on the CPU as well."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle

from test_gemm_gpu import check


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    bands = [(1, 16), (17, 32), (33, 700)]
    while len(out) < 36:
        lo, hi = bands[len(out) % 3]
        M = int(rng.integers(lo, hi + 1))
        trans_b = bool(rng.integers(0, 4) > 0)  # mostly B [N][K], the decode layout
        K = int(rng.choice([64, 520, 1024, 2048, 4096, 4100, 9000, 14336, 30000]))
        if rng.integers(0, 3) == 0:
            K += int(rng.integers(-7, 8))  # ragged K (a multiple of 8 or not)
        N = int(rng.choice([48, 333, 1000, 4096, 8211, 16384])) + int(rng.integers(0, 3)) * 17
        split = int(rng.choice([0, 1, 2, 3, 4, 5, 8, 12, 30]))
        dtype = "bf16" if rng.integers(0, 2) else "f16"
        if (M * K + N * K) > 40_000_000 or M * N * K > 30e9:
            continue
        out.append((M, N, K, split, dtype, trans_b))
    # grids that fill the device: the in-workgroup split-K schedule (ragged M, K not a multiple of 64)
    out += [(3000, 4096, 1536, 4, "bf16", True), (4096, 4096, 2056, 4, "f16", True)]
    return out


CASES = _cases()


def _family(desc):
    for key in ("mtk_skinny_few_", "mtk_skinny_parts_", "_long", "mtk_skinny_"):
        if key in desc:
            return key
    if "_s" in desc.split("kernels:")[-1].split()[0][-2:]:
        return "tile in-workgroup split-K"
    if "splitk_reduce" in desc:
        return "tile two-pass"
    return "tile one pass"


def test_sweep_reaches_every_plan():
    # CPU: the planner alone (no device), on the sweep's cases
    fams = {}
    for M, N, K, split, dtype, trans_b in CASES:
        d = mtk.GemmPlan(None, M, N, K, dtype=dtype, has_bias=True, split_k=split, trans_b=trans_b).describe()
        fams.setdefault(_family(d), []).append((M, N, K, split))
    for want in ("mtk_skinny_few_", "mtk_skinny_parts_", "_long", "mtk_skinny_", "tile in-workgroup split-K", "tile two-pass",
                 "tile one pass"):
        assert want in fams, (want, sorted(fams))


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_plan_sweep(dev, case):
    M, N, K, split, dtype, trans_b = CASES[case]
    A = oracle.normal(300 + case, (M, K), 0, 1, dtype)
    B = oracle.normal(400 + case, (N, K) if trans_b else (K, N), 0, 1 / np.sqrt(K), dtype)
    bias = oracle.normal(500 + case, (N,), 0, 0.05, dtype)
    d = mtk.GemmPlan(dev, M, N, K, dtype=dtype, has_bias=True, split_k=split, trans_b=trans_b).describe()
    print(f"[sweep {case}] {d}", flush=True)
    check(dev, A, B, bias, trans_b=trans_b, dtype=dtype, split_k=split, label=f"sweep {case}")
