"""mtk_gemm_run_noalloc: mtk_gemm_run without a caller workspace and without any allocation (the
plan's workspace is the library's static device scratch), called through the C ABI and checked
against mtk_gemm_run on the same inputs: the same kernels, so the outputs must agree bit for bit.
Two calls in a row, the second with a smaller problem, for each split-K schedule."""
import ctypes

import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle

pytestmark = pytest.mark.gpu


def _run_both(dev, M, N, K, split_k, split_mode, seed, expect=None):
    A = oracle.normal(seed, (M, K), 0, 1 / np.sqrt(K))
    B = oracle.normal(seed + 1, (N, K), 0, 1 / np.sqrt(K))
    bias = oracle.uniform(seed + 2, (N,), -0.5, 0.5)
    plan = mtk.GemmPlan(dev, M, N, K, trans_b=True, has_bias=True, split_k=split_k, split_mode=split_mode)
    print(f"[noalloc] {plan.describe()} workspace={plan.workspace_bytes}", flush=True)
    if expect:
        assert expect in plan.describe(), plan.describe()
    assert 0 < plan.workspace_bytes <= (64 << 20)
    dA, dB, dbias = dev.upload(A), dev.upload(B), dev.upload(bias)
    c_ref, c_na = dev.empty(M * N * 2), dev.empty(M * N * 2)
    ws = dev.empty(plan.workspace_bytes)
    dev.fill_u16(c_na, 0x7E00, M * N)  # NaN: every element must be written
    plan.run(dA, dB, dbias, c_ref, ws)
    args = mtk.GemmArgs(A=dA.ptr, B=dB.ptr, bias=dbias.ptr, C=c_na.ptr, workspace=None)
    mtk._check(mtk.lib().mtk_gemm_run_noalloc(plan.handle, ctypes.byref(args)))
    dev.sync()
    ref = dev.download(c_ref, (M, N), np.float16)
    got = dev.download(c_na, (M, N), np.float16)
    for b in (dA, dB, dbias, c_ref, c_na, ws):
        b.free()
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), (M, N, K, split_k, split_mode)
    # and within the oracle's bar (fp32-accumulated GEMM, matmul.swift:498-510)
    r = oracle.compare(got.astype(np.float64), oracle.gemm(A, B, bias))
    assert r["ok"], r


@pytest.mark.parametrize("split_mode", ["serial", "two_pass"])
def test_noalloc_matches_run_two_calls(dev, split_mode):
    # first call: the larger problem; second call: a smaller one (the static scratch keeps the
    # first call's contents, which the second must not depend on)
    if split_mode == "serial":  # in-workgroup split-K: one fp32 tile per output tile
        _run_both(dev, 2048, 2048, 1100, 4, split_mode, 10)
        _run_both(dev, 512, 768, 700, 3, split_mode, 20)
    else:  # two-pass: fp32 partials [split_k][M][N], then the reduce kernel
        _run_both(dev, 1024, 1536, 2100, 8, split_mode, 30)
        _run_both(dev, 200, 300, 900, 4, split_mode, 40)


def test_noalloc_skinny_partials(dev):
    # the partial-writing skinny kernel (16 < M <= 32, long K: the reference's default run
    # M=32, N=3072, K=80000, split-K 30, matmul.swift:334) sets its partial pointer on its own launch
    # path; 30 fp32 partials of 32 x 3072 (11.8 MB) in the static scratch, then a smaller problem
    _run_both(dev, 32, 3072, 80000, 30, "auto", 60, expect="skinny partials")
    _run_both(dev, 24, 1000, 9000, 6, "auto", 70, expect="skinny partials")
    # decode shapes (M <= 16) whose partitions are longer than 512 K take the same kernel
    _run_both(dev, 16, 4096, 14336, 8, "auto", 80, expect="skinny partials M=16")
    _run_both(dev, 3, 1000, 10000, 5, "auto", 90, expect="skinny partials M=3")


def test_noalloc_config2_full_size(dev):
    # BASELINE config 2 (4096 x 4096 x 4100, split-K 4, in-workgroup): its 64 MiB workspace is the
    # scratch's whole size
    _run_both(dev, 4096, 4096, 4100, 4, "auto", 50)


def test_noalloc_errors(dev):
    plan = mtk.GemmPlan(dev, 4096, 4096, 4100, has_bias=False, split_k=4, split_mode="two_pass")
    assert plan.workspace_bytes > (64 << 20)
    buf = dev.empty(4096 * 4100 * 2)
    c = dev.empty(4096 * 4096 * 2)
    args = mtk.GemmArgs(A=buf.ptr, B=buf.ptr, bias=None, C=c.ptr, workspace=None)
    st = mtk.lib().mtk_gemm_run_noalloc(plan.handle, ctypes.byref(args))
    assert st == mtk.MTK_ERR_UNSUPPORTED and b"static scratch" in mtk.lib().mtk_last_error()
    small = mtk.GemmPlan(dev, 256, 256, 256, split_k=2, split_mode="two_pass")
    args = mtk.GemmArgs(A=buf.ptr, B=buf.ptr, bias=None, C=c.ptr, workspace=c.ptr)  # workspace must be NULL
    assert mtk.lib().mtk_gemm_run_noalloc(small.handle, ctypes.byref(args)) == mtk.MTK_ERR_INVALID
    dev.sync()
    buf.free()
    c.free()
