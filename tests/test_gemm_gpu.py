"""GEMM parity on the GPU, through the C ABI, against the CPU oracle (matmul.swift:498-510).

Acceptance (written out per test): relative Frobenius error <= 1e-3 and, element-wise,
|y - yhat| <= ulp_out(|yhat|) + 2 * K * 2^-24 * sum_k |a_k b_k| (oracle.dot_bound).
For bf16 outputs the Frobenius bar is 1e-3 plus the error of rounding the oracle itself to bf16
(a bf16 output alone carries ~1.1-1.7e-3 relative RMS rounding error, more than 1e-3)."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle

pytestmark = pytest.mark.gpu


def _f32(x, dtype):
    return oracle.to_f32(x, dtype).astype(np.float64)


def check(dev, A, B, bias, *, trans_b=True, dtype="f16", split_k=1, tile=0, rows=None, label=""):
    print(f"[gemm] {label} A{A.shape} B{B.shape} trans_b={trans_b} {dtype} split_k={split_k} tile={tile}", flush=True)
    got = mtk.gemm(dev, A, B, bias, trans_b=trans_b, dtype=dtype, split_k=split_k, tile=tile)
    exp = oracle.gemm(A, B, bias, trans_b=trans_b, dtype=dtype, rows=rows)
    a, b = _f32(A, dtype), _f32(B, dtype)
    if rows is not None:
        sel = slice(*rows)
        got, exp, a = got[sel], exp[sel], a[sel]
    absdot = np.abs(a) @ (np.abs(b).T if trans_b else np.abs(b))
    if bias is not None:
        absdot = absdot + np.abs(_f32(bias, dtype))
    rel_tol = 1e-3 + (oracle.rel_frobenius(oracle.to_f32(oracle.from_f32(exp, dtype), dtype), exp)
                      if dtype == "bf16" else 0.0)
    res = oracle.compare(_f32(got, dtype), exp, bound=oracle.dot_bound(exp, absdot, A.shape[1], dtype),
                         rel_tol=rel_tol)
    ref_tol = mtk.validate(got, exp, abs_tol=5e-3, dtype=dtype)  # the reference's own check, reported
    print(f"   rel_fro={res['rel_fro']:.3e} max_abs={res['max_abs']:.3e} worst/bound={res.get('worst_ratio', 0):.3f} "
          f"ref5e-3_mismatches={ref_tol['mismatches']}", flush=True)
    assert res["ok"], res
    return got, exp


def test_config1_256_cubed_nn_seed0(dev):
    # fp16 C = A.B, M=N=K=256, row-major, A and B from one U[-1,1) stream, seed 0.
    AB = oracle.uniform(0, (2, 256, 256), -1.0, 1.0)
    check(dev, AB[0], AB[1], None, trans_b=False, label="config1")


def test_fixtures(dev, golden_dir):
    fx = np.load(f"{golden_dir}/seeded.npz")
    got = mtk.gemm(dev, fx["gemm_nn_A"], fx["gemm_nn_B"], None, trans_b=False)
    assert oracle.compare(got.astype(np.float32), fx["gemm_nn_C"])["ok"]
    got = mtk.gemm(dev, fx["gemm_nt_A"], fx["gemm_nt_B"], fx["gemm_nt_bias"], trans_b=True)
    assert oracle.compare(got.astype(np.float32), fx["gemm_nt_C"])["ok"]
    got = mtk.gemm(dev, fx["gemm_bf16_A"], fx["gemm_bf16_B"], fx["gemm_bf16_bias"], trans_b=True, dtype="bf16")
    assert oracle.compare(oracle.to_f32(got, "bf16"), fx["gemm_bf16_C"], rel_tol=5e-3)["ok"]


@pytest.mark.parametrize("split_k", [1, 4, 5])
def test_all_ones_k4100_exact(dev, split_k):
    # fp32 sum = K + bias exactly; the f16 output is its round-to-nearest-even (4100 itself is
    # representable). The reference's split-K tail bug (matmul.swift:266-277 outside the split
    # branches) would give 4112 + bias with split-K = 4.
    M, N, K = 64, 96, 4100
    A = np.ones((M, K), np.float16)
    B = np.ones((N, K), np.float16)
    bias = np.arange(-8, N - 8, dtype=np.float16)
    got = mtk.gemm(dev, A, B, bias, split_k=split_k)
    exp = (K + bias.astype(np.float32)).astype(np.float16)
    assert np.array_equal(got, np.broadcast_to(exp, (M, N)))


@pytest.mark.parametrize("n", [1, 2, 3, 7, 16, 31, 33, 63, 64, 65, 127, 129, 200, 255, 257, 300])
@pytest.mark.parametrize("trans_b", [True, False])
def test_cube_sweep(dev, n, trans_b):
    # mirrors profileCorrectness (matmul.swift:338-343): M = N = K = i
    A = oracle.uniform(100 + n, (n, n), -1, 1)
    B = oracle.uniform(200 + n, (n, n), -1, 1)
    bias = oracle.uniform(300 + n, (n,), -0.5, 0.5)
    check(dev, A, B, bias, trans_b=trans_b, label=f"cube{n}")


@pytest.mark.parametrize("tile", [128, 256])
@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_ragged_tiles_dtypes(dev, tile, trans_b, dtype):
    M, N, K = 300, 264, 520  # edge tiles in M and N, K tail of 8, vec 8
    A = oracle.normal(1, (M, K), 0, 1, dtype)
    B = oracle.normal(2, (N, K) if trans_b else (K, N), 0, 1, dtype)
    bias = oracle.normal(3, (N,), 0, 1, dtype)
    check(dev, A, B, bias, trans_b=trans_b, dtype=dtype, tile=tile, label="ragged")


@pytest.mark.parametrize("K", [516, 4100, 129, 66])
def test_k_tails_and_vector_widths(dev, K):
    # B [N][K]: K = 516 / 4100 / 66 -> direct-to-LDS with an element-masked K tail (rows only 4- or
    # 8-byte aligned); K = 129 -> odd leading dimension, 2-byte scalar loads. B [K][N]: vec 4 / 1.
    M, N = 130, 72
    A = oracle.normal(4, (M, K), 0, 1)
    B = oracle.normal(5, (N, K), 0, 1)
    bias = oracle.uniform(6, (N,), -0.5, 0.5)
    check(dev, A, B, bias, label=f"K{K}")
    check(dev, A, np.ascontiguousarray(B.T), bias, trans_b=False, label=f"K{K}-nn")


@pytest.mark.parametrize("split_k", [2, 4, 7, 16])
def test_split_k(dev, split_k):
    M, N, K = 512, 512, 516  # reduced config 2
    A = oracle.normal(7, (M, K), 0, 1 / np.sqrt(K))
    B = oracle.normal(8, (N, K), 0, 1 / np.sqrt(K))
    bias = oracle.uniform(9, (N,), -0.5, 0.5)
    check(dev, A, B, bias, split_k=split_k, label="splitk")


def test_split_k_without_bias_and_odd_n(dev):
    M, N, K = 77, 61, 700  # N % 8 != 0 -> scalar reduce path
    A = oracle.normal(10, (M, K), 0, 1)
    B = oracle.normal(11, (N, K), 0, 1)
    check(dev, A, B, None, split_k=3, label="splitk-odd")


def test_config2_full_size(dev):
    # BASELINE config 2 at full size: M=N=4096, K=4100, split-K=4, bias; A,B ~ N(0,1)/sqrt(K),
    # bias ~ U[-0.5, 0.5). Every output element against the oracle (matmul.swift:498-510), for the
    # in-workgroup and the two-pass split-K schedules and for split-K 1.
    M = N = 4096
    K = 4100
    A = oracle.normal(1, (M, K), 0, 1 / np.sqrt(K))
    B = oracle.normal(2, (N, K), 0, 1 / np.sqrt(K))
    bias = oracle.uniform(3, (N,), -0.5, 0.5)
    exp = oracle.gemm(A, B, bias, trans_b=True)
    absdot = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)).T + np.abs(bias.astype(np.float64))
    bound = oracle.dot_bound(exp, absdot, K)
    for split_k, mode in ((4, "auto"), (4, "two_pass"), (1, "auto")):
        got = mtk.gemm(dev, A, B, bias, split_k=split_k, split_mode=mode)
        res = oracle.compare(got.astype(np.float64), exp, bound=bound)
        print(f"[gemm] config2 split_k={split_k} {mode}: {res}", flush=True)
        assert res["ok"], res


def test_strided_operands(dev):
    M, N, K = 96, 80, 200
    lda, ldb, ldc = 264, 208, 96
    A = oracle.normal(12, (M, lda), 0, 1)
    B = oracle.normal(13, (N, ldb), 0, 1)
    bias = oracle.normal(14, (N,), 0, 1)
    plan = mtk.GemmPlan(dev, M, N, K, has_bias=True, lda=lda, ldb=ldb, ldc=ldc)
    dA, dB, db = dev.upload(A), dev.upload(B), dev.upload(bias)
    dC = dev.upload(np.full((M, ldc), 7.0, np.float16))
    plan.run(dA, dB, db, dC)
    dev.sync()
    C = dev.download(dC, (M, ldc), np.float16)
    exp = oracle.gemm(np.ascontiguousarray(A[:, :K]), np.ascontiguousarray(B[:, :K]), bias)
    assert oracle.compare(C[:, :N].astype(np.float64), exp)["ok"]
    assert np.all(C[:, N:] == 7.0)  # padding columns untouched
    for b in (dA, dB, db, dC):
        b.free()


@pytest.mark.parametrize("M,N,K,lda,ldb,split_k", [
    (100, 96, 131, 132, 134, 1),   # odd K, even leading dimensions: last element ends mid-dword
    (70, 66, 131, 132, 132, 3),
    (64, 80, 40, 40, 40, 1),       # K below one 64-deep tile: the partial tile is the only tile
    (96, 64, 4100, 4100, 4100, 65),  # one K-tile per split: the last split holds only the partial tile
    (256, 256, 4101, 4102, 4104, 4),
])
def test_partial_last_k_tile(dev, M, N, K, lda, ldb, split_k):
    A = oracle.normal(50, (M, lda), 0, 1)
    B = oracle.normal(51, (N, ldb), 0, 1)
    bias = oracle.uniform(52, (N,), -0.5, 0.5)
    print(f"[gemm] partial K tile M={M} N={N} K={K} lda={lda} ldb={ldb} split_k={split_k}", flush=True)
    plan = mtk.GemmPlan(dev, M, N, K, has_bias=True, lda=lda, ldb=ldb, split_k=split_k)
    assert "direct-to-LDS" in plan.describe()
    dA, dB, db = dev.upload(A), dev.upload(B), dev.upload(bias)
    dC = dev.empty(M * N * 2)
    ws = dev.empty(plan.workspace_bytes) if plan.workspace_bytes else None
    plan.run(dA, dB, db, dC, ws)
    dev.sync()
    C = dev.download(dC, (M, N), np.float16)
    a, b = np.ascontiguousarray(A[:, :K]), np.ascontiguousarray(B[:, :K])
    exp = oracle.gemm(a, b, bias)
    absdot = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)).T + np.abs(bias.astype(np.float64))
    res = oracle.compare(C.astype(np.float64), exp, bound=oracle.dot_bound(exp, absdot, K))
    print(f"   {res}", flush=True)
    assert res["ok"], res
    for x in (dA, dB, db, dC, ws):
        if x is not None:
            x.free()


@pytest.mark.parametrize("M,N,K,trans_b,dtype,split_k,tile", [
    (256, 256, 256, True, "f16", 1, 0),
    (300, 200, 1000, True, "f16", 1, 0),     # ragged tiles, K tail on B only
    (300, 200, 1000, False, "f16", 3, 0),    # A [K][M] and B [K][N]: both operands K-major
    (512, 512, 4100, True, "bf16", 4, 256),
    (130, 514, 700, False, "bf16", 1, 128),
    (64, 96, 72, True, "f16", 2, 0),
])
def test_transpose_left(dev, M, N, K, trans_b, dtype, split_k, tile):
    # The reference's transpose.left: A stored [K][M] (matmul.swift:72-90). The oracle takes A as
    # [M][K], so it is given the host transpose of the same data.
    At = oracle.normal(60, (K, M), 0, 1 / np.sqrt(K), dtype)
    B = oracle.normal(61, (N, K) if trans_b else (K, N), 0, 1 / np.sqrt(K), dtype)
    bias = oracle.uniform(62, (N,), -0.5, 0.5, dtype)
    print(f"[gemm] transpose.left M={M} N={N} K={K} trans_b={trans_b} {dtype} split_k={split_k} tile={tile}",
          flush=True)
    got = mtk.gemm(dev, At, B, bias, trans_a=True, trans_b=trans_b, dtype=dtype, split_k=split_k, tile=tile)
    A = np.ascontiguousarray(At.T)
    exp = oracle.gemm(A, B, bias, trans_b=trans_b, dtype=dtype)
    a, b = _f32(A, dtype), _f32(B, dtype)
    absdot = np.abs(a) @ (np.abs(b).T if trans_b else np.abs(b)) + np.abs(_f32(bias, dtype))
    rel_tol = 1e-3 + (oracle.rel_frobenius(oracle.to_f32(oracle.from_f32(exp, dtype), dtype), exp)
                      if dtype == "bf16" else 0.0)
    res = oracle.compare(_f32(got, dtype), exp, bound=oracle.dot_bound(exp, absdot, K, dtype), rel_tol=rel_tol)
    print(f"   {res}", flush=True)
    assert res["ok"], res
    # same numbers as the default layout of the same data (different summation split: tolerance)
    ref = mtk.gemm(dev, A, B, bias, trans_b=trans_b, dtype=dtype, split_k=split_k, tile=tile)
    assert oracle.compare(_f32(got, dtype), _f32(ref, dtype), rel_tol=rel_tol)["ok"]


@pytest.mark.parametrize("M,N,K,lda,ldb,trans_a,trans_b,dtype,split_k,tile,k_stagger", [
    (512, 512, 4100, 0, 0, False, True, "f16", 4, 128, -1),     # K tail in the last partition
    (512, 512, 4100, 0, 0, False, True, "f16", 4, 128, 16),     # staggered partition ends
    (300, 200, 1000, 0, 0, False, False, "f16", 3, 128, 4),     # ragged tiles, B [K][N]
    (256, 256, 4101, 4102, 4104, False, True, "f16", 4, 256, 6),  # odd K, padded rows
    (64, 40, 200, 0, 0, False, True, "f16", 4, 256, -1),        # 4 K-tiles: the last partition is the partial tile
    (1024, 1024, 2048, 0, 0, False, True, "f16", 4, 256, 8),    # no K tail: the last partition ends at K
    (384, 320, 1536, 0, 0, True, True, "bf16", 2, 128, 10),     # A [K][M]
    (384, 320, 1500, 0, 0, True, False, "bf16", 3, 256, -1),    # A [K][M], B [K][N]
    (4096, 4096, 4100, 0, 0, False, True, "f16", 4, 0, 16),     # config 2 at full size, its default layout
])
def test_split_k_schedules_identical(dev, M, N, K, lda, ldb, trans_a, trans_b, dtype, split_k, tile, k_stagger):
    # In-workgroup split-K (partitions in sequence, running sum in the workspace, added in the
    # epilogue) and the two-pass schedule do the same arithmetic for one partition layout: the
    # outputs agree bit for bit; the in-workgroup one also passes the oracle check.
    a_shape = (K, lda or M) if trans_a else (M, lda or K)
    b_shape = (N, ldb or K) if trans_b else (K, ldb or N)
    A = oracle.normal(80, a_shape, 0, 1 / np.sqrt(K), dtype)
    B = oracle.normal(81, b_shape, 0, 1 / np.sqrt(K), dtype)
    bias = oracle.uniform(82, (N,), -0.5, 0.5, dtype)
    print(f"[gemm] split schedules M={M} N={N} K={K} lda={lda} ldb={ldb} trans_a={trans_a} trans_b={trans_b} "
          f"{dtype} split_k={split_k} tile={tile} k_stagger={k_stagger}", flush=True)
    dA, dB, db = dev.upload(A), dev.upload(B), dev.upload(bias)
    outs = {}
    for mode in ("serial", "two_pass"):
        plan = mtk.GemmPlan(dev, M, N, K, trans_a=trans_a, trans_b=trans_b, dtype=dtype, has_bias=True,
                            split_k=split_k, tile=tile, lda=lda, ldb=ldb, split_mode=mode, k_stagger=k_stagger)
        kernel = plan.describe().split()[-1]
        assert (kernel.rsplit("_", 1)[1][0] == "s") == (mode == "serial"), plan.describe()
        dC, ws = dev.empty(M * N * 2), dev.empty(plan.workspace_bytes)
        plan.run(dA, dB, db, dC, ws)
        dev.sync()
        outs[mode] = dev.download(dC, (M, N), np.uint16).copy()
        dC.free()
        ws.free()
    for x in (dA, dB, db):
        x.free()
    same = np.array_equal(outs["serial"], outs["two_pass"])
    print(f"   identical={same}", flush=True)
    assert same
    got = oracle.to_f32(outs["serial"], dtype).astype(np.float64)
    Ak = A[:, :M] if trans_a else A[:, :K]
    Ak = np.ascontiguousarray(Ak.T) if trans_a else np.ascontiguousarray(Ak)
    Bk = np.ascontiguousarray(B[:, :K] if trans_b else B[:, :N])
    rows = np.r_[0:min(M, 48), max(0, M - 16):M] if M > 1024 else np.arange(M)
    a = Ak[rows]
    exp = oracle.gemm(a, Bk, bias, trans_b=trans_b, dtype=dtype)
    af, bf = _f32(a, dtype), _f32(Bk, dtype)
    absdot = np.abs(af) @ (np.abs(bf).T if trans_b else np.abs(bf)) + np.abs(_f32(bias, dtype))
    rel_tol = 1e-3 + (oracle.rel_frobenius(oracle.to_f32(oracle.from_f32(exp, dtype), dtype), exp)
                      if dtype == "bf16" else 0.0)
    res = oracle.compare(got[rows], exp, bound=oracle.dot_bound(exp, absdot, K, dtype), rel_tol=rel_tol)
    print(f"   {res}", flush=True)
    assert res["ok"], res


def test_run_errors(dev):
    plan = mtk.GemmPlan(dev, 64, 64, 512, has_bias=True, split_k=2)
    assert plan.workspace_bytes == 2 * 64 * 64 * 4
    with pytest.raises(mtk.MtkError):
        plan.run(0, 0, 0, 0)
    dA = dev.empty(64 * 512 * 2)
    with pytest.raises(mtk.MtkError) as e:  # bias promised but missing
        plan.run(dA, dA, None, dA, dev.empty(plan.workspace_bytes))
    assert e.value.status == mtk.MTK_ERR_INVALID
    with pytest.raises(mtk.MtkError) as e:  # split-K plan needs its workspace
        plan.run(dA, dA, dA, dA, None)
    assert "workspace" in e.value.message


@pytest.mark.parametrize("tile", [0, 128, 256])
def test_reference_main_shape_large_k(dev, tile):
    # the reference's own default run (matmul.swift:334): M=32, N=3072, K=80000, split-K 30 (the
    # plan's choice, the partial-writing skinny kernel; 128x128 tiles; 256x256 tiles); every output
    # element is checked
    M, N, K = 32, 3072, 80000
    A = oracle.normal(50, (M, K), 0, 1 / np.sqrt(K))
    B = oracle.normal(51, (N, K), 0, 1 / np.sqrt(K))
    bias = oracle.uniform(52, (N,), -0.5, 0.5)
    check(dev, A, B, bias, split_k=30, tile=tile, label="reference main()")


def test_config3_decode_skinny_full_size(dev):
    # bf16 M=16, N=14336, K=4096, split-K=8, A ~ N(0,1), B ~ N(0,0.02),
    # bias ~ N(0,0.02), fp32 accumulate, bf16 out. Every output element is checked.
    M, N, K = 16, 14336, 4096
    A = oracle.normal(4, (M, K), 0, 1, "bf16")
    B = oracle.normal(5, (N, K), 0, 0.02, "bf16")
    bias = oracle.normal(6, (N,), 0, 0.02, "bf16")
    plan = mtk.GemmPlan(dev, M, N, K, dtype="bf16", has_bias=True, split_k=8)
    assert "skinny" in plan.describe() and "split_k=8" in plan.describe()
    check(dev, A, B, bias, dtype="bf16", split_k=8, label="config3")


@pytest.mark.parametrize("M,N,K,split_k,dtype", [
    (17, 1000, 4104, 5, "f16"), (32, 333, 2048, 2, "bf16"), (24, 4096, 16384, 0, "f16"), (32, 64, 2056, 3, "bf16"),
    (29, 130, 70000, 30, "f16"),
    # M <= 16 with partitions longer than 512 K (rows M..31 of the kernel's A read zero)
    (16, 4096, 14336, 8, "bf16"), (3, 1000, 10000, 5, "f16"), (1, 520, 2048, 2, "bf16")])
def test_skinny_partials_shapes(dev, M, N, K, split_k, dtype):
    # 16 < M <= 32 with long K, or M <= 16 with partitions longer than 512 K: the partial-writing
    # skinny kernel + the two-pass reduce (partitions of whole 64-element K-tiles; the last chunk
    # of a partition and the last partition ragged; N not a multiple of the 64-column block)
    plan = mtk.GemmPlan(dev, M, N, K, dtype=dtype, has_bias=True, split_k=split_k)
    assert "skinny partials" in plan.describe(), plan.describe()
    A = oracle.normal(60 + M, (M, K), 0, 1, dtype)
    B = oracle.normal(70 + M, (N, K), 0, 1 / np.sqrt(K), dtype)
    bias = oracle.normal(80 + M, (N,), 0, 0.05, dtype)
    check(dev, A, B, bias, dtype=dtype, split_k=split_k, label="skinny partials")
    check(dev, A, B, None, dtype=dtype, split_k=split_k, label="skinny partials, no bias")


@pytest.mark.parametrize("M,N,K,split_k,dtype", [
    (1, 4096, 4096, 8, "bf16"), (3, 100, 1000, 3, "f16"), (16, 64, 128, 1, "f16"), (7, 333, 2048, 2, "bf16"),
    (16, 14336, 4096, 4, "f16"), (16, 48, 4104, 8, "f16"),
    # persistent grid: more 16-column groups than workgroups, odd and even counts per workgroup
    (5, 8211, 512, 1, "f16"), (2, 9000, 2048, 1, "bf16"),
    # at most four groups per workgroup with split-K >= 4: one reduction (all groups in LDS);
    # the last group ragged; just past four groups per workgroup: reductions every two groups
    (16, 16384, 2048, 4, "bf16"), (9, 16000, 4096, 8, "f16"), (16, 16400, 4096, 8, "f16"),
    # many column groups per workgroup (several LDS reductions each); partitions shorter than
    # the 512 elements one load instruction covers
    (16, 60000, 256, 2, "bf16"), (4, 4097, 1024, 8, "f16"),
    # more columns per workgroup (4297) than the kernel keeps bias values for in LDS (8 per
    # thread: 512 at split-K 1): the bias is read from global memory in the reductions
    (2, 1100000, 64, 1, "f16")])
def test_skinny_shapes(dev, M, N, K, split_k, dtype):
    A = oracle.normal(20 + M, (M, K), 0, 1, dtype)
    B = oracle.normal(30 + M, (N, K), 0, 0.05, dtype)
    bias = oracle.normal(40 + M, (N,), 0, 0.05, dtype)
    check(dev, A, B, bias, dtype=dtype, split_k=split_k, label="skinny")
    check(dev, A, B, None, dtype=dtype, split_k=split_k, label="skinny-nobias")
