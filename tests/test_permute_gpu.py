"""OIDHW -> DHWIO weight re-layout on the GPU (C ABI: mtk_permute_plan / mtk_permute_run) against the
oracle's restatement of the reference kernel (ConvolutionShared.swift:4606-4627). Exact: the
reference validates it with tolerance 0 (validateFlatOutput, 5381-5406)."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle
from oracle import generators as gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [
    (1, 1, 1, 1, 1), (5, 3, 1, 3, 3), (96, 64, 3, 3, 3),   # odd sizes: 2-byte path; C*T, O % 8: 16-byte
    (128, 128, 3, 3, 3), (70, 130, 1, 1, 1), (512, 512, 3, 3, 3),  # the reference's profile shape (AGENTS.md:51)
    (256, 256, 1, 3, 3),
])
def test_permute_exact(dev, shape):
    print(f"[permute] OIDHW {shape}", flush=True)
    w = oracle.normal(140, shape)
    got = mtk.permute_oidhw_to_dhwio(dev, w)
    exp = oracle.permute_oidhw_to_dhwio(w)
    assert np.array_equal(got.view(np.uint16), exp.view(np.uint16))


def _sweep_shapes():
    rng = np.random.default_rng(4606)
    return [tuple(int(v) for v in (rng.integers(1, 300), rng.integers(1, 300), rng.integers(1, 4), rng.integers(1, 6),
                                   rng.integers(1, 6))) for _ in range(24)]


@pytest.mark.parametrize("shape", _sweep_shapes())
def test_permute_sweep_exact(dev, shape):
    # seeded random O, I and filter extents (both load widths, ragged everything): bit exact
    print(f"[permute sweep] OIDHW {shape}", flush=True)
    w = oracle.normal(141, shape)
    got = mtk.permute_oidhw_to_dhwio(dev, w)
    assert np.array_equal(got.view(np.uint16), oracle.permute_oidhw_to_dhwio(w).view(np.uint16))


def test_permute_then_conv(dev):
    # the reference's PermuteThenTensorOpSession3D: OIDHW weights re-laid out on the GPU feed the
    # conv kernel and give the DHWIO conv's result bit for bit
    d = oracle.ConvDims.conv3d(N=1, D=5, H=9, W=10, C=64, O=64, PF=1, PBk=1, PT=1, PB=1, PL=1, PR=1)
    x = gen.conv3d_activation(d)
    w = gen.conv3d_weights(d)
    w_oidhw = np.ascontiguousarray(np.transpose(w, (4, 3, 0, 1, 2)))
    w2 = mtk.permute_oidhw_to_dhwio(dev, w_oidhw)
    assert np.array_equal(w2.view(np.uint16), w.view(np.uint16))
    y1 = mtk.conv(dev, d, x, w2)
    y0 = mtk.conv(dev, d, x, w)
    assert np.array_equal(y1.view(np.uint16), y0.view(np.uint16))


def _oidhw(w):
    """DHWIO [KD][KH][KW][C][O] (or HWIO) -> OIDHW [O][C][KD][KH][KW] (or OIHW), exact."""
    return np.ascontiguousarray(np.transpose(w, (w.ndim - 1, w.ndim - 2) + tuple(range(w.ndim - 2))))


@pytest.mark.parametrize("case", [
    dict(rank=3, N=1, D=5, H=9, W=10, C=64, O=64, PF=1, PBk=1, PT=1, PB=1, PL=1, PR=1),  # fast gather
    dict(rank=3, N=2, D=6, H=7, W=8, C=128, O=96, SZ=2, SY=1, SX=2, DY=2, PT=2, PB=2),  # strided, dilated
    dict(rank=2, N=2, H=17, W=19, C=64, O=72, PT=1, PB=1, PL=1, PR=1),                 # OIHW, rank 2
    dict(rank=3, N=1, D=4, H=6, W=7, C=24, O=20, PL=1, PR=1),                          # generic gather, 2-byte re-layout
    dict(rank=2, N=1, H=11, W=9, C=3, O=10, PT=1, PB=1, PL=1, PR=1),                   # 2-byte activation loads
])
@pytest.mark.parametrize("bias", [False, True])
def test_oidhw_conv_plan(dev, case, bias):
    # the reference's PermuteThenTensorOpSession3D (ConvolutionShared.swift:1676-1857) as one plan:
    # each run re-lays the OIDHW weights out in the workspace and convolves from there; bit-exact
    # against the oracle (integer generators: exact fp32 sums) and against permute-then-conv
    case = dict(case)
    rank = case.pop("rank")
    d = (oracle.ConvDims.conv3d if rank == 3 else oracle.ConvDims.conv2d)(**case)
    x, w = gen.conv3d_activation(d), gen.conv3d_weights(d)
    b = gen.conv3d_bias(d) if bias else None
    if rank == 2:
        w = w.reshape(d.KH, d.KW, d.C, d.O)
    print(f"[oidhw conv] rank {rank} {case} bias={bias}", flush=True)
    y = mtk.conv(dev, d, x, _oidhw(w), b, weight_layout="OIDHW")
    exp = oracle.conv(d, x, w.reshape(d.w_shape()), b).astype(np.float16).reshape(y.shape)
    assert np.array_equal(y.view(np.uint16), exp.view(np.uint16))
    y2 = mtk.conv(dev, d, x, mtk.permute_oidhw_to_dhwio(dev, _oidhw(w).reshape(d.O, d.C, d.KD, d.KH, d.KW)), b)
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16))


@pytest.mark.parametrize("case", [
    dict(rank=3, N=1, D=5, H=9, W=10, C=64, O=64, PF=1, PBk=1, PT=1, PB=1, PL=1, PR=1),
    dict(rank=2, N=2, H=13, W=15, C=128, O=256, PT=1, PB=1, PL=1, PR=1),
    dict(rank=3, N=2, D=6, H=7, W=8, C=40, O=36, SZ=2, SX=2, DY=2, PT=2, PB=2),
])
def test_oidhw_random_data(dev, case):
    # on seeded U[-1, 1) data (inexact sums) the OIDHW plan gives the DHWIO convolution's result bit
    # for bit (the re-layout moves bits; the convolution is the same kernel on the same operands)
    case = dict(case)
    rank = case.pop("rank")
    d = (oracle.ConvDims.conv3d if rank == 3 else oracle.ConvDims.conv2d)(**case)
    rng = np.random.default_rng(5)
    x = rng.uniform(-1, 1, d.x_shape()).astype(np.float16)
    w = rng.uniform(-1, 1, d.w_shape()).astype(np.float16)
    b = rng.uniform(-1, 1, (d.O,)).astype(np.float16)
    wo = np.ascontiguousarray(np.transpose(w, (4, 3, 0, 1, 2)))  # [O][C][KD][KH][KW]
    if rank == 2:
        w, wo = w.reshape(d.KH, d.KW, d.C, d.O), wo.reshape(d.O, d.C, d.KH, d.KW)
    print(f"[oidhw random] rank {rank} {case}", flush=True)
    y = mtk.conv(dev, d, x, wo, b, weight_layout="OIDHW")
    assert np.array_equal(y.view(np.uint16), mtk.conv(dev, d, x, w, b).view(np.uint16))


def test_oidhw_conv_reference_profile_shape(dev):
    # the reference's permute + conv profile (AGENTS.md:49-53): N1 D3 256x256 C=O=512 3x3x3, no
    # padding; integer generators (exact fp32 sums, |sum| <= 4158): the fused plan equals the
    # DHWIO plan bit for bit and sampled output rows equal the oracle bit for bit
    d = oracle.ConvDims.conv3d(N=1, D=3, H=256, W=256, C=512, O=512)
    x, w = gen.conv3d_activation(d), gen.conv3d_weights(d)
    y = mtk.conv(dev, d, x, _oidhw(w), weight_layout="OIDHW")
    y0 = mtk.conv(dev, d, x, w)
    assert np.array_equal(y.view(np.uint16), y0.view(np.uint16))
    rows = y.reshape(-1, d.OW, d.O)
    for r0 in (0, 101, 253):
        exp = oracle.conv(d, x, w, rows=(r0, r0 + 1)).reshape(-1, d.OW, d.O)[r0]
        assert np.array_equal(rows[r0].view(np.uint16), exp.astype(np.float16).view(np.uint16)), r0


def test_oidhw_conv_errors(dev):
    d = oracle.ConvDims.conv3d(N=1, D=3, H=8, W=8, C=64, O=64)
    plan = mtk.ConvPlan(dev, mtk.conv_desc(d, weight_layout="OIDHW"))
    assert plan.workspace_bytes == 64 * 64 * 27 * 2
    x, w, y = dev.empty(3 * 8 * 8 * 64 * 2), dev.empty(64 * 64 * 27 * 2), dev.empty(6 * 6 * 64 * 2)
    with pytest.raises(mtk.MtkError) as e:  # no workspace
        plan.run(x, w, None, y)
    assert e.value.status == mtk.MTK_ERR_INVALID
    with pytest.raises(mtk.MtkError) as e:  # workspace overlapping the weights
        plan.run(x, w, None, y, w.ptr + 256)
    assert "overlap" in e.value.message
    for layout in (2, 7):  # only DHWIO (0) and OIDHW (1)
        bad = mtk.conv_desc(d)
        bad.weight_layout = layout
        with pytest.raises(mtk.MtkError) as e:
            mtk.ConvPlan(dev, bad)
        assert e.value.status == mtk.MTK_ERR_INVALID
    for b in (x, w, y):
        b.free()
    # a workspace placed right after weights whose size is not a multiple of 256 bytes does not
    # overlap them (the workspace is the weight size rounded up; the weights' extent is exact)
    d = oracle.ConvDims.conv3d(N=1, D=3, H=8, W=8, C=8, O=12)  # 3*3*3*8*12*2 = 5184 bytes
    plan = mtk.ConvPlan(dev, mtk.conv_desc(d, weight_layout="OIDHW"))
    wb = 27 * 8 * 12 * 2
    assert plan.workspace_bytes == (wb + 255) // 256 * 256
    x, y = dev.empty(3 * 8 * 8 * 8 * 2), dev.empty(6 * 6 * 12 * 2)
    both = dev.empty(wb + 16 + plan.workspace_bytes)
    ws = (both.ptr + wb + 15) // 16 * 16
    plan.run(x, both.ptr, None, y, ws)  # accepted: w ends where the workspace begins
    with pytest.raises(mtk.MtkError) as e:
        plan.run(x, both.ptr, None, y, ws - 16)
    assert "overlap" in e.value.message
    dev.sync()
    for b in (x, y, both):
        b.free()


def test_permute_errors(dev):
    with pytest.raises(mtk.MtkError) as e:
        mtk.PermutePlan(dev, 0, 4, 3, 3, 3)
    assert e.value.status == mtk.MTK_ERR_INVALID
    plan = mtk.PermutePlan(dev, 8, 8, 1, 1, 1)
    buf = dev.empty(8 * 8 * 2 * 2)
    with pytest.raises(mtk.MtkError) as e:  # overlapping source and destination
        plan.run(buf, buf.ptr + 16)
    assert "overlap" in e.value.message
