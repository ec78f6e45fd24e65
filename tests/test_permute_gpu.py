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


def test_permute_errors(dev):
    with pytest.raises(mtk.MtkError) as e:
        mtk.PermutePlan(dev, 0, 4, 3, 3, 3)
    assert e.value.status == mtk.MTK_ERR_INVALID
    plan = mtk.PermutePlan(dev, 8, 8, 1, 1, 1)
    buf = dev.empty(8 * 8 * 2 * 2)
    with pytest.raises(mtk.MtkError) as e:  # overlapping source and destination
        plan.run(buf, buf.ptr + 16)
    assert "overlap" in e.value.message
