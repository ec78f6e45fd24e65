"""Convolution parity on the GPU (implicit GEMM, one launch for 2-D and 3-D), through the C ABI.

On the reference's integer-pattern generators every fp32 partial sum is exact, so the device
output must equal RNE_f16(oracle) bit for bit. Random inputs use the fp32-dot bound."""
import json
import os

import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle
from oracle import generators as gen

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CASES = json.load(open(os.path.join(ROOT, "tests", "golden", "cases.json")))


def _dims(kind, c):
    return oracle.ConvDims.conv2d(**c) if "2d" in kind else oracle.ConvDims.conv3d(**c)


def _run(dev, dims, x, w, bias=None, rank=None):
    desc = mtk.conv_desc(dims, has_bias=bias is not None, rank=rank)
    print(f"[conv] rank={desc.rank} {dims.as_dict()} bias={bias is not None}", flush=True)
    plan = mtk.ConvPlan(dev, desc)
    shape = plan.out_shape()
    dx, dw = dev.upload(x), dev.upload(w)
    db = dev.upload(bias) if bias is not None else None
    dy = dev.empty(int(np.prod(shape)) * 2)
    plan.run(dx, dw, db, dy)
    dev.sync()
    y = dev.download(dy, shape, np.float16)
    for buf in (dx, dw, db, dy):
        if buf is not None:
            buf.free()
    return y.reshape(dims.y_shape())


@pytest.mark.parametrize("kind", sorted(CASES))
def test_reference_case_lists_bit_exact(dev, kind):
    spec = CASES[kind]
    for c in spec["cases"]:
        dims = _dims(kind, c)
        if spec["generator"] == "conv2d_shared":
            x, w = gen.conv2d_shared_activation(dims), gen.conv2d_shared_weights(dims)
        else:
            x, w = gen.conv3d_activation(dims), gen.conv3d_weights(dims)
        for bias in (None, gen.conv3d_bias(dims)):
            y = _run(dev, dims, x, w, bias)
            exp = oracle.conv(dims, x, w, bias)
            assert np.array_equal(y.view(np.uint16), exp.astype(np.float16).view(np.uint16)), (kind, c)
            v = mtk.validate(y, exp, abs_tol=2e-2)  # the reference's validateOutput tolerance
            assert v["mismatches"] == 0


def test_probe_known_answers(dev, golden_dir):
    kat = json.load(open(os.path.join(golden_dir, "kat_probe.json")))
    dims = oracle.ConvDims.conv2d(N=1, H=5, W=5, C=1, O=1, PT=1, PB=1, PL=1, PR=1)
    x = gen.probe_activation().reshape(dims.x_shape())
    for name, w in (("centre_tap", gen.probe_centre_tap()), ("dense", gen.probe_dense())):
        y = _run(dev, dims, x, w.reshape(dims.w_shape()))
        assert np.array_equal(y.reshape(5, 5).astype(np.float64), np.array(kat[name]["expected"])), name


@pytest.mark.parametrize("c,o", [(64, 64), (128, 96), (64, 200), (8, 16), (16, 12), (4, 8), (3, 5), (24, 40)])
def test_channels_and_gathers(dev, c, o):
    # C % 64 == 0 -> fast gather; otherwise the generic gather with 8/4/1-wide loads
    dims = oracle.ConvDims.conv2d(N=2, H=11, W=13, C=c, O=o, PT=1, PB=1, PL=1, PR=1)
    x = gen.conv3d_activation(dims)
    w = gen.conv3d_weights(dims)
    b = gen.conv3d_bias(dims)
    y = _run(dev, dims, x, w, b)
    exp = oracle.conv(dims, x, w, b)
    assert np.array_equal(y.view(np.uint16), exp.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("rank,kd,kh,kw,o,n,hw", [(3, 2, 4, 4, 96, 1, 0), (3, 3, 3, 4, 256, 1, 0), (2, 1, 7, 7, 64, 2, 0),
                                                  (2, 1, 5, 5, 320, 2, 0), (2, 1, 7, 7, 256, 4, 96), (2, 1, 5, 5, 256, 4, 96)])
def test_filter_tap_counts(dev, rank, kd, kh, kw, o, n, hw):
    # the fast gather (per-row padding masks of up to 10 taps per dimension) with filters of 32 to 49
    # taps, bit exact on the integer generators, padding on every side; hw = 96: enough tiles for the
    # 256x256 kernel
    if rank == 2:
        dims = oracle.ConvDims.conv2d(N=n, H=hw or 15, W=hw or 12, C=64, O=o, KH=kh, KW=kw, PT=kh // 2,
                                      PB=kh - 1 - kh // 2, PL=kw // 2, PR=kw // 2)
    else:
        dims = oracle.ConvDims.conv3d(N=1, D=6, H=9, W=10, C=128, O=o, KD=kd, KH=kh, KW=kw, PF=1, PBk=kd - 1,
                                      PT=1, PB=kh - 2, PL=2, PR=kw - 1)
    assert "gather=fast" in mtk.ConvPlan(dev, mtk.conv_desc(dims, has_bias=True, rank=rank)).describe()
    x, w, b = gen.conv3d_activation(dims), gen.conv3d_weights(dims), gen.conv3d_bias(dims)
    y = _run(dev, dims, x, w, b, rank=rank)
    assert _bit_exact(dims, y, x, w, b)


@pytest.mark.parametrize("rank", [2, 3])
def test_random_strides_dilations_padding(dev, rank):
    rng = np.random.default_rng(rank)
    if rank == 2:
        dims = oracle.ConvDims.conv2d(N=3, H=21, W=17, C=64, O=72, KH=3, KW=5, SY=2, SX=1, DY=1, DX=2,
                                      PT=2, PB=0, PL=3, PR=1)
    else:
        dims = oracle.ConvDims.conv3d(N=2, D=7, H=9, W=10, C=128, O=40, SZ=2, SY=1, SX=2, DZ=1, DY=2, DX=1,
                                      PF=1, PBk=2, PT=1, PB=1, PL=0, PR=2)
    x = rng.uniform(-1, 1, dims.x_shape()).astype(np.float16)
    w = rng.uniform(-1, 1, dims.w_shape()).astype(np.float16)
    b = rng.uniform(-1, 1, dims.O).astype(np.float16)
    y = _run(dev, dims, x, w, b)
    exp = oracle.conv(dims, x, w, b)
    absdot = np.abs(oracle.conv(dims, np.abs(x), np.abs(w))).astype(np.float64) + np.abs(b.astype(np.float64))
    Kl = dims.KD * dims.KH * dims.KW * dims.C
    res = oracle.compare(y.astype(np.float64), exp, bound=oracle.dot_bound(exp, absdot * (1 + 1e-6), Kl))
    print(f"   {res}", flush=True)
    assert res["ok"], res


def _bit_exact(dims, y, x, w, b):
    # every output element: the integer generators make the fp32 sums exact, so the device's f16
    # output must be RNE_f16 of the oracle's value
    exp = oracle.conv(dims, x, w, b)
    return np.array_equal(y.view(np.uint16), exp.astype(np.float16).view(np.uint16))


def _random_within_bound(dev, dims, seed):
    # BASELINE's seeded U[-1,1) data and bias: every element within the fp32 dot-product bound
    x = oracle.uniform(seed, dims.x_shape(), -1, 1)
    w = oracle.uniform(seed + 1, dims.w_shape(), -1, 1)
    b = oracle.uniform(seed + 2, (dims.O,), -1, 1)
    y = _run(dev, dims, x, w, b)
    exp = oracle.conv(dims, x, w, b)
    absdot = np.abs(oracle.conv(dims, np.abs(x), np.abs(w))).astype(np.float64) + np.abs(b.astype(np.float64))
    Kl = dims.KD * dims.KH * dims.KW * dims.C
    res = oracle.compare(y.astype(np.float64), exp, bound=oracle.dot_bound(exp, absdot * (1 + 1e-6), Kl))
    print(f"   seeded U[-1,1): {res}", flush=True)
    return res["ok"]


CFG4A = dict(N=8, H=128, W=128, C=256, O=256, PT=1, PB=1, PL=1, PR=1)
CFG4B = dict(N=1, D=16, H=64, W=64, C=128, O=128, PF=1, PBk=1, PT=1, PB=1, PL=1, PR=1)


def test_config4a_conv2d_full_size(dev):
    # conv2d NHWC 8x128x128x256, 3x3x256x256, stride 1, pad 1, + bias, at full
    # size: bit-exact on the reference's integer generators, and within the dot-product bound on
    # BASELINE's seeded U[-1,1) data (seeds 7, 8, 9)
    dims = oracle.ConvDims.conv2d(**CFG4A)
    x, w, b = gen.conv2d_shared_activation(dims), gen.conv2d_shared_weights(dims), gen.conv3d_bias(dims)
    assert _bit_exact(dims, _run(dev, dims, x, w, b), x, w, b)
    assert _random_within_bound(dev, dims, 7)


def test_config4b_conv3d_full_size(dev):
    # conv3d NDHWC 1x16x64x64x128 -> 128, 3x3x3, pad 1 on every axis.
    dims = oracle.ConvDims.conv3d(**CFG4B)
    x, w, b = gen.conv3d_activation(dims), gen.conv3d_weights(dims), gen.conv3d_bias(dims)
    assert _bit_exact(dims, _run(dev, dims, x, w, b), x, w, b)
    assert _bit_exact(dims, _run(dev, dims, x, w, None), x, w, None)
    assert _random_within_bound(dev, dims, 7)
