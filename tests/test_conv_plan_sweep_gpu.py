"""Convolution parity over a seeded sweep of shapes that crosses every plan the library can choose.

Each case draws the rank, batch, spatial extents, channels, output channels, filter size, strides,
dilations and per-side padding from a fixed seed and runs through the C ABI on the reference's
integer-pattern generators (ConvolutionShared.swift:4874-4992), on which every fp32 partial sum is
exact: the device output must equal RNE_f16 of the oracle (ConvolutionShared.swift:4994-5096) bit
for bit. The CPU test checks that the case list reaches the fast gather on both tile sizes and the
generic gather at each load width."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle
from oracle import generators as gen

from test_conv_gpu import _bit_exact, _run


def _out(n, k, s, d, p0, p1):
    return (n + p0 + p1 - d * (k - 1) - 1) // s + 1


def _cases():
    rng = np.random.default_rng(4994)
    out = []
    while len(out) < 30:
        rank = 2 if rng.integers(0, 3) else 3
        C = int(rng.choice([3, 8, 12, 24, 64, 64, 128, 192]))
        O = int(rng.choice([5, 16, 40, 64, 96, 130, 256, 300]))
        N = int(rng.integers(1, 4))
        k = [int(rng.integers(1, 6)) for _ in range(3)]
        s = [int(rng.integers(1, 4)) for _ in range(3)]
        d = [int(rng.integers(1, 3)) for _ in range(3)]
        ext = [int(rng.integers(4, 14)), int(rng.integers(6, 40)), int(rng.integers(6, 40))]
        pad = [[int(rng.integers(0, 4)) for _ in range(2)] for _ in range(3)]
        if rank == 2:
            k[0], s[0], d[0], ext[0], pad[0] = 1, 1, 1, 1, [0, 0]
        if any(_out(ext[i], k[i], s[i], d[i], *pad[i]) < 1 for i in range(3)):
            continue
        if rank == 2:
            dims = oracle.ConvDims.conv2d(N=N, H=ext[1], W=ext[2], C=C, O=O, KH=k[1], KW=k[2], SY=s[1], SX=s[2],
                                          DY=d[1], DX=d[2], PT=pad[1][0], PB=pad[1][1], PL=pad[2][0], PR=pad[2][1])
        else:
            dims = oracle.ConvDims.conv3d(N=N, D=ext[0], H=ext[1], W=ext[2], C=C, O=O, KD=k[0], KH=k[1], KW=k[2],
                                          SZ=s[0], SY=s[1], SX=s[2], DZ=d[0], DY=d[1], DX=d[2], PF=pad[0][0],
                                          PBk=pad[0][1], PT=pad[1][0], PB=pad[1][1], PL=pad[2][0], PR=pad[2][1])
        out.append((rank, dims))
    # enough output rows for the 256x256 fast kernel
    out.append((2, oracle.ConvDims.conv2d(N=4, H=96, W=96, C=128, O=256, KH=3, KW=3, SY=1, SX=1, DY=2, DX=1,
                                          PT=2, PB=1, PL=1, PR=0)))
    return out


CASES = _cases()


def _plan_key(desc):
    kern = desc.split("kernels:")[-1].split()[-1]
    return kern.replace("mtk_conv_f16_", "")


def test_sweep_reaches_every_plan():
    # CPU: the planner alone (no device)
    seen = {_plan_key(mtk.ConvPlan(None, mtk.conv_desc(dims, has_bias=True, rank=rank)).describe())
            for rank, dims in CASES}
    for want in ("fast_256x256_d", "fast_128x128_d", "gen_128x128_v8", "gen_128x128_v4", "gen_128x128_v1"):
        assert want in seen, (want, sorted(seen))


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_conv_plan_sweep(dev, case):
    rank, dims = CASES[case]
    x, w, b = gen.conv3d_activation(dims), gen.conv3d_weights(dims), gen.conv3d_bias(dims)
    print(f"[conv sweep {case}] {mtk.ConvPlan(dev, mtk.conv_desc(dims, has_bias=True, rank=rank)).describe()}",
          flush=True)
    y = _run(dev, dims, x, w, b, rank=rank)
    assert _bit_exact(dims, y, x, w, b)
