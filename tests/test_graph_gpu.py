"""HIP-graph submission of repeated plan runs (mtk_graph_*): the counterpart of the reference's
duplicatedCount dispatches in one command buffer (matmul.swift:447-449, 470-472).

Every replay is checked bit for bit against an eager run of the same plan, with eager work and
synchronisations between replays; a graph that rotates two argument sets fills both outputs."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle
from oracle import generators as gen

pytestmark = pytest.mark.gpu


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint16)


def _replays_match(dev, plan, args_eager, out_buf, shape, eager_other):
    """Eager run -> reference bits; then a 2-step graph replayed 3 times, each replay preceded by
    unrelated eager work (`eager_other`) and followed by a sync and a bitwise check."""
    dev.upload_into(out_buf, np.zeros(shape, np.uint16))
    plan.launch(args_eager)
    dev.sync()
    ref = dev.download(out_buf, shape, np.uint16).copy()
    g = plan.graph([args_eager], steps=2)
    try:
        for rep in range(3):
            dev.upload_into(out_buf, np.full(shape, 0x7E00, np.uint16))  # poison the output
            eager_other()
            dev.sync()
            g.launch()
            dev.sync()
            got = dev.download(out_buf, shape, np.uint16)
            print(f"   replay {rep}: identical={np.array_equal(got, ref)}", flush=True)
            assert np.array_equal(got, ref), f"graph replay {rep} differs from the eager run"
    finally:
        g.close()
    return ref


def test_gemm_split_k_graph_replays(dev):
    M, N, K = 512, 384, 1000
    A = oracle.normal(70, (M, K), 0, 1 / np.sqrt(K))
    B = oracle.normal(71, (N, K), 0, 1 / np.sqrt(K))
    bias = oracle.uniform(72, (N,), -0.5, 0.5)
    print(f"[graph] gemm M={M} N={N} K={K} split_k=4", flush=True)
    plan = mtk.GemmPlan(dev, M, N, K, has_bias=True, split_k=4)
    dA, dB, db = dev.upload(A), dev.upload(B), dev.upload(bias)
    dC, dC2 = dev.empty(M * N * 2), dev.empty(M * N * 2)
    ws = dev.empty(plan.workspace_bytes)
    other = mtk.GemmPlan(dev, 128, 128, 256)
    oA = dev.upload(oracle.normal(73, (128, 256)))
    oC = dev.empty(128 * 128 * 2)
    ref = _replays_match(dev, plan, plan.args(dA, dB, db, dC, ws), dC, (M, N),
                         lambda: other.run(oA, oA, None, oC))
    exp = oracle.gemm(A, B, bias)
    assert oracle.compare(ref.view(np.float16).astype(np.float64), exp)["ok"]
    # two argument sets in one graph: run i uses set i % 2 (different outputs, shared workspace)
    dev.upload_into(dC, np.zeros((M, N), np.uint16))
    dev.upload_into(dC2, np.zeros((M, N), np.uint16))
    g = plan.graph([plan.args(dA, dB, db, dC, ws), plan.args(dA, dB, db, dC2, ws)], steps=4)
    g.launch()
    dev.sync()
    g.close()
    assert np.array_equal(dev.download(dC, (M, N), np.uint16), ref)
    assert np.array_equal(dev.download(dC2, (M, N), np.uint16), ref)
    for x in (dA, dB, db, dC, dC2, ws, oA, oC):
        x.free()


def test_attention_graph_replays(dev):
    shp = (1, 200, 4, 128)
    Q, K, V = (oracle.normal(74 + i, shp) for i in range(3))
    print(f"[graph] attention {shp} causal", flush=True)
    plan = mtk.AttentionPlan(dev, 1, 4, 200, 200, 128, causal=True)
    dQ, dK, dV = dev.upload(Q), dev.upload(K), dev.upload(V)
    dO = dev.empty(Q.nbytes)
    other = mtk.AttentionPlan(dev, 1, 4, 200, 200, 128, causal=False)
    dO2 = dev.empty(Q.nbytes)
    ref = _replays_match(dev, plan, plan.args(dQ, dK, dV, dO), dO, shp, lambda: other.run(dQ, dK, dV, dO2))
    exp = oracle.attention(Q, K, V, causal=True)
    assert oracle.compare(ref.view(np.float16).astype(np.float64), exp)["ok"]
    for x in (dQ, dK, dV, dO, dO2):
        x.free()


def test_conv_graph_replays(dev):
    d = oracle.ConvDims.conv2d(N=2, H=20, W=18, C=64, O=64, PT=1, PB=1, PL=1, PR=1)
    x, w = gen.conv3d_activation(d), gen.conv3d_weights(d)
    print("[graph] conv2d 2x20x18x64 -> 64, 3x3, pad 1", flush=True)
    desc = mtk.conv_desc(d)
    plan = mtk.ConvPlan(dev, desc)
    dx, dw = dev.upload(x), dev.upload(w)
    shape = plan.out_shape()
    dy = dev.empty(int(np.prod(shape)) * 2)
    ref = _replays_match(dev, plan, plan.args(dx, dw, None, dy), dy, shape, lambda: dev.sync())
    exp = oracle.conv(d, x, w).astype(np.float16)
    assert np.array_equal(ref.reshape(d.y_shape()), exp.view(np.uint16))
    for b in (dx, dw, dy):
        b.free()


def test_graph_errors(dev):
    with pytest.raises(mtk.MtkError) as e:
        mtk.GemmPlan(None, 64, 64, 64).graph([mtk.GemmArgs()], steps=1)  # dry plan
    assert e.value.status == mtk.MTK_ERR_INVALID
    plan = mtk.GemmPlan(dev, 64, 64, 64)
    with pytest.raises(mtk.MtkError):
        plan.graph([plan.args(0, 0, None, 0)], steps=1)  # null operands are refused at creation
    dA = dev.empty(64 * 64 * 2)
    with pytest.raises(mtk.MtkError):
        plan.graph([plan.args(dA, dA, None, dA)], steps=0)
    dA.free()
