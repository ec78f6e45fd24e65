"""Flash-attention forward parity for head dimensions other than 128, on the GPU through the C ABI,
against the CPU oracle (Network.swift:134-179, 286-311, which takes any head dimension).

The reference's generator and run(headDimension:) accept any head dimension K
(Sources/attention/attention.swift:25 kBlocks, 84-91 masked remainder store, 192-199 remainder
block of the Q.K^T walk, 398). The kernels here are compiled for padded head dimensions 64, 128,
256 and 512 (the last: multiples of 8 above 256, 16 queries per wavefront); head dimensions up to
256 that are not a multiple of 8 run the element-staged kernels.

Acceptance as in test_attention_gpu.py: relative Frobenius <= 1e-3 (f16 out) and element-wise
|y - yhat| <= ulp_out(|yhat|) + 2^-10 * sum_j P_ij |V_jd| (bf16: 2^-7 and its rounding floor)."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle
from test_attention_gpu import _probs_rows_f64, check

pytestmark = pytest.mark.gpu

# multiples of 8 (direct-to-LDS kernels padded to 64 / 128 / 256 / 512) and others (element-staged)
FAST_D = [8, 40, 64, 72, 96, 120, 136, 200, 256, 264, 384, 504, 512]
GEN_D = [1, 3, 17, 63, 65, 100, 129, 255]


def qkv_d(seed, B, S, H, D, Skv=None, Hkv=None, dtype="f16"):
    Skv, Hkv = Skv or S, Hkv or H
    return (oracle.normal(seed, (B, S, H, D), 0, 1, dtype), oracle.normal(seed + 1, (B, Skv, Hkv, D), 0, 1, dtype),
            oracle.normal(seed + 2, (B, Skv, Hkv, D), 0, 1, dtype))


@pytest.mark.parametrize("D", FAST_D + GEN_D)
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_sweep(dev, D, causal):
    Q, K, V = qkv_d(300 + D, 2, 300, 3, D, Skv=270)
    check(dev, Q, K, V, causal, label=f"D{D}")


@pytest.mark.parametrize("S", [1, 63, 64, 65, 129, 1000])
@pytest.mark.parametrize("D", [64, 96, 256, 100, 320])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_sequence_sweep(dev, S, D, causal):
    # profileCorrectness's S sweep (attention.swift:391-396) at other head dimensions
    Q, K, V = qkv_d(2000 + S, 1, S, 4, D)
    check(dev, Q, K, V, causal, label=f"D{D} S{S}")


@pytest.mark.parametrize("D", [64, 256, 33, 512])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_bf16(dev, D, causal):
    Q, K, V = qkv_d(40, 2, 333, 2, D, dtype="bf16")
    check(dev, Q, K, V, causal, dtype="bf16", label=f"bf16 D{D}")


@pytest.mark.parametrize("D", [64, 256, 100, 448])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_grouped_kv(dev, D, causal):
    # grouped K/V heads: same bits as K/V repeated over each group
    Q, K, V = qkv_d(70, 2, 200, 8, D, Skv=230, Hkv=2)
    got, _ = check(dev, Q, K, V, causal, label=f"D{D} H8/Hkv2")
    full = mtk.attention(dev, Q, np.repeat(K, 4, 2), np.repeat(V, 4, 2), causal=causal)
    assert np.array_equal(got.view(np.uint16), full.view(np.uint16))


@pytest.mark.parametrize("S,Skv", [(1, 1), (255, 256), (300, 270), (513, 700), (1000, 1000)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_d64_ping_pong(dev, S, Skv, causal, dtype):
    # the 256-query ping-pong kernel at D = 64 (the plan's choice for non-causal grids that fill the
    # device): against the oracle, and bit for bit against the 128-query kernel, whose arithmetic
    # it shares
    Q, K, V = qkv_d(500 + S, 2, S, 3, 64, Skv=Skv, dtype=dtype)
    got, _ = check(dev, Q, K, V, causal, dtype=dtype, label=f"D64 q_rows=256 {S}x{Skv}", q_rows=256)
    ref = mtk.attention(dev, Q, K, V, causal=causal, dtype=dtype, q_rows=128)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("causal", [False, True])
def test_d64_ping_pong_grouped_kv(dev, causal):
    Q, K, V = qkv_d(71, 2, 400, 8, 64, Skv=330, Hkv=2)
    got, _ = check(dev, Q, K, V, causal, label="D64 q_rows=256 H8/Hkv2", q_rows=256)
    full = mtk.attention(dev, Q, np.repeat(K, 4, 2), np.repeat(V, 4, 2), causal=causal, q_rows=128)
    assert np.array_equal(got.view(np.uint16), full.view(np.uint16))


@pytest.mark.parametrize("D", [64, 96, 256, 37, 512])
def test_head_dim_closed_forms(dev, D):
    B, S, H = 1, 200, 2
    Q, K, _ = qkv_d(90, B, S, H, D)
    row = oracle.normal(91, (1, 1, H, D))
    Vc = np.broadcast_to(row, (B, S, H, D)).copy()
    O = mtk.attention(dev, Q, K, Vc)  # constant V rows -> O = that row
    assert np.allclose(O.astype(np.float32), np.broadcast_to(row.astype(np.float32), O.shape), atol=2e-3, rtol=1e-3)
    V = oracle.normal(92, (B, S, H, D))
    O = mtk.attention(dev, Q, K, V, causal=True)  # the first query sees only key 0
    assert np.array_equal(O[:, 0], V[:, 0])


def test_head_dim_lse(dev):
    # the forward's row log-sum-exp at D = 64, 100 and 384 against float64
    for D in (64, 100, 384):
        Q, K, V = qkv_d(95, 1, 150, 2, D)
        _, lse = mtk.attention(dev, Q, K, V, causal=True, return_lse=True)
        s = np.einsum("bihd,bjhd->bhij", Q.astype(np.float64), K.astype(np.float64)) / np.sqrt(D)
        s = np.where(np.arange(150)[None, :] > np.arange(150)[:, None], -np.inf, s)
        mx = s.max(-1, keepdims=True)
        ref = (mx + np.log(np.exp(s - mx).sum(-1, keepdims=True)))[..., 0]
        assert np.allclose(lse, ref, atol=1e-4, rtol=1e-5), D


def test_odd_head_dim_unaligned_pointers(dev):
    # element-staged plans (D % 8 != 0) take 2-byte aligned tensors: offset every pointer by one
    # element inside larger buffers and compare with the aligned run
    B, S, H, D = 1, 130, 2, 23
    Q, K, V = qkv_d(97, B, S, H, D)
    ref = mtk.attention(dev, Q, K, V)
    plan = mtk.AttentionPlan(dev, B, H, S, S, D)
    bufs = [dev.empty(x.nbytes + 16) for x in (Q, K, V, Q)]
    for b, x in zip(bufs[:3], (Q, K, V)):
        host = np.zeros(x.size + 8, np.uint16)
        host[1:1 + x.size] = x.view(np.uint16).ravel()
        dev.upload_into(b, host)
    plan.run(*(b.ptr + 2 for b in bufs))
    dev.sync()
    out = dev.download(bufs[3], (Q.size + 8,), np.uint16)[1:1 + Q.size].view(np.float16).reshape(Q.shape)
    for b in bufs:
        b.free()
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


def test_head_dim_limits(dev):
    for D in (257, 300 + 1, 520, 0):  # above 256 only multiples of 8, up to 512
        with pytest.raises(mtk.MtkError) as e:
            mtk.AttentionPlan(dev, 1, 1, 16, 16, D)
        assert e.value.status == mtk.MTK_ERR_UNSUPPORTED
    with pytest.raises(mtk.MtkError):  # the ping-pong kernel is for D = 128 and 64 only
        mtk.AttentionPlan(dev, 1, 1, 16, 16, 96, q_rows=256)
    with pytest.raises(mtk.MtkError):  # D above 256: 64 query rows per workgroup, chosen by the plan
        mtk.AttentionPlan(dev, 1, 1, 16, 16, 264, q_rows=128)
    assert "rows/wg=64 " in mtk.AttentionPlan(dev, 1, 2, 100, 100, 512).describe()
    with pytest.raises(mtk.MtkError):  # the backward: multiples of 8 up to 256
        mtk.AttentionBwdPlan(dev, 1, 1, 16, 16, 264)
    plan = mtk.AttentionPlan(dev, 1, 1, 16, 16, 24)  # D % 8 == 0: 16-byte alignment required
    buf = dev.empty(4096)
    with pytest.raises(mtk.MtkError):
        plan.run(buf.ptr + 2, buf.ptr, buf.ptr, buf.ptr)
    buf.free()


@pytest.mark.parametrize("D", [64, 96, 256, 512])
def test_config5_shape_head_dims(dev, D):
    # config 5's shape (B=2, H=32, S=4096) at other head dimensions, both masks: 256 query rows of
    # every (b, h) per mask (4 blocks of 64 spread over the sequence, first and last included)
    # against the oracle, element by element
    B, S, H = 2, 4096, 32
    Q, K, V = qkv_d(10, B, S, H, D)
    absv = np.abs(V.astype(np.float64)).transpose(0, 2, 1, 3)
    for causal in (False, True):
        print(f"[attn] config5 shape D={D} causal={causal}", flush=True)
        got = mtk.attention(dev, Q, K, V, causal=causal)
        worst = 0.0
        for r0 in np.linspace(0, S - 64, 4).astype(int):
            r0 = int(r0)
            r1 = r0 + 64
            exp = oracle.attention(Q, K, V, causal=causal, rows=(r0, r1))[:, r0:r1]
            abspv = (_probs_rows_f64(Q, K, r0, r1, causal) @ absv).transpose(0, 2, 1, 3)
            res = oracle.compare(got[:, r0:r1].astype(np.float64), exp, bound=oracle.ulp(exp) + 2.0 ** -10 * abspv)
            assert res["ok"], (D, causal, r0, res)
            worst = max(worst, res["worst_ratio"])
        print(f"   256 rows per (b, h) within bound, worst err/bound {worst:.3f}", flush=True)
