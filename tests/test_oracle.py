"""Pins the CPU oracle (oracle/oracle.c) before any device result is compared to it.

Each oracle function is checked against something other than its own formula:
library routines (numpy float16 casts, torch bfloat16 casts, numpy float64
matmul / einsum, scipy correlate), closed forms (all-ones, identity, zero,
constant rows, Q = 0, one-hot logits), exactness on the reference's integer
generators, the reference's known-answer probe, and the committed fixtures.
The inputs are chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails at least one check.
"""
import json
import os

import numpy as np
import pytest

import oracle
from oracle import generators as gen

# ---------------------------------------------------------------- conversions


def test_f16_to_f32_all_bit_patterns(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = orc.to_f32(bits, "f16")
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]) == np.isnan(ref[~finite]))


def test_f32_to_f16_rne_matches_numpy(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),  # f16 subnormal range
        (rng.standard_normal(50000) * 7e4).astype(np.float32),  # overflow range
        # exact ties between adjacent f16 values (round-half-even cases)
        ((np.arange(-2048, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26], np.float32),
    ])
    got = orc.from_f32(x, "f16").view(np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_matches_torch(orc):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32),
                        (np.arange(-512, 512, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -7)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.from_f32(x, "bf16")
    assert np.array_equal(got, ref)
    back = orc.to_f32(got, "bf16")
    assert np.array_equal(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_seeded_generators_are_deterministic_and_distributed(orc):
    a = orc.uniform(0, (1 << 16,), -1, 1)
    assert np.array_equal(a.view(np.uint16), orc.uniform(0, (1 << 16,), -1, 1).view(np.uint16))
    assert not np.array_equal(a.view(np.uint16), orc.uniform(1, (1 << 16,), -1, 1).view(np.uint16))
    af = a.astype(np.float64)
    assert af.min() >= -1 and af.max() <= 1 and abs(af.mean()) < 0.02 and abs(af.var() - 1 / 3) < 0.01
    n = orc.normal(5, (1 << 16,), 0.0, 2.0).astype(np.float64)
    assert abs(n.mean()) < 0.05 and abs(n.std() - 2.0) < 0.05
    nb = orc.to_f32(orc.normal(6, (1 << 16,), 0.0, 0.02, dtype="bf16"), "bf16")
    assert abs(nb.std() - 0.02) < 0.001


# ---------------------------------------------------------------- GEMM


def test_gemm_all_ones_k_tail_closed_form(orc):
    # All-ones A, B with K = 4100 and a small-integer bias: C = K + bias exactly in fp32 and in fp16
    # (spacing 4 in [4096, 8192)). The reference's split-K tail bug (K residual added once per split)
    # would give 4112.
    M, N, K = 3, 5, 4100
    A = np.ones((M, K), np.float16)
    B = np.ones((N, K), np.float16)
    bias = np.array([0, 1, -2, 3, 4], np.float16)
    C = orc.gemm(A, B, bias, trans_b=True)
    assert np.array_equal(C, np.broadcast_to((K + bias.astype(np.float32)), (M, N)))


def test_gemm_identity_and_zero(orc):
    M = 24
    B = orc.uniform(3, (M, 17), -1, 1)  # [K][N] with K == M
    bias = orc.uniform(4, (17,), -0.5, 0.5)
    eye = np.eye(M, dtype=np.float16)
    C = orc.gemm(eye, B, bias, trans_b=False)
    assert np.array_equal(C, B.astype(np.float32) + bias.astype(np.float32))
    C = orc.gemm(eye, np.ascontiguousarray(B.T), bias, trans_b=True)  # NT: B stored [N][K]
    assert np.array_equal(C, B.astype(np.float32) + bias.astype(np.float32))
    C = orc.gemm(orc.uniform(5, (7, M), -1, 1), np.zeros((17, M), np.float16), bias, trans_b=True)
    assert np.array_equal(C, np.broadcast_to(bias.astype(np.float32), (7, 17)))


def test_gemm_integer_data_exact(orc):
    rng = np.random.default_rng(7)
    A = rng.integers(-8, 9, size=(31, 300)).astype(np.float16)
    B = rng.integers(-8, 9, size=(300, 45)).astype(np.float16)
    bias = rng.integers(-50, 50, size=45).astype(np.float16)
    ref = A.astype(np.int64) @ B.astype(np.int64) + bias.astype(np.int64)
    assert np.array_equal(orc.gemm(A, B, bias, trans_b=False), ref.astype(np.float32))
    assert np.array_equal(orc.gemm(A, np.ascontiguousarray(B.T), bias, trans_b=True), ref.astype(np.float32))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("trans_b", [True, False])
def test_gemm_random_vs_float64(orc, dtype, trans_b):
    M, N, K = 37, 53, 259
    A = orc.normal(11, (M, K), 0, 1, dtype=dtype)
    B = orc.normal(12, (N, K) if trans_b else (K, N), 0, 1, dtype=dtype)
    bias = orc.normal(13, (N,), 0, 1, dtype=dtype)
    a = orc.to_f32(A, dtype).astype(np.float64)
    b = orc.to_f32(B, dtype).astype(np.float64)
    b = b.T if trans_b else b
    ref = a @ b + orc.to_f32(bias, dtype).astype(np.float64)
    got = orc.gemm(A, B, bias, trans_b=trans_b, dtype=dtype)
    tol = K * 2.0 ** -24 * (np.abs(a) @ np.abs(b)) + 1e-6
    assert np.all(np.abs(got - ref) <= tol)
    # Row subsets compute the same rows.
    part = orc.gemm(A, B, bias, trans_b=trans_b, dtype=dtype, rows=(5, 9))
    assert np.array_equal(part[5:9], got[5:9]) and not part[:5].any()


def test_gemm_fixture_regression(orc, golden_dir):
    fx = np.load(os.path.join(golden_dir, "seeded.npz"))
    A = orc.uniform(0, (48, 70), -1, 1)
    assert np.array_equal(A.view(np.uint16), fx["gemm_nn_A"].view(np.uint16))
    assert np.array_equal(orc.gemm(fx["gemm_nn_A"], fx["gemm_nn_B"], None, trans_b=False), fx["gemm_nn_C"])
    assert np.array_equal(orc.gemm(fx["gemm_nt_A"], fx["gemm_nt_B"], fx["gemm_nt_bias"], trans_b=True),
                          fx["gemm_nt_C"])
    assert np.array_equal(orc.gemm(fx["gemm_bf16_A"], fx["gemm_bf16_B"], fx["gemm_bf16_bias"], trans_b=True,
                                   dtype="bf16"), fx["gemm_bf16_C"])


# ---------------------------------------------------------------- attention


def attention_f64(Q, K, V, causal):
    q = Q.astype(np.float64)
    k = K.astype(np.float64)
    v = V.astype(np.float64)
    B, S, H, D = q.shape
    Skv = k.shape[1]
    s = np.einsum("bihd,bjhd->bhij", q, k) / np.sqrt(D)
    if causal:
        mask = np.arange(Skv)[None, :] > (np.arange(S)[:, None] + (Skv - S))
        s = np.where(mask[None, None], -np.inf, s)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhij,bjhd->bihd", p, v), p


# head dimensions: the reference's run(headDimension:) takes any value (attention.swift:398)
@pytest.mark.parametrize("D", [1, 3, 24, 64, 96, 200, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_random_vs_float64(orc, causal, D):
    Q = orc.normal(20, (2, 45, 3, D))
    K = orc.normal(21, (2, 45, 3, D))
    V = orc.normal(22, (2, 45, 3, D))
    ref, p = attention_f64(Q, K, V, causal)
    got = orc.attention(Q, K, V, causal=causal)
    absv = np.einsum("bhij,bjhd->bihd", p, np.abs(V.astype(np.float64)))
    assert np.all(np.abs(got - ref) <= 2.0 ** -16 * absv + 1e-6)


def test_attention_closed_forms(orc):
    B, S, H, D = 1, 29, 2, 32
    K = orc.normal(30, (B, S, H, D))
    row = orc.normal(31, (1, 1, H, D))
    Vc = np.broadcast_to(row, (B, S, H, D)).copy()
    Q = orc.normal(32, (B, S, H, D))
    # constant V rows: O = that row (sum P = 1 within fp32 rounding)
    O = orc.attention(Q, K, Vc)
    assert np.allclose(O, np.broadcast_to(row.astype(np.float32), O.shape), rtol=0, atol=4e-6 * 3)
    # Q = 0: uniform weights -> O = mean of V rows; causal -> prefix means
    V = orc.normal(33, (B, S, H, D))
    Z = np.zeros_like(Q)
    O = orc.attention(Z, K, V)
    assert np.allclose(O, np.broadcast_to(V.astype(np.float64).mean(1, keepdims=True), O.shape), atol=2e-6)
    O = orc.attention(Z, K, V, causal=True)
    pref = np.cumsum(V.astype(np.float64), 1) / np.arange(1, S + 1)[None, :, None, None]
    assert np.allclose(O, pref, atol=2e-6)
    # S = 1: O = V0; first causal row: O = V0
    O = orc.attention(Q[:, :1], K[:, :1], V[:, :1])
    assert np.array_equal(O, V[:, :1].astype(np.float32))
    assert np.array_equal(orc.attention(Q, K, V, causal=True)[:, 0], V[:, 0].astype(np.float32))
    # one dominant logit: key 7 aligned with a large query -> O ~= V[7]
    Kh = np.zeros((B, S, H, D), np.float16)
    Kh[:, 7] = 1.0
    Qh = np.full((B, S, H, D), 8.0, np.float16)  # logit 8*32/sqrt(32) = 45 vs 0
    O = orc.attention(Qh, Kh, V)
    assert np.allclose(O, np.broadcast_to(V[:, 7:8].astype(np.float32), O.shape), atol=1e-6)


def test_attention_key_permutation_invariance(orc):
    Q = orc.normal(40, (1, 16, 1, 64))
    K = orc.normal(41, (1, 16, 1, 64))
    V = orc.normal(42, (1, 16, 1, 64))
    perm = np.random.default_rng(3).permutation(16)
    a = orc.attention(Q, K, V)
    b = orc.attention(Q, K[:, perm], V[:, perm])
    assert np.allclose(a, b, atol=1e-5)
    # ...but not invariant to permuting only K (catches a K/V index mix-up)
    c = orc.attention(Q, K[:, perm], V)
    assert not np.allclose(a, c, atol=1e-3)


def test_attention_fixture_regression(orc, golden_dir):
    fx = np.load(os.path.join(golden_dir, "seeded.npz"))
    assert np.array_equal(orc.attention(fx["attn_Q"], fx["attn_K"], fx["attn_V"]), fx["attn_O"])
    assert np.array_equal(orc.attention(fx["attn_Q"], fx["attn_K"], fx["attn_V"], causal=True), fx["attn_O_causal"])


# ---------------------------------------------------------------- convolution


def conv_f64_padfirst(dims, x, w, bias=None):
    """Independent restatement: zero-pad the input, then correlate every tap (no bounds checks)."""
    xp = np.pad(x.astype(np.float64), ((0, 0), (dims.PF, dims.PBk), (dims.PT, dims.PB), (dims.PL, dims.PR), (0, 0)))
    wf = w.astype(np.float64)
    y = np.zeros(dims.y_shape())
    OD, OH, OW = dims.OD, dims.OH, dims.OW
    for kd in range(dims.KD):
        for kh in range(dims.KH):
            for kw in range(dims.KW):
                z0, h0, w0 = kd * dims.DZ, kh * dims.DY, kw * dims.DX
                win = xp[:, z0:z0 + (OD - 1) * dims.SZ + 1:dims.SZ, h0:h0 + (OH - 1) * dims.SY + 1:dims.SY,
                         w0:w0 + (OW - 1) * dims.SX + 1:dims.SX, :]
                y += np.einsum("ndhwc,co->ndhwo", win, wf[kd, kh, kw])
    if bias is not None:
        y += bias.astype(np.float64)
    return y


def _case_dims(kind, c):
    if kind in ("conv2d_shared", "conv2d_padded"):
        return oracle.ConvDims.conv2d(**c)
    return oracle.ConvDims.conv3d(**c)


def _case_data(generator, dims):
    if generator == "conv2d_shared":
        return gen.conv2d_shared_activation(dims), gen.conv2d_shared_weights(dims)
    return gen.conv3d_activation(dims), gen.conv3d_weights(dims)



# ---------------------------------------------------------------- attention backward

def _bwd_autograd_f64(Q, K, V, G, causal):
    """float64 gradients of sum(G * O) by torch autograd (CPU): independent of the oracle's loops."""
    import torch

    t = lambda x: torch.tensor(np.asarray(x, np.float64)).permute(0, 2, 1, 3).contiguous().requires_grad_(True)
    q, k, v = t(Q), t(K), t(V)
    g = torch.tensor(np.asarray(G, np.float64)).permute(0, 2, 1, 3)
    D, Sq, Skv = q.shape[-1], q.shape[2], k.shape[2]
    s = q @ k.transpose(-1, -2).contiguous() / np.sqrt(D)
    p_keep = torch.ones(Sq, 1, dtype=torch.float64)
    if causal:
        mask = torch.arange(Skv)[None, :] > (torch.arange(Sq)[:, None] + (Skv - Sq))
        s = s.masked_fill(mask, -1e30)  # exp underflows to exactly 0
        p_keep = (~mask.all(-1, keepdim=True)).to(torch.float64)  # rows with no visible key: O = 0
    o = (torch.softmax(s, -1) * p_keep) @ v
    (o * g).sum().backward()
    back = lambda x: x.grad.permute(0, 2, 1, 3).numpy()
    return back(q), back(k), back(v)


@pytest.mark.parametrize("causal,Sq,Skv", [(False, 33, 33), (True, 33, 33), (False, 17, 40), (True, 40, 17)])
def test_attention_bwd_vs_autograd(orc, causal, Sq, Skv):
    # Network.swift:313-402 restated; checked against float64 autograd of the same loss on the
    # same (f16-rounded) inputs, including S_q != S_kv and the bottom-right causal alignment
    B, H, D = 2, 2, 64
    Q = orc.normal(50, (B, Sq, H, D))
    K = orc.normal(51, (B, Skv, H, D))
    V = orc.normal(52, (B, Skv, H, D))
    G = orc.normal(53, (B, Sq, H, D))
    dQ, dK, dV, _ = orc.attention_bwd(Q, K, V, G, causal=causal)
    for name, got, ref in zip(("dQ", "dK", "dV"), (dQ, dK, dV), _bwd_autograd_f64(Q, K, V, G, causal)):
        err = np.abs(got - ref).max()
        assert err <= 2e-5 * max(1.0, np.abs(ref).max()), (name, err)


def test_attention_bwd_finite_differences(orc):
    # The reference's own recipe (Network.swift:45-59): perturb one entry of Q, K or V by +-0.001,
    # difference the loss Phi = sum dO * O (here in float64), divide by 0.002.
    B, S, H, D = 1, 9, 1, 16
    Q = orc.normal(60, (B, S, H, D))
    K = orc.normal(61, (B, S, H, D))
    V = orc.normal(62, (B, S, H, D))
    G = orc.normal(63, (B, S, H, D))
    for causal in (False, True):
        dQ, dK, dV, _ = orc.attention_bwd(Q, K, V, G, causal=causal)
        base = [x.astype(np.float64) for x in (Q, K, V)]
        rng = np.random.default_rng(7)
        for which, grad in ((0, dQ), (1, dK), (2, dV)):
            for _ in range(6):
                idx = (0, rng.integers(S), 0, rng.integers(D))
                vals = []
                for step in (+1e-3, -1e-3):
                    xs = [x.copy() for x in base]
                    xs[which][idx] += step
                    O, _ = attention_f64(*xs, causal)
                    vals.append(float(np.sum(G.astype(np.float64) * O)))
                fd = (vals[0] - vals[1]) / 2e-3
                assert abs(fd - grad[idx]) <= 1e-4 * max(1.0, abs(fd)), (which, idx, fd, grad[idx])


def test_attention_bwd_closed_forms(orc):
    B, S, H, D = 1, 23, 2, 32
    K = orc.normal(70, (B, S, H, D))
    Q = orc.normal(71, (B, S, H, D))
    G = orc.normal(72, (B, S, H, D))
    # constant V rows: O = v for every query, so dP_ij = dO_i . v = D_i and dS = 0: dQ = dK = 0
    row = orc.normal(73, (1, 1, H, D))
    Vc = np.broadcast_to(row, (B, S, H, D)).copy()
    dQ, dK, dV, Dt = orc.attention_bwd(Q, K, Vc, G)
    scale = np.abs(G.astype(np.float64)).max() * np.abs(row.astype(np.float64)).sum() * np.abs(K.astype(np.float64)).max()
    assert np.abs(dQ).max() <= 1e-5 * scale and np.abs(dK).max() <= 1e-5 * scale
    # Q = 0 (non-causal): uniform P = 1/S, so every dV row is the mean of the dO rows
    V = orc.normal(74, (B, S, H, D))
    dQ, dK, dV, Dt = orc.attention_bwd(np.zeros_like(Q), K, V, G)
    mean = G.astype(np.float64).mean(1, keepdims=True)
    assert np.allclose(dV, np.broadcast_to(mean, dV.shape), atol=2e-6)
    # D-term = sum_d O . dO with O from the forward oracle, summed over d in order in fp32
    O = orc.attention(Q, K, V)
    _, _, _, Dt = orc.attention_bwd(Q, K, V, G)
    acc = np.zeros((B, S, H), np.float32)
    g32 = G.astype(np.float32)
    for d in range(D):
        acc = (acc + O[..., d] * g32[..., d]).astype(np.float32)
    assert np.array_equal(Dt, acc.transpose(0, 2, 1))


def test_attention_bwd_key_permutation_equivariance(orc):
    # permuting keys and values together permutes dK, dV the same way and leaves dQ unchanged
    Q = orc.normal(80, (1, 16, 1, 64))
    K = orc.normal(81, (1, 16, 1, 64))
    V = orc.normal(82, (1, 16, 1, 64))
    G = orc.normal(83, (1, 16, 1, 64))
    perm = np.random.default_rng(5).permutation(16)
    dQ, dK, dV, _ = orc.attention_bwd(Q, K, V, G)
    pQ, pK, pV, _ = orc.attention_bwd(Q, K[:, perm], V[:, perm], G)
    assert np.allclose(dQ, pQ, atol=1e-5) and np.allclose(dK[:, perm], pK, atol=1e-5)
    assert np.allclose(dV[:, perm], pV, atol=1e-5)
    # ...and computing only some (b, h) pairs leaves the others untouched and the computed ones equal
    Q2 = orc.normal(84, (2, 16, 3, 64))
    K2 = orc.normal(85, (2, 16, 3, 64))
    V2 = orc.normal(86, (2, 16, 3, 64))
    G2 = orc.normal(87, (2, 16, 3, 64))
    full = orc.attention_bwd(Q2, K2, V2, G2)
    part = orc.attention_bwd(Q2, K2, V2, G2, pairs=(2, 4))  # (b, h) = (0, 2), (1, 0)
    for f, p in zip(full[:3], part[:3]):
        assert np.array_equal(p[0, :, 2], f[0, :, 2]) and np.array_equal(p[1, :, 0], f[1, :, 0])
        assert not p[0, :, :2].any() and not p[1, :, 1:].any()


def test_attention_grouped_kv_heads_equal_repeated_heads(orc):
    # grouped K/V heads: query head h reads K/V head h // (H // Hkv). Forward and dQ equal multi-head
    # attention on K/V repeated over each group, bit for bit (same values, same loop order); dK and
    # dV equal the group sums of the repeated problem's per-head gradients (up to summation order).
    B, S, H, Hkv, D = 2, 24, 6, 2, 32
    Q, G = orc.normal(140, (B, S, H, D)), orc.normal(143, (B, S, H, D))
    K, V = orc.normal(141, (B, S + 5, Hkv, D)), orc.normal(142, (B, S + 5, Hkv, D))
    Ke, Ve = np.repeat(K, H // Hkv, 2), np.repeat(V, H // Hkv, 2)
    for causal in (False, True):
        assert np.array_equal(orc.attention(Q, K, V, causal=causal), orc.attention(Q, Ke, Ve, causal=causal))
        dQ, dK, dV, Dt = orc.attention_bwd(Q, K, V, G, causal=causal)
        fQ, fK, fV, fD = orc.attention_bwd(Q, Ke, Ve, G, causal=causal)
        assert np.array_equal(dQ, fQ) and np.array_equal(Dt, fD)
        for got, full in ((dK, fK), (dV, fV)):
            summed = full.reshape(B, S + 5, Hkv, H // Hkv, D).sum(3)
            assert np.allclose(got, summed, rtol=1e-5, atol=1e-6)
    # a transposed grouping (h % Hkv) would differ
    Kt, Vt = np.tile(K, (1, 1, H // Hkv, 1)), np.tile(V, (1, 1, H // Hkv, 1))
    assert not np.array_equal(orc.attention(Q, K, V), orc.attention(Q, Kt, Vt))
    # pairs select (b, K/V head) with every query head of the group
    part = orc.attention_bwd(Q, K, V, G, pairs=(1, 2))  # (b, hk) = (0, 1): query heads 3..5
    full = orc.attention_bwd(Q, K, V, G)
    assert np.array_equal(part[0][0, :, 3:], full[0][0, :, 3:]) and not part[0][0, :, :3].any()
    assert np.array_equal(part[1][0, :, 1], full[1][0, :, 1]) and not part[1][1].any()


def test_attention_bwd_fixture_regression(orc, golden_dir):
    fx = np.load(os.path.join(golden_dir, "seeded.npz"))
    for tag, causal in (("", False), ("_causal", True)):
        dQ, dK, dV, Dt = orc.attention_bwd(fx["bwd_Q"], fx["bwd_K"], fx["bwd_V"], fx["bwd_dO"], causal=causal)
        assert np.array_equal(dQ, fx["bwd_dQ" + tag]) and np.array_equal(dK, fx["bwd_dK" + tag])
        assert np.array_equal(dV, fx["bwd_dV" + tag]) and np.array_equal(Dt, fx["bwd_D" + tag])

def test_conv_reference_cases_exact(orc, golden_dir):
    """Every reference case list, on the reference's integer generators: oracle fp32 == float64, bit-exact."""
    cases = json.load(open(os.path.join(golden_dir, "cases.json")))
    n = 0
    for kind, spec in cases.items():
        for c in spec["cases"]:
            dims = _case_dims(kind, c)
            x, w = _case_data(spec["generator"], dims)
            bias = gen.conv3d_bias(dims)
            y = orc.conv(dims, x, w)
            assert np.array_equal(y.astype(np.float64), conv_f64_padfirst(dims, x, w)), (kind, c)
            yb = orc.conv(dims, x, w, bias)
            assert np.array_equal(yb.astype(np.float64), conv_f64_padfirst(dims, x, w, bias)), (kind, c)
            n += 1
    assert n == 21


def test_conv_centre_tap_identity(orc):
    # ConvolutionShared 2-D case 1: 5x5, C=O=1, 1..25 input, centre tap, no padding -> interior copy.
    dims = oracle.ConvDims.conv2d(N=1, H=5, W=5, C=1, O=1)
    x, w = gen.conv2d_shared_activation(dims), gen.conv2d_shared_weights(dims)
    y = orc.conv(dims, x, w)
    assert np.array_equal(y[0, 0, :, :, 0], x[0, 0, 1:4, 1:4, 0].astype(np.float32))


def test_conv_probe_known_answers(orc, golden_dir):
    kat = json.load(open(os.path.join(golden_dir, "kat_probe.json")))
    dims = oracle.ConvDims.conv2d(N=1, H=5, W=5, C=1, O=1, PT=1, PB=1, PL=1, PR=1)
    x = gen.probe_activation().reshape(dims.x_shape())
    assert np.array_equal(x.reshape(5, 5).astype(np.float64), np.array(kat["activation"]))
    for name, w in (("centre_tap", gen.probe_centre_tap()), ("dense", gen.probe_dense())):
        y = orc.conv(dims, x, w.reshape(dims.w_shape()))
        assert np.array_equal(y.reshape(5, 5).astype(np.float64), np.array(kat[name]["expected"])), name
    # hand check of the top-left window: 1*5 + 2*6 + 6*8 + 7*9 = 128
    assert kat["dense"]["expected"][0][0] == 128.0


def test_conv_vs_scipy_correlate(orc):
    signal = pytest.importorskip("scipy.signal")
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 1, 12, 13, 1)).astype(np.float16)
    w = rng.standard_normal((1, 3, 3, 1, 1)).astype(np.float16)
    dims = oracle.ConvDims.conv2d(N=1, H=12, W=13, C=1, O=1, PT=1, PB=1, PL=1, PR=1)
    ref = signal.correlate2d(x[0, 0, :, :, 0].astype(np.float64), w[0, :, :, 0, 0].astype(np.float64), mode="same")
    y = orc.conv(dims, x, w)
    assert np.allclose(y[0, 0, :, :, 0], ref, atol=1e-4)


def test_conv3d_depth_padding_and_strides_random(orc):
    rng = np.random.default_rng(10)
    dims = oracle.ConvDims.conv3d(N=2, D=6, H=7, W=9, C=5, O=6, SZ=2, SY=1, SX=2, DZ=1, DY=2, DX=1,
                                  PF=1, PBk=1, PT=2, PB=1, PL=1, PR=0)
    x = rng.standard_normal(dims.x_shape()).astype(np.float16)
    w = rng.standard_normal(dims.w_shape()).astype(np.float16)
    b = rng.standard_normal(dims.O).astype(np.float16)
    y = orc.conv(dims, x, w, b)
    ref = conv_f64_padfirst(dims, x, w, b)
    assert np.allclose(y, ref, atol=1e-4)
    # A kernel that is not symmetric must not equal its flip (catches a flipped/convolution kernel).
    yf = orc.conv(dims, x, np.ascontiguousarray(w[::-1, ::-1, ::-1]), b)
    assert not np.allclose(yf, ref, atol=1e-2)


# ---------------------------------------------------------------- weight re-layout

@pytest.mark.parametrize("shape", [(1, 1, 1, 1, 1), (5, 3, 1, 3, 3), (8, 4, 3, 3, 3), (3, 7, 2, 5, 4)])
def test_permute_oidhw_to_dhwio_exact(orc, shape):
    # ConvolutionShared.swift:4606-4627 restated; pinned by an independent numpy transpose and by the
    # reference's own check (validateFlatOutput, tolerance 0: exact, 5381-5406)
    w = orc.normal(130, shape)
    got = orc.permute_oidhw_to_dhwio(w)
    ref = np.transpose(w, (2, 3, 4, 1, 0))
    assert got.shape == ref.shape and np.array_equal(got.view(np.uint16), np.ascontiguousarray(ref).view(np.uint16))
    # a permutation: every source element appears exactly once
    assert np.array_equal(np.sort(got.view(np.uint16).ravel()), np.sort(w.view(np.uint16).ravel()))


def test_permute_then_conv_equals_dhwio_conv(orc):
    # the reference's PermuteThenTensorOpSession3D path: OIDHW weights re-laid out, then the DHWIO conv
    d = orc.ConvDims.conv3d(N=1, D=4, H=5, W=6, C=3, O=4, PF=1, PBk=1, PT=1, PB=1, PL=1, PR=1)
    x = gen.conv3d_activation(d)
    w_dhwio = gen.conv3d_weights(d)
    w_oidhw = np.ascontiguousarray(np.transpose(w_dhwio, (4, 3, 0, 1, 2)))
    assert np.array_equal(orc.conv(d, x, orc.permute_oidhw_to_dhwio(w_oidhw)), orc.conv(d, x, w_dhwio))
