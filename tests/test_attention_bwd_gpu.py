"""Flash-attention backward on the GPU (C ABI: mtk_attn_bwd_plan / mtk_attn_bwd_run) against the CPU
oracle of the reference's gradients (Network.swift:205-281, 313-402), and the forward's row
log-sum-exp output (its input).

Tolerance. The kernels accumulate in fp32 but, like the forward's P.V, feed P and dS to the matrix
cores rounded to the input format (unit roundoff u = 2^-11 for f16, 2^-8 for bf16), and compute
D = rowsum(dO * O) from the stored (rounded) O. Per element:
  dV_j = sum_i P_ij dO_i           |err| <= ulp_out + 2u * sum_i P_ij |dO_i|
  dK_j = sum_i dS_ij Q_i           |err| <= ulp_out + 2u * sum_i (|dS_ij| + s P_ij dD_i) |Q_i|
  dQ_i = sum_j dS_ij K_j           |err| <= ulp_out + 2u * sum_j (|dS_ij| + s P_ij dD_i) |K_j|
with dD_i = sum_d |O_id dO_id| (the D error is at most u dD_i) and s = 1/sqrt(D); the magnitudes
are computed in float64 from the same inputs. Relative Frobenius error: <= 2e-3 (f16), 2e-2 (bf16).
"""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle

pytestmark = pytest.mark.gpu


def _f64(x, dtype):
    return oracle.to_f32(x, dtype).astype(np.float64)


def _bhsd(x, dtype):
    """[B][S][H][D] -> float64 [B][H][S][D] (batched BLAS products below)."""
    return np.ascontiguousarray(_f64(x, dtype).transpose(0, 2, 1, 3))


def _magnitudes(Q, K, V, G, causal, dtype):
    """float64 P, |dS| and the per-row D magnitude for the tolerance bound, [B][H][Sq][Skv]."""
    q, k, v, g = (_bhsd(x, dtype) for x in (Q, K, V, G))
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    s = (q @ k.transpose(0, 1, 3, 2)) / np.sqrt(D)
    vis = np.ones((Sq, Skv), bool)
    if causal:
        vis = np.arange(Skv)[None, :] <= (np.arange(Sq)[:, None] + (Skv - Sq))
    s = np.where(vis[None, None], s, -np.inf)
    m = np.max(s, -1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.where(vis[None, None], np.exp(s - m), 0.0)
    del s
    den = p.sum(-1, keepdims=True)
    p = np.where(den > 0, p / np.where(den > 0, den, 1), 0.0)
    o = p @ v
    dd = np.sum(o * g, -1, keepdims=True)
    ds = np.abs(p * ((g @ v.transpose(0, 1, 3, 2)) - dd) / np.sqrt(D))
    dmag = np.sum(np.abs(o * g), -1, keepdims=True)  # [B][H][Sq][1]
    return p, ds, dmag


def _check(name, got, exp, bound_terms, dtype):
    got = oracle.to_f32(got, dtype).astype(np.float64)
    exp = exp.astype(np.float64)
    u = 2.0 ** -11 if dtype == "f16" else 2.0 ** -8
    bound = oracle.ulp(exp, dtype) + 2 * u * bound_terms + 1e-30
    err = np.abs(got - exp)
    rel = oracle.rel_frobenius(got, exp)
    worst = float(np.max(err / bound))
    print(f"   {name}: rel_frob={rel:.2e} worst err/bound={worst:.3f}", flush=True)
    assert np.all(np.isfinite(got)), name
    assert rel <= (2e-3 if dtype == "f16" else 2e-2), (name, rel)
    assert worst <= 1.0, (name, worst)


def _run_and_check(dev, B, H, Sq, Skv, causal, dtype, seed=90, pairs=None, Hkv=None, D=128):
    """GPU forward (for O and lse) and backward once, then the oracle check: on every (b, h) pair,
    or, with `pairs` (a list of [p0, p1) ranges of flattened b * H + h), on those pairs chunk by
    chunk (the float64 bound terms cost S_q * S_kv memory per pair)."""
    Hkv = Hkv or H
    group = H // Hkv
    print(f"[attn bwd] B={B} H={H} H_kv={Hkv} S_q={Sq} S_kv={Skv} causal={causal} {dtype} pairs={pairs}", flush=True)
    Q = oracle.normal(seed, (B, Sq, H, D), dtype=dtype)
    K = oracle.normal(seed + 1, (B, Skv, Hkv, D), dtype=dtype)
    V = oracle.normal(seed + 2, (B, Skv, Hkv, D), dtype=dtype)
    G = oracle.normal(seed + 3, (B, Sq, H, D), dtype=dtype)
    O, lse = mtk.attention(dev, Q, K, V, causal=causal, dtype=dtype, return_lse=True)
    dQ, dK, dV = mtk.attention_bwd(dev, Q, K, V, O, G, lse, causal=causal, dtype=dtype)
    if group > 1:
        # dQ is what full multi-head attention on K/V repeated over each group gives, bit for bit
        Ke, Ve = np.repeat(K, group, 2), np.repeat(V, group, 2)
        Oe, lse_e = mtk.attention(dev, Q, Ke, Ve, causal=causal, dtype=dtype, return_lse=True)
        assert np.array_equal(Oe.view(np.uint16), O.view(np.uint16)) and np.array_equal(lse_e, lse)
        fQ, _, _ = mtk.attention_bwd(dev, Q, Ke, Ve, Oe, G, lse_e, causal=causal, dtype=dtype)
        assert np.array_equal(fQ.view(np.uint16), dQ.view(np.uint16))
    assert all(np.all(np.isfinite(oracle.to_f32(x, dtype))) for x in (dQ, dK, dV))
    for rng in (pairs or [None]):
        eQ, eK, eV, _ = oracle.attention_bwd(Q, K, V, G, causal=causal, dtype=dtype, pairs=rng)
        _check_pairs(Q, K, V, G, dQ, dK, dV, eQ, eK, eV, causal, dtype, group, rng, H)


def _check_pairs(Q, K, V, G, dQ, dK, dV, eQ, eK, eV, causal, dtype, group, rng, H):
    D = Q.shape[3]
    if group > 1:
        K, V = np.repeat(K, group, 2), np.repeat(V, group, 2)  # magnitudes per query head
    if rng is not None:  # compare the computed (b, h) pairs only; Q/K/V magnitudes restricted to them
        assert group == 1
        bh = [(p // H, p % H) for p in range(*rng)]
        sub = lambda x: np.stack([x[b, :, h] for b, h in bh])[:, :, None]  # [n][S][1][D]
        Q, K, V, G = sub(Q), sub(K), sub(V), sub(G)
        dQ, dK, dV, eQ, eK, eV = (sub(x) for x in (dQ, dK, dV, eQ, eK, eV))
    p, ads, dmag = _magnitudes(Q, K, V, G, causal, dtype)
    s = 1.0 / np.sqrt(D)
    q, k, g = (np.abs(_bhsd(x, dtype)) for x in (Q, K, G))
    w = ads + s * p * dmag  # [B][H][Sq][Skv]
    del ads
    back = lambda t: t.transpose(0, 2, 1, 3)  # [B][H][S][D] -> [B][S][H][D]
    per_group = lambda t: t.reshape(t.shape[0], t.shape[1], -1, group, D).sum(3)  # sum a group's query heads
    _check("dV", dV, eV, per_group(back(p.transpose(0, 1, 3, 2) @ g)), dtype)
    _check("dK", dK, eK, per_group(back(w.transpose(0, 1, 3, 2) @ q)), dtype)
    _check("dQ", dQ, eQ, back(w @ k), dtype)


@pytest.mark.parametrize("B,H,Sq,Skv,causal,dtype", [
    (1, 2, 77, 77, False, "f16"),
    (1, 2, 77, 77, True, "f16"),
    (2, 1, 130, 200, False, "f16"),   # S_kv > S_q, ragged tiles
    (2, 1, 200, 130, True, "f16"),    # causal with S_q > S_kv: the first queries see no key
    (1, 3, 256, 256, True, "bf16"),
    (1, 1, 1, 1, False, "f16"),
    (1, 2, 300, 64, False, "bf16"),
])
def test_attention_bwd_matches_oracle(dev, B, H, Sq, Skv, causal, dtype):
    _run_and_check(dev, B, H, Sq, Skv, causal, dtype)


@pytest.mark.parametrize("B,H,Hkv,Sq,Skv,causal,dtype", [
    (1, 4, 1, 200, 200, False, "f16"),
    (2, 8, 2, 130, 300, True, "f16"),
    (1, 6, 3, 257, 129, True, "bf16"),
])
def test_attention_bwd_grouped_kv_heads(dev, B, H, Hkv, Sq, Skv, causal, dtype):
    # grouped K/V heads (the reference's Hk, attention.swift:20, 120): dK, dV of a K/V head sum over
    # the query heads that read it
    _run_and_check(dev, B, H, Sq, Skv, causal, dtype, seed=70, Hkv=Hkv)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_bwd_config5_full_size(dev, causal):
    # BASELINE config 5 shape (B=2, H=32, S=4096, D=128); every output must be finite, and sixteen
    # (b, h) pairs in two chunks (b=0 h=0..3 and 28..31, b=1 h=0..3 and 28..31) are checked element
    # by element against the oracle (which costs ~S^2 D per pair).
    _run_and_check(dev, 2, 32, 4096, 4096, causal, "f16", seed=10, pairs=[(0, 4), (28, 36), (60, 64)])


@pytest.mark.parametrize("q_rows", [128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_lse_output(dev, causal, q_rows):
    # lse_i = log sum_j exp(s_ij / sqrt(D)); writing it leaves O unchanged bit for bit
    B, H, Sq, Skv, D = 2, 2, 333, 290, 128
    Q = oracle.normal(95, (B, Sq, H, D))
    K = oracle.normal(96, (B, Skv, H, D))
    V = oracle.normal(97, (B, Skv, H, D))
    O0 = mtk.attention(dev, Q, K, V, causal=causal, q_rows=q_rows)
    O1, lse = mtk.attention(dev, Q, K, V, causal=causal, q_rows=q_rows, return_lse=True)
    assert np.array_equal(O0.view(np.uint16), O1.view(np.uint16))
    s = np.einsum("bihd,bjhd->bhij", Q.astype(np.float64), K.astype(np.float64)) / np.sqrt(D)
    if causal:
        vis = np.arange(Skv)[None, :] <= (np.arange(Sq)[:, None] + (Skv - Sq))
        s = np.where(vis[None, None], s, -np.inf)
    m = s.max(-1)
    with np.errstate(invalid="ignore", divide="ignore"):
        ref = m + np.log(np.exp(s - m[..., None]).sum(-1))
    finite = np.isfinite(ref)
    assert np.array_equal(finite, np.isfinite(lse)) and np.all(np.isneginf(lse[~finite]))
    assert np.allclose(lse[finite], ref[finite], rtol=0, atol=2e-5 * (1 + np.abs(ref[finite])).max())


def test_attention_bwd_constant_v_rows(dev):
    # constant V rows: dP_ij = D_i for every key, so dS = 0 and dQ = dK = 0 up to rounding
    B, H, S, D = 1, 2, 150, 128
    Q = oracle.normal(101, (B, S, H, D))
    K = oracle.normal(102, (B, S, H, D))
    row = oracle.normal(103, (1, 1, H, D))
    V = np.broadcast_to(row, (B, S, H, D)).copy()
    G = oracle.normal(104, (B, S, H, D))
    O, lse = mtk.attention(dev, Q, K, V, return_lse=True)
    dQ, dK, dV = mtk.attention_bwd(dev, Q, K, V, O, G, lse)
    assert np.abs(dQ.astype(np.float64)).max() < 0.05 and np.abs(dK.astype(np.float64)).max() < 0.05
    _, _, eV, _ = oracle.attention_bwd(Q, K, V, G)
    assert oracle.rel_frobenius(dV.astype(np.float64), eV) < 2e-3


def test_attention_bwd_errors(dev):
    for D in (60, 264):  # head dimensions: multiples of 8 up to 256
        with pytest.raises(mtk.MtkError) as e:
            mtk.AttentionBwdPlan(dev, 1, 1, 64, 64, D=D)
        assert e.value.status == mtk.MTK_ERR_UNSUPPORTED
    plan = mtk.AttentionBwdPlan(dev, 1, 1, 64, 64)
    assert plan.workspace_bytes >= 64 * 4
    buf = dev.empty(64 * 128 * 2)
    with pytest.raises(mtk.MtkError) as e:  # no workspace
        plan.run(buf, buf, buf, buf, buf, buf, buf, buf, buf, None)
    assert "workspace" in e.value.message
    with pytest.raises(mtk.MtkError):  # missing lse
        plan.run(buf, buf, buf, buf, buf, None, buf, buf, buf, buf)
