"""Flash-attention forward parity on the GPU, through the C ABI, against the CPU oracle
(Network.swift:134-179, 286-311), on [B][S][H][D] tensors with D = 128.

Acceptance: relative Frobenius error <= 1e-3 (f16 output) and, element-wise,
|y - yhat| <= ulp_out(|yhat|) + 2^-10 * sum_j P_ij |V_jd|: P enters the P.V product rounded to
the 16-bit input type (<= 2^-11 relative each for f16), plus fp32 softmax/accumulation error far
below that. bf16 uses 2^-7 (P rounded to bf16, 2^-8 relative) and the bf16 output-rounding floor."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle

pytestmark = pytest.mark.gpu


def probs_f64(Q, K, causal, dtype="f16"):
    q = oracle.to_f32(Q, dtype).astype(np.float64)
    k = oracle.to_f32(K, dtype).astype(np.float64)
    Sq, Skv, D = q.shape[1], k.shape[1], q.shape[3]
    s = np.einsum("bihd,bjhd->bhij", q, k) / np.sqrt(D)
    if causal:
        mask = np.arange(Skv)[None, :] > (np.arange(Sq)[:, None] + (Skv - Sq))
        s = np.where(mask[None, None], -np.inf, s)
    mx = s.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    p = np.exp(s - mx)
    den = p.sum(-1, keepdims=True)
    return np.where(den > 0, p / np.where(den > 0, den, 1), 0.0)


def check(dev, Q, K, V, causal, dtype="f16", label="", q_rows=0):
    print(f"[attn] {label} Q{Q.shape} Skv={K.shape[1]} causal={causal} {dtype} q_rows={q_rows}", flush=True)
    got = mtk.attention(dev, Q, K, V, causal=causal, dtype=dtype, q_rows=q_rows)
    exp = oracle.attention(Q, K, V, causal=causal, dtype=dtype)
    group = Q.shape[2] // K.shape[2]  # grouped K/V heads: bound terms per query head
    K, V = np.repeat(K, group, 2), np.repeat(V, group, 2)
    p = probs_f64(Q, K, causal, dtype)
    absv = np.abs(oracle.to_f32(V, dtype).astype(np.float64))
    abspv = np.einsum("bhij,bjhd->bihd", p, absv)
    if dtype == "f16":
        bound, rel_tol = oracle.ulp(exp) + 2.0 ** -10 * abspv, 1e-3
    else:
        bound = oracle.ulp(exp, "bf16") + 2.0 ** -7 * abspv
        rel_tol = 4e-3 + oracle.rel_frobenius(oracle.to_f32(oracle.from_f32(exp, "bf16"), "bf16"), exp)
    res = oracle.compare(oracle.to_f32(got, dtype), exp, bound=bound, rel_tol=rel_tol)
    ref = mtk.validate(got, exp, abs_tol=5e-3, dtype=dtype)  # the reference's own check (attention.swift:536)
    print(f"   rel_fro={res['rel_fro']:.3e} max_abs={res['max_abs']:.3e} worst/bound={res['worst_ratio']:.3f} "
          f"ref5e-3_mismatches={ref['mismatches']}", flush=True)
    assert res["ok"], res
    return got, exp


def qkv(seed, B, S, H, Skv=None, dtype="f16"):
    Skv = Skv or S
    return (oracle.normal(seed, (B, S, H, 128), 0, 1, dtype), oracle.normal(seed + 1, (B, Skv, H, 128), 0, 1, dtype),
            oracle.normal(seed + 2, (B, Skv, H, 128), 0, 1, dtype))


def test_fixtures(dev, golden_dir):
    fx = np.load(f"{golden_dir}/seeded.npz")
    for causal, key in ((False, "attn_O"), (True, "attn_O_causal")):
        got = mtk.attention(dev, fx["attn_Q"], fx["attn_K"], fx["attn_V"], causal=causal)
        assert oracle.compare(got.astype(np.float32), fx[key])["ok"]


# query rows per workgroup: 128 (32 per wavefront) and 256 (64 per wavefront) kernels
ROWS = [128, 256]


@pytest.mark.parametrize("S", [1, 7, 31, 64, 65, 127, 128, 129, 255, 257, 511, 1000, 1023])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_rows", ROWS)
def test_sequence_sweep(dev, S, causal, q_rows):
    # mirrors profileCorrectness (attention.swift:391-396): S = 1..1023, D = 128, H = 8
    Q, K, V = qkv(1000 + S, 1, S, 8)
    check(dev, Q, K, V, causal, label=f"S{S}", q_rows=q_rows)


@pytest.mark.parametrize("sq,skv", [(100, 300), (300, 100), (64, 1), (700, 260)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_rows", ROWS)
def test_unequal_lengths(dev, sq, skv, causal, q_rows):
    Q, K, V = qkv(77, 2, sq, 3, Skv=skv)
    check(dev, Q, K, V, causal, label=f"{sq}x{skv}", q_rows=q_rows)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_rows", ROWS)
def test_bf16(dev, causal, q_rows):
    Q, K, V = qkv(5, 2, 333, 4, dtype="bf16")
    check(dev, Q, K, V, causal, dtype="bf16", label="bf16", q_rows=q_rows)


@pytest.mark.parametrize("q_rows", ROWS)
def test_closed_forms(dev, q_rows):
    B, S, H = 1, 300, 2
    Q, K, _ = qkv(9, B, S, H)
    row = oracle.normal(12, (1, 1, H, 128))
    Vc = np.broadcast_to(row, (B, S, H, 128)).copy()
    O = mtk.attention(dev, Q, K, Vc, q_rows=q_rows)  # constant V rows -> O = that row
    assert np.allclose(O.astype(np.float32), np.broadcast_to(row.astype(np.float32), O.shape), atol=2e-3, rtol=1e-3)
    V = oracle.normal(13, (B, S, H, 128))
    O = mtk.attention(dev, np.zeros_like(Q), K, V, causal=True, q_rows=q_rows)  # Q = 0 -> prefix means
    pref = np.cumsum(V.astype(np.float64), 1) / np.arange(1, S + 1)[None, :, None, None]
    assert np.allclose(O.astype(np.float64), pref, atol=3e-3)
    O = mtk.attention(dev, Q, K, V, causal=True, q_rows=q_rows)  # first query sees only key 0
    assert np.array_equal(O[:, 0], V[:, 0])
    O = mtk.attention(dev, Q, K, V, causal=True, q_rows=q_rows)  # query 256 (second block of 256)
    assert np.array_equal(O, mtk.attention(dev, Q, K, V, causal=True, q_rows=384 - q_rows))  # both kernels: same bits


@pytest.mark.parametrize("H,Hkv", [(8, 2), (6, 1), (4, 4)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_rows", ROWS)
def test_grouped_kv_heads(dev, H, Hkv, causal, q_rows):
    # the reference's Hq / Hk dimensions (attention.swift:20, 120): query head h reads K/V head
    # h // (H // Hkv); same bits as multi-head attention on K/V repeated over each group
    B, Sq, Skv = 2, 300, 270
    Q = oracle.normal(60, (B, Sq, H, 128))
    K, V = oracle.normal(61, (B, Skv, Hkv, 128)), oracle.normal(62, (B, Skv, Hkv, 128))
    got, _ = check(dev, Q, K, V, causal, label=f"H{H}/Hkv{Hkv}", q_rows=q_rows)
    full = mtk.attention(dev, Q, np.repeat(K, H // Hkv, 2), np.repeat(V, H // Hkv, 2), causal=causal, q_rows=q_rows)
    assert np.array_equal(got.view(np.uint16), full.view(np.uint16))


def _probs_rows_f64(Q, K, r0, r1, causal):
    """float64 softmax probabilities of query rows r0..r1-1, [B][H][rows][S_kv] (BLAS products)."""
    q = Q[:, r0:r1].astype(np.float64).transpose(0, 2, 1, 3)  # [B][H][rows][D]
    k = K.astype(np.float64).transpose(0, 2, 3, 1)            # [B][H][D][S_kv]
    s = (q @ k) / np.sqrt(Q.shape[3])
    if causal:  # rows r0.. see keys j <= i (S_q == S_kv)
        s = np.where(np.arange(K.shape[1])[None, :] > np.arange(r0, r1)[:, None], -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    return p / p.sum(-1, keepdims=True)


@pytest.mark.parametrize("causal", [False, True])
def test_config5_full_size(dev, causal):
    # B=2, H=32, S=4096, D=128, Q,K,V ~ N(0,1), scale 1/sqrt(D). Every query row
    # of every (b, h) against the oracle, element by element; the float64 bound terms are computed
    # in blocks of 256 query rows.
    B, S, H = 2, 4096, 32
    Q, K, V = qkv(10, B, S, H)
    absv = np.abs(V.astype(np.float64)).transpose(0, 2, 1, 3)  # [B][H][S][D]
    got = mtk.attention(dev, Q, K, V, causal=causal)
    exp = oracle.attention(Q, K, V, causal=causal)
    worst, rel_num, rel_den = 0.0, 0.0, 0.0
    for r0 in range(0, S, 256):
        r1 = r0 + 256
        e = exp[:, r0:r1].astype(np.float64)
        abspv = (_probs_rows_f64(Q, K, r0, r1, causal) @ absv).transpose(0, 2, 1, 3)
        res = oracle.compare(got[:, r0:r1].astype(np.float64), e, bound=oracle.ulp(e) + 2.0 ** -10 * abspv)
        assert res["ok"], (causal, r0, res)
        worst = max(worst, res["worst_ratio"])
        rel_num += float(np.sum((got[:, r0:r1].astype(np.float64) - e) ** 2))
        rel_den += float(np.sum(e ** 2))
    rel = np.sqrt(rel_num / rel_den)
    print(f"[attn] config5 causal={causal}: all {S} rows of all {B * H} (b, h) within bound, worst err/bound "
          f"{worst:.3f}, rel_fro {rel:.2e}", flush=True)
    assert rel <= 1e-3
