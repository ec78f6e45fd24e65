"""Flash-attention backward parity over a seeded sweep of shapes that crosses every kernel set.

Each case draws batch, K/V heads, query heads per K/V head, query and key lengths (independently),
head dimension (multiples of 8 up to 256), mask and dtype from a fixed seed, runs the forward and
the backward through the C ABI and checks dQ, dK and dV on every (b, h) pair against the CPU oracle
of the reference's gradients (Network.swift:205-281, 313-402) with the acceptance of
test_attention_bwd_gpu (grouped heads: dQ also bit for bit against K/V repeated over each group).
The CPU test checks that the case list reaches the kernel sets laid out for 64, 128 and 256."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk

from test_attention_bwd_gpu import _run_and_check


def _cases():
    rng = np.random.default_rng(20513)
    out = []
    while len(out) < 20:
        B = int(rng.integers(1, 3))
        hkv = int(rng.choice([1, 2]))
        group = int(rng.choice([1, 2, 4]))
        Sq = int(rng.choice([1, 33, 64, 100, 200, 257]))
        Skv = Sq if rng.integers(0, 2) else int(rng.choice([17, 128, 190, 300]))
        D = int(rng.choice([8, 16, 40, 64, 72, 96, 128, 136, 200, 256]))
        causal = bool(rng.integers(0, 2))
        dtype = "bf16" if rng.integers(0, 3) == 0 else "f16"
        if B * hkv * group * Sq * Skv * D > 4e8:
            continue
        out.append((B, hkv * group, hkv, Sq, Skv, D, causal, dtype))
    return out


CASES = _cases()


def _kernels(case):
    B, H, Hkv, Sq, Skv, D, causal, dtype = case
    d = mtk.AttentionBwdPlan(None, B=B, H=H, H_kv=Hkv, S_q=Sq, S_kv=Skv, D=D, causal=causal, dtype=dtype).describe()
    return d.split("kernels:")[-1].split()


def test_sweep_reaches_every_kernel_set():
    # CPU: the planner alone (no device)
    seen = {k.replace("_causal", "").replace("_bf16", "").replace("_f16", "") for c in CASES for k in _kernels(c)}
    for want in ("mtk_attn_bwd_dkdv_d64", "mtk_attn_bwd_dkdv", "mtk_attn_bwd256_dkdv", "mtk_attn_bwd_dq_d64",
                 "mtk_attn_bwd_dq", "mtk_attn_bwd256_dq"):
        assert want in seen, (want, sorted(seen))


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_attention_bwd_plan_sweep(dev, case):
    B, H, Hkv, Sq, Skv, D, causal, dtype = CASES[case]
    print(f"[bwd sweep {case}] {' '.join(_kernels(CASES[case]))}", flush=True)
    _run_and_check(dev, B, H, Sq, Skv, causal, dtype, seed=1000 + 10 * case, Hkv=Hkv, D=D)
