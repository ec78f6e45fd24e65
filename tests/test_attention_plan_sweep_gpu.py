"""Flash-attention forward parity over a seeded sweep of shapes that crosses every kernel family.

Each case draws batch, K/V heads, query heads per K/V head, query and key lengths (independently:
the causal diagonal is offset by S_kv - S_q), head dimension (multiples of 8 up to 512 and other
values up to 256), mask and dtype from a fixed seed, runs through the C ABI and is checked on the
whole output against the CPU oracle (Network.swift:134-179, 286-311) with the acceptance of
test_attention_gpu.check. The CPU test checks that the case list reaches the 128-query kernels laid
out for 64, 128 and 256, the wide (512) kernel and the element-staged kernels."""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle

from test_attention_gpu import check

DS = [8, 16, 24, 40, 64, 72, 96, 128, 136, 200, 256, 264, 320, 512, 1, 5, 36, 100, 130, 250]


def _cases():
    rng = np.random.default_rng(13417)
    out = []
    while len(out) < 40:
        B = int(rng.integers(1, 3))
        hkv = int(rng.choice([1, 2, 3]))
        group = int(rng.choice([1, 2, 4]))
        Sq = int(rng.choice([1, 17, 64, 100, 129, 256, 300, 513]))
        Skv = Sq if rng.integers(0, 2) else int(rng.choice([1, 33, 128, 200, 257, 640]))
        D = int(rng.choice(DS))
        causal = bool(rng.integers(0, 2))
        dtype = "bf16" if rng.integers(0, 3) == 0 else "f16"
        if B * hkv * group * Sq * Skv * D > 2.5e9:
            continue
        out.append((B, hkv * group, hkv, Sq, Skv, D, causal, dtype))
    return out


CASES = _cases()


def _kernel(case):
    B, H, Hkv, Sq, Skv, D, causal, dtype = case
    d = mtk.AttentionPlan(None, B=B, H=H, H_kv=Hkv, S_q=Sq, S_kv=Skv, D=D, causal=causal, dtype=dtype).describe()
    return d.split("kernels:")[-1].split()[-1]


def test_sweep_reaches_every_kernel_family():
    # CPU: the planner alone (no device)
    seen = {_kernel(c).replace("_causal", "").replace("_bf16", "").replace("_f16", "") for c in CASES}
    for want in ("mtk_attn_fwd", "mtk_attn_fwd_d64", "mtk_attn_fwd_d256", "mtk_attn_fwd_d512", "mtk_attn_fwd_g64",
                 "mtk_attn_fwd_g128", "mtk_attn_fwd_g256"):
        assert want in seen, (want, sorted(seen))


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_attention_plan_sweep(dev, case):
    B, H, Hkv, Sq, Skv, D, causal, dtype = CASES[case]
    Q = oracle.normal(700 + case, (B, Sq, H, D), 0, 1, dtype)
    K = oracle.normal(800 + case, (B, Skv, Hkv, D), 0, 1, dtype)
    V = oracle.normal(900 + case, (B, Skv, Hkv, D), 0, 1, dtype)
    check(dev, Q, K, V, causal, dtype, label=f"sweep {case}: {_kernel(CASES[case])} H_kv={Hkv}")
