"""Flash-attention backward for head dimensions other than 128 (the reference's gradients take any
headDimension: Sources/attention/Network.swift:64-107, 205-402), on the GPU through the C ABI,
against the CPU oracle with the tolerance of tests/test_attention_bwd_gpu.py.

D <= 64 (multiples of 8) runs the 32-row wavefront kernels laid out for 64, 64 < D <= 128 the
same kernels laid out for 128, with the chunks past D loaded as zeros; 128 < D <= 256 runs the
16-row wavefront kernels laid out for 256. All three are checked on ragged sequence lengths, both
masks, bf16, grouped K/V heads and the config 5 shape."""
import pytest

import example_matmul_metal4_amd as mtk
from test_attention_bwd_gpu import _run_and_check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D", [8, 16, 32, 56, 64, 72, 96, 120, 136, 160, 192, 248, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_sweep(dev, D, causal):
    _run_and_check(dev, 1, 2, 130, 97, causal, "f16", seed=300 + D, D=D)


@pytest.mark.parametrize("D", [40, 64, 256])
@pytest.mark.parametrize("B,H,Hkv,Sq,Skv,causal,dtype", [
    (1, 2, 2, 77, 77, True, "bf16"),
    (2, 4, 2, 200, 260, False, "f16"),   # grouped K/V heads, S_kv > S_q
    (1, 3, 1, 260, 129, True, "f16"),    # causal with S_q > S_kv: the first queries see no key
    (1, 1, 1, 1, 1, False, "f16"),
])
def test_head_dim_shapes(dev, D, B, H, Hkv, Sq, Skv, causal, dtype):
    _run_and_check(dev, B, H, Sq, Skv, causal, dtype, seed=400 + D, Hkv=Hkv, D=D)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_config5_shape(dev, D, causal):
    # the config 5 shape (B=2, H=32, S=4096) at D = 64 and 256: every output finite, eight (b, h)
    # pairs (b=0 h=0..3, b=1 h=28..31) element by element against the oracle
    _run_and_check(dev, 2, 32, 4096, 4096, causal, "f16", seed=10, pairs=[(0, 4), (60, 64)], D=D)


def test_head_dim_plan(dev):
    for D, kernels in ((64, ("mtk_attn_bwd_dkdv_d64_f16", "mtk_attn_bwd_dq_d64_f16")),
                       (72, ("mtk_attn_bwd_dkdv_f16", "mtk_attn_bwd_dq_f16")),
                       (256, ("mtk_attn_bwd256_dkdv_f16", "mtk_attn_bwd256_dq_f16"))):
        desc = mtk.AttentionBwdPlan(dev, 1, 2, 100, 100, D=D).describe()
        assert all(k in desc for k in kernels), desc
