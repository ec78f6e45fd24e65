"""Second-backend agreement, the counterpart of the reference's MPSGraph check
(Sources/ConvolutionShared/ConvolutionShared.swift:2403-2462: both backends validated against the CPU
expected, then compared with each other by compareOutputs, 5381-5406). The second backend here is
PyTorch on the same GPU (hipBLASLt for the GEMM, MIOpen for the convolutions, float32 matrix
products for attention); it is a sanity cross-check, never the oracle: the CPU oracle stays the
reference for parity, and torch's own result must also pass it.
"""
import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle
from oracle import generators as gen

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("torch sees no GPU")
    return torch.device("cuda:0")


def _agree(name, ours, theirs, expected, abs_tol):
    """validateOutput for both against the CPU expected, compareOutputs between them. Both backends
    round their outputs to fp16, so the per-element tolerance is the reference's absolute one plus one
    fp16 ulp of the expected value (two correct fp16 results can differ by one ulp)."""
    ours = np.asarray(ours, np.float64)
    theirs = np.asarray(theirs, np.float64)
    exp = np.asarray(expected, np.float64)
    tol = abs_tol + oracle.ulp(exp, "f16")
    bad_ours, bad_theirs = (np.abs(ours - exp) > tol).sum(), (np.abs(theirs - exp) > tol).sum()
    diff = np.abs(ours - theirs)
    print(f"   {name}: ours max|err| {np.abs(ours - exp).max():.3e} ({bad_ours} over), torch max|err| "
          f"{np.abs(theirs - exp).max():.3e} ({bad_theirs} over), ours vs torch max|diff| {diff.max():.3e}, "
          f"mismatches {(diff > tol).sum()}", flush=True)
    assert bad_ours == 0 and bad_theirs == 0, name
    assert (diff > tol).sum() == 0, name


@pytest.mark.parametrize("M,N,K,split_k", [(256, 256, 256, 1), (1000, 700, 4100, 4), (4096, 4096, 4100, 4)])
def test_gemm_agrees_with_hipblaslt(dev, M, N, K, split_k):
    cuda = _cuda()
    A = oracle.normal(110, (M, K), 0, 1 / np.sqrt(K))
    B = oracle.normal(111, (N, K), 0, 1 / np.sqrt(K))
    bias = oracle.uniform(112, (N,), -0.5, 0.5)
    ours = mtk.gemm(dev, A, B, bias, trans_b=True, split_k=split_k).astype(np.float32)
    ta, tb, tbias = (torch.from_numpy(x).to(cuda) for x in (A, B, bias))
    theirs = (torch.matmul(ta, tb.t().contiguous()) + tbias).float().cpu().numpy()
    rows = np.arange(M) if M <= 1024 else np.r_[0:64, M - 64:M]
    exp = oracle.gemm(A[rows], B, bias, trans_b=True)
    _agree(f"gemm {M}x{N}x{K}", ours[rows], theirs[rows], exp, 5e-3)  # matmul.swift:505


@pytest.mark.parametrize("rank", [2, 3])
def test_conv_agrees_with_miopen(dev, rank):
    cuda = _cuda()
    if rank == 2:
        d = oracle.ConvDims.conv2d(N=2, H=33, W=35, C=64, O=96, PT=1, PB=1, PL=1, PR=1)
    else:
        d = oracle.ConvDims.conv3d(N=1, D=6, H=17, W=19, C=64, O=64, PF=1, PBk=1, PT=1, PB=1, PL=1, PR=1)
    x = gen.conv3d_activation(d)
    w = gen.conv3d_weights(d)
    ours = mtk.conv(dev, d, x, w).reshape(d.y_shape()).astype(np.float32)
    tx = torch.from_numpy(np.ascontiguousarray(x.reshape(d.x_shape()))).to(cuda)
    tw = torch.from_numpy(np.ascontiguousarray(w.reshape(d.w_shape()))).to(cuda)
    if rank == 2:  # NHWC x HWIO -> NCHW x OIHW
        y = torch.nn.functional.conv2d(tx[:, 0].permute(0, 3, 1, 2).contiguous(),
                                       tw[0].permute(3, 2, 0, 1).contiguous(), padding=1)
        theirs = y.permute(0, 2, 3, 1).contiguous().float().cpu().numpy()[:, None]
    else:  # NDHWC x DHWIO -> NCDHW x OIDHW
        y = torch.nn.functional.conv3d(tx.permute(0, 4, 1, 2, 3).contiguous(),
                                       tw.permute(4, 3, 0, 1, 2).contiguous(), padding=1)
        theirs = y.permute(0, 2, 3, 4, 1).contiguous().float().cpu().numpy()
    exp = oracle.conv(d, x, w)
    _agree(f"conv{rank}d", ours.reshape(exp.shape), theirs.reshape(exp.shape), exp, 2e-2)  # :5185, 5221


@pytest.mark.parametrize("causal", [False, True])
def test_attention_fwd_bwd_agree_with_torch(dev, causal):
    cuda = _cuda()
    B, S, H, D = 1, 300, 2, 128
    Q, K, V, G = (oracle.normal(120 + i, (B, S, H, D)) for i in range(4))
    O, lse = mtk.attention(dev, Q, K, V, causal=causal, return_lse=True)
    dQ, dK, dV = mtk.attention_bwd(dev, Q, K, V, O, G, lse, causal=causal)
    # torch in float32 with explicit contiguous products (no half-precision batched products)
    t = lambda a: torch.from_numpy(a.astype(np.float32)).to(cuda).permute(0, 2, 1, 3).contiguous().requires_grad_(True)
    q, k, v = t(Q), t(K), t(V)
    g = torch.from_numpy(G.astype(np.float32)).to(cuda).permute(0, 2, 1, 3).contiguous()
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / np.sqrt(D)
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool, device=cuda), 1), float("-inf"))
    o = torch.matmul(torch.softmax(s, -1), v)
    (o * g).sum().backward()
    back = lambda x: x.permute(0, 2, 1, 3).detach().cpu().numpy()
    exp = oracle.attention(Q, K, V, causal=causal)
    _agree("attention O", O.astype(np.float32), back(o), exp, 5e-3)  # attention.swift:536
    eQ, eK, eV, _ = oracle.attention_bwd(Q, K, V, G, causal=causal)
    for name, ours, theirs, e in (("dQ", dQ, q.grad, eQ), ("dK", dK, k.grad, eK), ("dV", dV, v.grad, eV)):
        scale = max(1.0, float(np.abs(e).max()))
        _agree(f"attention {name}", ours.astype(np.float32) / scale, back(theirs) / scale, e / scale, 5e-3)
