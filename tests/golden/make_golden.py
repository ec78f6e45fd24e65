"""Writes the committed golden fixtures under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

Outputs
* ``cases.json`` -- the reference's own validation case lists, as data, with the
  file:line each list comes from. These shapes are what the reference's
  executables validate; the parity tests run every one of them.
* ``kat_probe.json`` -- known answers of the reference's offset probe
  (convolution.swift:204-216, 372-392): a 5x5 input of 1..25 with a centre-tap
  or dense 1..9 kernel, "same" zero padding. The expected values are computed
  here by an independent pure-Python loop over a zero-padded copy of the input
  (pad first, then correlate), not by the oracle.
* ``seeded.npz`` -- small seeded inputs (by seed) and the oracle's fp32 outputs (GEMM,
  attention forward, attention backward),
  a regression pin for the oracle and the first thing the GPU tests check.

The seeded fixtures are regenerated bit-identically by the SplitMix64 + RNE
generator in oracle/oracle.c; the test suite checks that too.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

CONV2D_SHARED = {  # ConvolutionShared.swift:2143-2211 (no padding)
    "source": "Sources/ConvolutionShared/ConvolutionShared.swift:2143-2211",
    "generator": "conv2d_shared",
    "cases": [
        dict(N=1, H=5, W=5, C=1, O=1, KH=3, KW=3, SY=1, SX=1, DY=1, DX=1),
        dict(N=1, H=5, W=5, C=4, O=8, KH=3, KW=3, SY=1, SX=1, DY=1, DX=1),
        dict(N=1, H=6, W=7, C=3, O=5, KH=3, KW=3, SY=1, SX=1, DY=1, DX=1),
        dict(N=1, H=7, W=8, C=3, O=4, KH=3, KW=3, SY=2, SX=2, DY=1, DX=1),
        dict(N=1, H=9, W=10, C=2, O=3, KH=3, KW=3, SY=1, SX=1, DY=2, DX=2),
    ],
}
CONV3D = {  # ConvolutionShared.swift:2693-2764 == convolution3d.swift:1235-1306 (no padding)
    "source": "Sources/ConvolutionShared/ConvolutionShared.swift:2693-2764; "
              "Sources/convolution3d/convolution3d.swift:1235-1306",
    "generator": "conv3d",
    "cases": [
        dict(N=1, D=5, H=5, W=5, C=1, O=1, SZ=1, SY=1, SX=1, DZ=1, DY=1, DX=1),
        dict(N=1, D=4, H=5, W=5, C=4, O=8, SZ=1, SY=1, SX=1, DZ=1, DY=1, DX=1),
        dict(N=2, D=7, H=6, W=7, C=3, O=5, SZ=2, SY=1, SX=1, DZ=1, DY=1, DX=1),
        dict(N=1, D=7, H=7, W=7, C=2, O=3, SZ=1, SY=1, SX=1, DZ=2, DY=2, DX=2),
    ],
}
CONV3D_PADDED = {  # ConvolutionShared.swift:2770-2878 (H/W padding 1, the iOS app's live path)
    "source": "Sources/ConvolutionShared/ConvolutionShared.swift:2770-2878",
    "generator": "conv3d",
    "cases": [
        dict(N=1, D=5, H=5, W=5, C=1, O=1, SZ=1, PT=1, PB=1, PL=1, PR=1),
        dict(N=1, D=4, H=5, W=5, C=4, O=8, SZ=1, PT=1, PB=1, PL=1, PR=1),
        dict(N=2, D=7, H=6, W=7, C=3, O=5, SZ=2, PT=1, PB=1, PL=1, PR=1),
        dict(N=1, D=5, H=17, W=19, C=8, O=12, SZ=1, PT=1, PB=1, PL=1, PR=1),
        dict(N=1, D=4, H=33, W=35, C=4, O=8, SZ=1, PT=1, PB=1, PL=1, PR=1),
    ],
}
CONV3D_LR_PADDED = {  # convolution3d_padding.swift:676-742 (left/right padding only)
    "source": "Sources/convolution3d_padding/convolution3d_padding.swift:676-742",
    "generator": "conv3d",
    "cases": [
        dict(N=1, D=5, H=5, W=5, C=1, O=1, SZ=1, PT=0, PB=0, PL=1, PR=1),
        dict(N=1, D=4, H=5, W=5, C=4, O=8, SZ=1, PT=0, PB=0, PL=1, PR=1),
        dict(N=2, D=7, H=6, W=7, C=3, O=5, SZ=2, PT=0, PB=0, PL=1, PR=1),
    ],
}
CONV2D_PADDED = {  # convolution2d_padding.swift:313-388 (same padding 1)
    "source": "Sources/convolution2d_padding/convolution2d_padding.swift:313-388",
    "generator": "padded2d",
    "cases": [
        dict(N=1, H=5, W=5, C=1, O=1, PT=1, PB=1, PL=1, PR=1),
        dict(N=1, H=5, W=5, C=4, O=8, PT=1, PB=1, PL=1, PR=1),
        dict(N=1, H=17, W=19, C=8, O=12, PT=1, PB=1, PL=1, PR=1),
        dict(N=1, H=33, W=35, C=4, O=8, PT=1, PB=1, PL=1, PR=1),
    ],
}


def probe_reference(act, ker):
    """Pure-Python 'same' correlation: zero-pad by 1, then slide the 3x3 window."""
    H, W = len(act), len(act[0])
    padded = [[0.0] * (W + 2) for _ in range(H + 2)]
    for i in range(H):
        for j in range(W):
            padded[i + 1][j + 1] = float(act[i][j])
    out = []
    for i in range(H):
        row = []
        for j in range(W):
            s = 0.0
            for a in range(3):
                for b in range(3):
                    s += padded[i + a][j + b] * float(ker[a][b])
            row.append(s)
        out.append(row)
    return out


def main():
    cases = {"conv2d_shared": CONV2D_SHARED, "conv3d": CONV3D, "conv3d_padded": CONV3D_PADDED,
             "conv3d_lr_padded": CONV3D_LR_PADDED, "conv2d_padded": CONV2D_PADDED}
    with open(os.path.join(HERE, "cases.json"), "w") as f:
        json.dump(cases, f, indent=1)

    act = [[float(5 * i + j + 1) for j in range(5)] for i in range(5)]
    centre = [[0, 0, 0], [0, 1, 0], [0, 0, 0]]
    dense = [[1, 2, 3], [4, 5, 6], [7, 8, 9]]
    kat = {
        "source": "Sources/convolution/convolution.swift:204-216 (data), 372-392 (referenceForOffset, offset 0)",
        "activation": act,
        "centre_tap": {"kernel": centre, "expected": probe_reference(act, centre)},
        "dense": {"kernel": dense, "expected": probe_reference(act, dense)},
    }
    with open(os.path.join(HERE, "kat_probe.json"), "w") as f:
        json.dump(kat, f, indent=1)

    fx = {}
    # GEMM, config-1 style (NN, U[-1,1), seed 0) at a small ragged size, and NT with bias and a K tail.
    A = oracle.uniform(0, (48, 70), -1, 1)
    B = oracle.uniform(1, (70, 40), -1, 1)
    fx["gemm_nn_A"], fx["gemm_nn_B"] = A, B
    fx["gemm_nn_C"] = oracle.gemm(A, B, None, trans_b=False)
    A = oracle.normal(2, (33, 100), 0, 0.1)
    B = oracle.normal(3, (65, 100), 0, 0.1)
    bias = oracle.uniform(4, (65,), -0.5, 0.5)
    fx["gemm_nt_A"], fx["gemm_nt_B"], fx["gemm_nt_bias"] = A, B, bias
    fx["gemm_nt_C"] = oracle.gemm(A, B, bias, trans_b=True)
    Ab = oracle.normal(5, (16, 96), 0, 1, dtype="bf16")
    Bb = oracle.normal(6, (80, 96), 0, 0.02, dtype="bf16")
    biasb = oracle.normal(7, (80,), 0, 0.02, dtype="bf16")
    fx["gemm_bf16_A"], fx["gemm_bf16_B"], fx["gemm_bf16_bias"] = Ab, Bb, biasb
    fx["gemm_bf16_C"] = oracle.gemm(Ab, Bb, biasb, trans_b=True, dtype="bf16")
    # attention [B][S][H][D], S not a multiple of any block, causal and not.
    Q = oracle.normal(10, (1, 37, 2, 128))
    K = oracle.normal(11, (1, 37, 2, 128))
    V = oracle.normal(12, (1, 37, 2, 128))
    fx["attn_Q"], fx["attn_K"], fx["attn_V"] = Q, K, V
    fx["attn_O"] = oracle.attention(Q, K, V)
    fx["attn_O_causal"] = oracle.attention(Q, K, V, causal=True)
    # attention backward (gradients of sum(dO * O)), one head, ragged S, causal and not
    Q = oracle.normal(13, (1, 21, 1, 128))
    K = oracle.normal(14, (1, 21, 1, 128))
    V = oracle.normal(15, (1, 21, 1, 128))
    G = oracle.normal(16, (1, 21, 1, 128))
    fx["bwd_Q"], fx["bwd_K"], fx["bwd_V"], fx["bwd_dO"] = Q, K, V, G
    for tag, causal in (("", False), ("_causal", True)):
        dQ, dK, dV, Dt = oracle.attention_bwd(Q, K, V, G, causal=causal)
        fx["bwd_dQ" + tag], fx["bwd_dK" + tag], fx["bwd_dV" + tag], fx["bwd_D" + tag] = dQ, dK, dV, Dt
    np.savez_compressed(os.path.join(HERE, "seeded.npz"), **fx)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
