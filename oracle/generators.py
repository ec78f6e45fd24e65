"""The reference's deterministic conv data generators (test infrastructure only).

Every value is a small integer times a power of two, so it is exact in fp16, and
every partial sum of products is a multiple of 2^-9; while |sum| < 2^15 an fp32
accumulator holds each partial sum exactly, in any order. That makes conv
outputs on these inputs bit-exact targets (oracle == float64 == device fp32).

Sources (reference repo):
  conv2d (ConvolutionShared)  activation ((i*7+3)%19-9)*0.0625   ConvolutionShared.swift:4874-4883
                              weights    ((j*5+1)%17-8)*0.03125  ConvolutionShared.swift:4885-4908
                              C=O=1 3x3 special case: 1..count input, centre-tap kernel (4876-4894)
  conv3d / padded conv3d      activation ((i*7+3)%29-14)*0.0625  ConvolutionShared.swift:4949-4955,
                                                                 convolution3d.swift:279-285,
                                                                 convolution3d_padding.swift:186-192
                              weights    ((j*5+1)%23-11)*0.03125 ConvolutionShared.swift:4957-4985
                              bias       ((o*11+5)%19-9)*0.0625  ConvolutionShared.swift:4987-4992
  padded conv2d               activation %29-14, weights %23-11  convolution2d_padding.swift:65-77
  offset probe                5x5 input 1..25, centre-tap / dense 1..9 kernels
                                                                 convolution.swift:204-216
j is the canonical HWIO / DHWIO flat index of the weight.
"""
from __future__ import annotations

import numpy as np


def _pattern(count: int, mul: int, add: int, mod: int, sub: int, scale: float) -> np.ndarray:
    i = np.arange(count, dtype=np.int64)
    return (((i * mul + add) % mod - sub).astype(np.float64) * scale).astype(np.float16)


def conv2d_shared_activation(dims) -> np.ndarray:
    count = dims.N * dims.H * dims.W * dims.C
    if dims.C == 1 and dims.O == 1 and dims.KH == 3 and dims.KW == 3:
        return (np.arange(count, dtype=np.float64) + 1).astype(np.float16).reshape(dims.x_shape())
    return _pattern(count, 7, 3, 19, 9, 0.0625).reshape(dims.x_shape())


def conv2d_shared_weights(dims) -> np.ndarray:
    count = dims.KH * dims.KW * dims.C * dims.O
    if dims.C == 1 and dims.O == 1 and dims.KH == 3 and dims.KW == 3:
        w = np.zeros(count, np.float16)
        w[1 * 3 + 1] = 1.0  # centre tap, HWIO index of (kh=1, kw=1, ic=0, oc=0)
        return w.reshape(dims.w_shape())
    return _pattern(count, 5, 1, 17, 8, 0.03125).reshape(dims.w_shape())


def conv3d_activation(dims) -> np.ndarray:
    return _pattern(dims.N * dims.D * dims.H * dims.W * dims.C, 7, 3, 29, 14, 0.0625).reshape(dims.x_shape())


def conv3d_weights(dims) -> np.ndarray:
    return _pattern(dims.KD * dims.KH * dims.KW * dims.C * dims.O, 5, 1, 23, 11, 0.03125).reshape(dims.w_shape())


def conv3d_bias(dims) -> np.ndarray:
    return _pattern(dims.O, 11, 5, 19, 9, 0.0625)


# convolution2d_padding.swift uses the 3-D formulas on a single image.
padded2d_activation = conv3d_activation
padded2d_weights = conv3d_weights


def probe_activation() -> np.ndarray:
    return (np.arange(25, dtype=np.float64) + 1).astype(np.float16).reshape(5, 5)


def probe_centre_tap() -> np.ndarray:
    w = np.zeros(9, np.float16)
    w[3 + 1] = 1.0
    return w.reshape(3, 3)


def probe_dense() -> np.ndarray:
    return (np.arange(9, dtype=np.float64) + 1).astype(np.float16).reshape(3, 3)
