"""CPU oracle for the tensor-op path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package, and only as the checker (or, for the baseline, as the
thing timed on the host CPU). The product path (``example_matmul_metal4_amd``
and ``libmtk.so``) never imports it.

This module is a ctypes wrapper over ``liboracle.so`` (oracle.c, a plain-C
restatement of the reference's CPU validation loops; see oracle.h for the
file:line each function follows), plus:

* the reference's deterministic integer-pattern data generators
  (``generators.py``), and
* the acceptance metrics (relative Frobenius error and the per-element
  fp32-dot bound), ``compare()``.

f16 tensors are numpy ``float16``; bf16 tensors are numpy ``uint16`` bit
patterns (numpy has no bfloat16).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, fields

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F16 = 0
BF16 = 1
DTYPES = {"f16": F16, "bf16": BF16}

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)
    return LIB_PATH


class ConvDims(ctypes.Structure):
    """Mirror of ``oracle_conv_dims`` (NDHWC / DHWIO / NDHWC)."""

    _fields_ = [(n, ctypes.c_int) for n in (
        "N", "D", "H", "W", "C", "O", "KD", "KH", "KW", "SZ", "SY", "SX", "DZ", "DY", "DX",
        "PF", "PBk", "PT", "PB", "PL", "PR")]

    @classmethod
    def conv2d(cls, N, H, W, C, O, KH=3, KW=3, SY=1, SX=1, DY=1, DX=1, PT=0, PB=0, PL=0, PR=0):
        return cls(N=N, D=1, H=H, W=W, C=C, O=O, KD=1, KH=KH, KW=KW, SZ=1, SY=SY, SX=SX, DZ=1, DY=DY,
                   DX=DX, PF=0, PBk=0, PT=PT, PB=PB, PL=PL, PR=PR)

    @classmethod
    def conv3d(cls, N, D, H, W, C, O, KD=3, KH=3, KW=3, SZ=1, SY=1, SX=1, DZ=1, DY=1, DX=1,
               PF=0, PBk=0, PT=0, PB=0, PL=0, PR=0):
        return cls(N=N, D=D, H=H, W=W, C=C, O=O, KD=KD, KH=KH, KW=KW, SZ=SZ, SY=SY, SX=SX, DZ=DZ, DY=DY,
                   DX=DX, PF=PF, PBk=PBk, PT=PT, PB=PB, PL=PL, PR=PR)

    def as_dict(self):
        return {f[0]: getattr(self, f[0]) for f in self._fields_}

    @property
    def OD(self):
        return (self.D + self.PF + self.PBk - ((self.KD - 1) * self.DZ + 1)) // self.SZ + 1

    @property
    def OH(self):
        return (self.H + self.PT + self.PB - ((self.KH - 1) * self.DY + 1)) // self.SY + 1

    @property
    def OW(self):
        return (self.W + self.PL + self.PR - ((self.KW - 1) * self.DX + 1)) // self.SX + 1

    def x_shape(self):
        return (self.N, self.D, self.H, self.W, self.C)

    def w_shape(self):
        return (self.KD, self.KH, self.KW, self.C, self.O)

    def y_shape(self):
        return (self.N, self.OD, self.OH, self.OW, self.O)

    def flops(self):
        """2*N*OD*OH*OW*O*KD*KH*KW*C, padded taps counted (ConvolutionShared.swift:5343-5349)."""
        return 2 * self.N * self.OD * self.OH * self.OW * self.O * self.KD * self.KH * self.KW * self.C


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        f32p = ctypes.POINTER(ctypes.c_float)
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_bf16_to_f32.restype = ctypes.c_float
        L.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_to_f32.argtypes = [ctypes.c_int, u16p, f32p, ctypes.c_size_t]
        L.oracle_from_f32.argtypes = [ctypes.c_int, f32p, u16p, ctypes.c_size_t]
        L.oracle_fill_uniform.argtypes = [ctypes.c_uint64, ctypes.c_double, ctypes.c_double, ctypes.c_int, u16p,
                                          ctypes.c_size_t]
        L.oracle_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_double, ctypes.c_double, ctypes.c_int, u16p,
                                         ctypes.c_size_t]
        L.oracle_gemm.argtypes = [ctypes.c_int] * 5 + [u16p, u16p, u16p, f32p] + [ctypes.c_int] * 3
        L.oracle_attention.argtypes = [ctypes.c_int] * 8 + [u16p, u16p, u16p, f32p] + [ctypes.c_int] * 3
        L.oracle_permute_oidhw_to_dhwio.argtypes = [u16p, u16p] + [ctypes.c_int] * 5
        L.oracle_attention_bwd.argtypes = ([ctypes.c_int] * 8 + [u16p, u16p, u16p, u16p, f32p, f32p, f32p, f32p]
                                           + [ctypes.c_int] * 3)
        L.oracle_conv_out_d.argtypes = [ctypes.POINTER(ConvDims)]
        L.oracle_conv.argtypes = [ctypes.POINTER(ConvDims), u16p, u16p, u16p, f32p, ctypes.c_long, ctypes.c_long,
                                  ctypes.c_int]
        _lib = L
    return _lib


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def _f32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _dt(dtype):
    return DTYPES[dtype] if isinstance(dtype, str) else int(dtype)


def _wrap(bits: np.ndarray, dtype):
    return bits.view(np.float16) if _dt(dtype) == F16 else bits


# ---------------------------------------------------------------- numbers

def to_f32(x, dtype="f16") -> np.ndarray:
    bits, p = _u16(x)
    out = np.empty(bits.shape, np.float32)
    lib().oracle_to_f32(_dt(dtype), p, _f32p(out), bits.size)
    return out


def from_f32(x, dtype="f16") -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_from_f32(_dt(dtype), _f32p(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), x.size)
    return _wrap(out, dtype)


def uniform(seed: int, shape, lo: float, hi: float, dtype="f16") -> np.ndarray:
    """SplitMix64(seed) -> fp64 uniform [lo, hi) -> RNE to dtype."""
    out = np.empty(int(np.prod(shape)), np.uint16)
    lib().oracle_fill_uniform(seed, lo, hi, _dt(dtype), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                              out.size)
    return _wrap(out.reshape(shape), dtype)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0, dtype="f16") -> np.ndarray:
    """SplitMix64(seed) -> fp64 Box-Muller N(mean, std^2) -> RNE to dtype."""
    out = np.empty(int(np.prod(shape)), np.uint16)
    lib().oracle_fill_normal(seed, mean, std, _dt(dtype), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                             out.size)
    return _wrap(out.reshape(shape), dtype)


# ---------------------------------------------------------------- ops

def gemm(A, B, bias=None, *, trans_b=True, dtype="f16", rows=None, threads=0) -> np.ndarray:
    """fp32 C = bias + A . op(B); A [M][K]; B [N][K] if trans_b else [K][N] (matmul.swift:498-510).

    ``rows=(r0, r1)`` computes only those rows (others are left zero)."""
    a, pa = _u16(A)
    b, pb = _u16(B)
    M, K = a.shape
    N = b.shape[0] if trans_b else b.shape[1]
    assert (b.shape[1] if trans_b else b.shape[0]) == K
    if bias is not None:
        bb, pbias = _u16(bias)
        assert bb.size == N
    else:
        pbias = None
    C = np.zeros((M, N), np.float32)
    r0, r1 = rows if rows is not None else (0, M)
    lib().oracle_gemm(_dt(dtype), M, N, K, 1 if trans_b else 0, pa, pb, pbias, _f32p(C), r0, r1, threads)
    return C


def attention(Q, K, V, *, causal=False, dtype="f16", rows=None, threads=0) -> np.ndarray:
    """fp32 O for Q,K,V laid out [B][S][H][D] (Network.swift:134-179, 286-311). K and V may have
    fewer heads H_kv dividing H: query head h reads K/V head h // (H // H_kv).

    ``rows=(q0, q1)`` computes only those query rows of every (b, h)."""
    q, pq = _u16(Q)
    k, pk = _u16(K)
    v, pv = _u16(V)
    B, Sq, H, D = q.shape
    Skv, Hkv = k.shape[1], k.shape[2]
    assert k.shape == (B, Skv, Hkv, D) and v.shape == k.shape and H % Hkv == 0
    O = np.zeros((B, Sq, H, D), np.float32)
    q0, q1 = rows if rows is not None else (0, Sq)
    lib().oracle_attention(_dt(dtype), B, H, Hkv, Sq, Skv, D, 1 if causal else 0, pq, pk, pv, _f32p(O), q0, q1, threads)
    return O


def attention_bwd(Q, K, V, dO, *, causal=False, dtype="f16", pairs=None, threads=0):
    """fp32 (dQ, dK, dV, Dterm) of the reference's loss sum(dO * O) for Q, K, V, dO laid out
    [B][S][H][D] (Network.swift:205-281, 313-402); Dterm is [B][H][S_q]. K and V may have fewer
    heads H_kv (grouped as in ``attention``); dK and dV then sum over each group's query heads.

    ``pairs=(p0, p1)`` computes only the (b, hk) pairs with flat index b*H_kv + hk in [p0, p1) (with
    every query head of the group); the other slices of the outputs stay zero."""
    q, pq = _u16(Q)
    k, pk = _u16(K)
    v, pv = _u16(V)
    g, pg = _u16(dO)
    B, Sq, H, D = q.shape
    Skv, Hkv = k.shape[1], k.shape[2]
    assert k.shape == (B, Skv, Hkv, D) and v.shape == k.shape and g.shape == q.shape and H % Hkv == 0
    dQ = np.zeros((B, Sq, H, D), np.float32)
    dK = np.zeros((B, Skv, Hkv, D), np.float32)
    dV = np.zeros((B, Skv, Hkv, D), np.float32)
    Dt = np.zeros((B, H, Sq), np.float32)
    p0, p1 = pairs if pairs is not None else (0, -1)
    lib().oracle_attention_bwd(_dt(dtype), B, H, Hkv, Sq, Skv, D, 1 if causal else 0, pq, pk, pv, pg, _f32p(dQ),
                               _f32p(dK), _f32p(dV), _f32p(Dt), p0, p1, threads)
    return dQ, dK, dV, Dt


def permute_oidhw_to_dhwio(w) -> np.ndarray:
    """[O][C][KD][KH][KW] 16-bit weights -> [KD][KH][KW][C][O] (ConvolutionShared.swift:4606-4627)."""
    src, ps = _u16(w)
    O, C, KD, KH, KW = src.shape
    out = np.empty((KD, KH, KW, C, O), np.uint16)
    lib().oracle_permute_oidhw_to_dhwio(ps, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), O, C, KD, KH, KW)
    return out.view(w.dtype) if np.asarray(w).dtype == np.float16 else out


def conv(dims: ConvDims, x, w, bias=None, *, rows=None, threads=0) -> np.ndarray:
    """fp32 NDHWC output of the padded, strided, dilated cross-correlation (f16 inputs)."""
    xx, px = _u16(x)
    ww, pw = _u16(w)
    assert xx.size == int(np.prod(dims.x_shape())) and ww.size == int(np.prod(dims.w_shape()))
    pbias = _u16(bias)[1] if bias is not None else None
    y = np.zeros(dims.y_shape(), np.float32)
    r0, r1 = rows if rows is not None else (0, -1)
    lib().oracle_conv(ctypes.byref(dims), px, pw, pbias, _f32p(y), r0, r1, threads)
    return y


# ---------------------------------------------------------------- acceptance metrics

def rel_frobenius(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    den = np.sqrt(np.sum(e * e))
    num = np.sqrt(np.sum((a - e) ** 2))
    return float(num / den) if den > 0 else float(num)


def ulp(x, dtype="f16") -> np.ndarray:
    """Spacing of the output format at |x| (f16: 10 mantissa bits, bf16: 7)."""
    x = np.abs(np.asarray(x, np.float64))
    mbits, emin = (10, -14) if _dt(dtype) == F16 else (7, -126)
    e = np.floor(np.log2(np.maximum(x, 2.0 ** emin)))
    return 2.0 ** (e - mbits)


def dot_bound(expected, abs_dot, k_len, dtype="f16") -> np.ndarray:
    """Per-element tolerance for an fp32-accumulated K-length dot stored in ``dtype``.

    ulp_out(|yhat|) covers the output's own rounding (half an ulp) plus a binade crossing;
    2 * gamma_K * sum_k |a_k b_k| (gamma_K = K * 2^-24) covers two fp32 sums of the same terms
    in different orders (device vs oracle), each within gamma_K * sum|a b| of the exact value.
    """
    return ulp(expected, dtype) + 2.0 * k_len * 2.0 ** -24 * np.asarray(abs_dot, np.float64)


def compare(actual, expected, *, bound=None, rel_tol=1e-3):
    """Acceptance check used by every parity test.

    * relative Frobenius error ||y - yhat||_F / ||yhat||_F <= rel_tol (1e-3 by default), and
    * when ``bound`` is given, |y - yhat| <= bound element-wise.

    Returns a dict of metrics with ``ok``.
    """
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    fro = rel_frobenius(a, e)
    err = np.abs(a - e)
    res = {"rel_fro": fro, "max_abs": float(err.max()) if err.size else 0.0,
           "ok": bool(fro <= rel_tol) and bool(np.all(np.isfinite(a)))}
    if bound is not None:
        bound = np.broadcast_to(np.asarray(bound, np.float64), err.shape)
        bad = err > bound
        res["n_bad"] = int(bad.sum())
        res["worst_ratio"] = float((err / np.maximum(bound, 1e-30)).max()) if err.size else 0.0
        res["ok"] = res["ok"] and res["n_bad"] == 0
    return res
