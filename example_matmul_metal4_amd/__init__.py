"""MI355X-native tensor-op path (GEMM + bias / split-K, flash-attention forward, conv2d/conv3d).

Python binding of the C ABI in include/mtk.h (libmtk.so + gfx950 code objects under ``lib/``).
It mirrors the reference's host-side verbs -- kernel-select (plans), shape/descriptor setup,
run, validate, profile -- so the parity tests read like the reference's own validation runs:

=====================================================  =========================================
reference (Swift + Metal)                               here
=====================================================  =========================================
MTLCreateSystemDefaultDevice / makeCommandQueue         ``Device()``           (mtk_init)
makeBuffer(.storageModeShared) + contents()             ``Device.upload / download / empty``
createSource + makeLibrary + makeFunction (GEMM)        ``GemmPlan``           (mtk_gemm_plan)
  matmul.swift:18-329, 364-390
createSource + pipeline (attention)                     ``AttentionPlan``      (mtk_attn_plan)
  attention.swift:23-382, 414-450
TensorOpSession*(device:dimensions:...)                 ``ConvPlan``           (mtk_conv_plan)
  ConvolutionShared.swift:856-920, 1002-1060, 1428-1490
dispatchThreadgroups + commit + waitUntilCompleted      ``Plan.run`` + ``Device.sync``
ProfileOptions{warmup, timed, duplicated}               ``Plan.profile``       (mtk_profile)
validateOutput / compareOutputs                         ``validate``           (mtk_validate_f16)
matmul.run / attention.run / TensorOpSession.run        ``gemm`` / ``attention`` / ``conv``
=====================================================  =========================================

There is no fallback: if libmtk.so or the code objects are missing, or there is no gfx950
device, the calls raise. f16 tensors are numpy ``float16``; bf16 tensors are numpy ``uint16``
bit patterns.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")
# $MTK_LIBRARY: another build of the same library (e.g. the host-sanitizer build the tests make)
LIB_PATH = os.environ.get("MTK_LIBRARY") or os.path.join(LIB_DIR, "libmtk.so")

MTK_OK = 0
MTK_ERR_INVALID = -1
MTK_ERR_NO_DEVICE = -2
MTK_ERR_UNSUPPORTED = -3
MTK_ERR_MODULE = -4
MTK_ERR_OOM = -5
MTK_ERR_LAUNCH = -6
MTK_ERR_HIP = -7

# GEMM split-K scheduling (mtk_gemm_desc.split_mode); the result is the same bit for bit
MTK_SPLIT_AUTO = 0
MTK_SPLIT_TWO_PASS = 1
MTK_SPLIT_SERIAL = 2
_SPLIT_MODES = {"auto": MTK_SPLIT_AUTO, "two_pass": MTK_SPLIT_TWO_PASS, "serial": MTK_SPLIT_SERIAL}

F16, BF16, F32 = 0, 1, 2
_DT = {"f16": F16, "bf16": BF16}


class MtkError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


# ------------------------------------------------------------------ ctypes mirror of mtk.h

class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("arch", ctypes.c_char * 32), ("compute_units", ctypes.c_int),
                ("clock_khz", ctypes.c_int), ("lds_bytes_per_cu", ctypes.c_int), ("wavefront_size", ctypes.c_int),
                ("global_mem_bytes", ctypes.c_size_t), ("peak_f16_tflops", ctypes.c_double)]


class GemmDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("M", "N", "K", "lda", "ldb", "ldc", "trans_b", "dtype", "has_bias",
                                            "split_k", "tile", "trans_a", "split_mode", "k_stagger")]


class GemmArgs(ctypes.Structure):
    _fields_ = [("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("C", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p)]


class AttnDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("B", "H", "S_q", "S_kv", "D", "causal", "dtype", "q_rows", "H_kv")]


class AttnArgs(ctypes.Structure):
    _fields_ = [("Q", ctypes.c_void_p), ("K", ctypes.c_void_p), ("V", ctypes.c_void_p), ("O", ctypes.c_void_p),
                ("lse", ctypes.c_void_p)]


class AttnBwdArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("Q", "K", "V", "O", "dO", "lse", "dQ", "dK", "dV", "workspace")]


class ConvDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "rank", "N", "D", "H", "W", "C", "O", "KD", "KH", "KW", "stride_d", "stride_h", "stride_w",
        "dil_d", "dil_h", "dil_w", "pad_front", "pad_back", "pad_top", "pad_bottom", "pad_left", "pad_right",
        "has_bias", "dtype", "weight_layout")]


class ConvArgs(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p)]


class PermuteDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("O", "C", "KD", "KH", "KW")]


class PermuteArgs(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("dst", ctypes.c_void_p)]


class Timing(ctypes.Structure):
    _fields_ = [("total_ms", ctypes.c_double), ("kernel_ms", ctypes.c_double * 4), ("n_kernels", ctypes.c_int),
                ("kernel_names", (ctypes.c_char * 64) * 4)]

    def as_dict(self):
        return {"total_ms": self.total_ms,
                "kernels": {self.kernel_names[i].value.decode(): self.kernel_ms[i] for i in range(self.n_kernels)}}


class Validation(ctypes.Structure):
    _fields_ = [("rel_frobenius", ctypes.c_double), ("max_abs_error", ctypes.c_double),
                ("mismatches", ctypes.c_longlong)]


#: Every entry point declared in include/mtk.h, with (restype, argtypes).
_VP = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
SIGNATURES = {
    "mtk_init": (ctypes.c_int, [ctypes.c_int, ctypes.c_char_p, _PP]),
    "mtk_destroy": (ctypes.c_int, [_VP]),
    "mtk_last_error": (ctypes.c_char_p, []),
    "mtk_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "mtk_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "mtk_get_device_info": (ctypes.c_int, [_VP, ctypes.POINTER(DeviceInfo)]),
    "mtk_alloc": (ctypes.c_int, [_VP, ctypes.c_size_t, _PP]),
    "mtk_free": (ctypes.c_int, [_VP, _VP]),
    "mtk_upload": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_size_t]),
    "mtk_download": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_size_t]),
    "mtk_fill_u16": (ctypes.c_int, [_VP, _VP, ctypes.c_uint16, ctypes.c_size_t]),
    "mtk_sync": (ctypes.c_int, [_VP]),
    "mtk_set_stream": (ctypes.c_int, [_VP, _VP]),
    "mtk_gemm_plan": (ctypes.c_int, [_VP, ctypes.POINTER(GemmDesc), _PP]),
    "mtk_gemm_run": (ctypes.c_int, [_VP, ctypes.POINTER(GemmArgs)]),
    "mtk_gemm_run_noalloc": (ctypes.c_int, [_VP, ctypes.POINTER(GemmArgs)]),
    "mtk_attn_plan": (ctypes.c_int, [_VP, ctypes.POINTER(AttnDesc), _PP]),
    "mtk_attn_run": (ctypes.c_int, [_VP, ctypes.POINTER(AttnArgs)]),
    "mtk_attn_bwd_plan": (ctypes.c_int, [_VP, ctypes.POINTER(AttnDesc), _PP]),
    "mtk_attn_bwd_run": (ctypes.c_int, [_VP, ctypes.POINTER(AttnBwdArgs)]),
    "mtk_conv_plan": (ctypes.c_int, [_VP, ctypes.POINTER(ConvDesc), _PP]),
    "mtk_conv_out_shape": (ctypes.c_int, [ctypes.POINTER(ConvDesc)] + [ctypes.POINTER(ctypes.c_int)] * 3),
    "mtk_conv_run": (ctypes.c_int, [_VP, ctypes.POINTER(ConvArgs)]),
    "mtk_permute_plan": (ctypes.c_int, [_VP, ctypes.POINTER(PermuteDesc), _PP]),
    "mtk_permute_run": (ctypes.c_int, [_VP, ctypes.POINTER(PermuteArgs)]),
    "mtk_plan_workspace_bytes": (ctypes.c_size_t, [_VP]),
    "mtk_plan_describe": (ctypes.c_int, [_VP, ctypes.c_char_p, ctypes.c_size_t]),
    "mtk_plan_work": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "mtk_plan_destroy": (ctypes.c_int, [_VP]),
    "mtk_profile": (ctypes.c_int, [_VP, _VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Timing)]),
    "mtk_graph_create": (ctypes.c_int, [_VP, _VP, ctypes.c_int, ctypes.c_int, _PP]),
    "mtk_graph_launch": (ctypes.c_int, [_VP]),
    "mtk_graph_destroy": (ctypes.c_int, [_VP]),
    "mtk_validate_f16": (ctypes.c_int, [_VP, ctypes.c_int, _VP, ctypes.c_size_t, ctypes.c_double,
                                        ctypes.POINTER(Validation)]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libmtk.so (built by ``example_matmul_metal4_amd.build``); raises if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m example_matmul_metal4_amd.build` "
                              "(this package has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(status: int):
    if status != MTK_OK:
        raise MtkError(status, lib().mtk_last_error().decode())


def _bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a
    if a.dtype == np.uint16:
        return a
    raise TypeError(f"16-bit storage expected (float16 or uint16 bf16 bits), got {a.dtype}")


# ------------------------------------------------------------------ device and buffers

class DeviceBuffer:
    def __init__(self, device: "Device", ptr: int, nbytes: int):
        self.device = device
        self.ptr = ptr
        self.nbytes = nbytes

    def free(self):
        if self.ptr:
            _check(lib().mtk_free(self.device.handle, ctypes.c_void_p(self.ptr)))
            self.ptr = 0

    def __int__(self):
        return self.ptr


class Device:
    """A context on one gfx950 GPU: its stream and the loaded code objects."""

    def __init__(self, device: int = 0, code_object_dir: str | None = None):
        h = ctypes.c_void_p()
        d = code_object_dir.encode() if code_object_dir else None
        _check(lib().mtk_init(device, d, ctypes.byref(h)))
        self.handle = h
        self._buffers: list[DeviceBuffer] = []

    @property
    def info(self) -> dict:
        i = DeviceInfo()
        _check(lib().mtk_get_device_info(self.handle, ctypes.byref(i)))
        return {"name": i.name.decode(), "arch": i.arch.decode(), "compute_units": i.compute_units,
                "clock_khz": i.clock_khz, "lds_bytes_per_cu": i.lds_bytes_per_cu,
                "wavefront_size": i.wavefront_size, "global_mem_bytes": i.global_mem_bytes,
                "peak_f16_tflops": i.peak_f16_tflops}

    def empty(self, nbytes: int) -> DeviceBuffer:
        p = ctypes.c_void_p()
        _check(lib().mtk_alloc(self.handle, nbytes, ctypes.byref(p)))
        b = DeviceBuffer(self, p.value, nbytes)
        self._buffers.append(b)
        return b

    def upload(self, host: np.ndarray) -> DeviceBuffer:
        host = np.ascontiguousarray(host)
        b = self.empty(host.nbytes)
        _check(lib().mtk_upload(self.handle, ctypes.c_void_p(b.ptr), host.ctypes.data_as(ctypes.c_void_p), host.nbytes))
        return b

    def upload_into(self, buf: DeviceBuffer, host: np.ndarray):
        """Copy host data into an existing buffer (ordered on the context's stream, then waits)."""
        host = np.ascontiguousarray(host)
        assert host.nbytes <= buf.nbytes
        _check(lib().mtk_upload(self.handle, ctypes.c_void_p(buf.ptr), host.ctypes.data_as(ctypes.c_void_p), host.nbytes))

    def download(self, buf: DeviceBuffer, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= buf.nbytes
        _check(lib().mtk_download(self.handle, out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(buf.ptr),
                                  out.nbytes))
        return out

    def fill_u16(self, buf: DeviceBuffer, value: int, count: int):
        _check(lib().mtk_fill_u16(self.handle, ctypes.c_void_p(buf.ptr), value, count))

    def sync(self):
        _check(lib().mtk_sync(self.handle))

    def close(self):
        if self.handle:
            for b in self._buffers:
                if b.ptr:
                    b.free()
            self._buffers.clear()
            lib().mtk_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ------------------------------------------------------------------ plans (kernel-select)

class _Plan:
    _args_type = None
    _run_fn = None

    def __init__(self, handle):
        self.handle = handle

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                lib().mtk_plan_destroy(self.handle)
                self.handle = None
        except Exception:
            pass

    @property
    def workspace_bytes(self) -> int:
        return int(lib().mtk_plan_workspace_bytes(self.handle))

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(1024)
        _check(lib().mtk_plan_describe(self.handle, buf, 1024))
        return buf.value.decode()

    def work(self) -> tuple[float, float]:
        """(algorithmic FLOPs, minimum HBM bytes) of one run."""
        f, b = ctypes.c_double(), ctypes.c_double()
        _check(lib().mtk_plan_work(self.handle, ctypes.byref(f), ctypes.byref(b)))
        return f.value, b.value

    def _run(self, args):
        _check(getattr(lib(), self._run_fn)(self.handle, ctypes.byref(args)))

    def launch(self, args):
        """Enqueue one run with prepared arguments (from ``args(...)``) on the context's stream."""
        self._run(args)

    def profile(self, arg_sets, warmup: int = 2, iters: int = 10) -> dict:
        """ProfileOptions{warmupIterations, timedIterations}: per-kernel average ms over ``iters``."""
        arr = (self._args_type * len(arg_sets))(*arg_sets)
        t = Timing()
        _check(lib().mtk_profile(self.handle, ctypes.cast(arr, ctypes.c_void_p), len(arg_sets), warmup, iters,
                                 ctypes.byref(t)))
        return t.as_dict()

    def graph(self, arg_sets, steps: int) -> "Graph":
        """`steps` runs (argument set i % len(arg_sets) for run i) recorded as one HIP graph: the
        duplicatedCount dispatches of one command buffer. The argument buffers must outlive it."""
        arr = (self._args_type * len(arg_sets))(*arg_sets)
        h = ctypes.c_void_p()
        _check(lib().mtk_graph_create(self.handle, ctypes.cast(arr, ctypes.c_void_p), len(arg_sets), steps,
                                      ctypes.byref(h)))
        return Graph(h)


class Graph:
    """An instantiated HIP graph of repeated plan runs (mtk_graph_*)."""

    def __init__(self, handle):
        self.handle = handle

    def launch(self):
        """Enqueue every recorded run on the context's stream (does not wait)."""
        _check(lib().mtk_graph_launch(self.handle))

    def close(self):
        if getattr(self, "handle", None):
            lib().mtk_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ptr(x):
    if x is None:
        return None
    return x.ptr if isinstance(x, DeviceBuffer) else int(x)


class GemmPlan(_Plan):
    """C[M][N] = bias + op(A) . op(B); A is [M][K] (default) or [K][M] when trans_a (the reference's
    transpose.left); B is [N][K] when trans_b (the reference default) else [K][N].

    k_stagger: split-K partition layout (0 = the plan's choice, -1 = uniform, > 0 = span of the
    per-tile boundary offsets in K-tiles); two plans with the same layout give the same result
    bit for bit whatever their split_mode."""

    _args_type = GemmArgs
    _run_fn = "mtk_gemm_run"

    def __init__(self, device: Device | None, M, N, K, *, trans_b=True, dtype="f16", has_bias=False, split_k=1,
                 tile=0, lda=0, ldb=0, ldc=0, trans_a=False, split_mode="auto", k_stagger=0):
        self.desc = GemmDesc(M=M, N=N, K=K, lda=lda, ldb=ldb, ldc=ldc, trans_b=1 if trans_b else 0,
                             dtype=_DT[dtype], has_bias=1 if has_bias else 0, split_k=split_k, tile=tile,
                             trans_a=1 if trans_a else 0,
                             split_mode=_SPLIT_MODES[split_mode] if isinstance(split_mode, str) else split_mode,
                             k_stagger=k_stagger)
        h = ctypes.c_void_p()
        _check(lib().mtk_gemm_plan(device.handle if device else None, ctypes.byref(self.desc), ctypes.byref(h)))
        super().__init__(h)

    @staticmethod
    def args(A, B, bias, C, workspace=None) -> GemmArgs:
        return GemmArgs(A=_ptr(A), B=_ptr(B), bias=_ptr(bias), C=_ptr(C), workspace=_ptr(workspace))

    def run(self, A, B, bias, C, workspace=None):
        self._run(self.args(A, B, bias, C, workspace))


class AttentionPlan(_Plan):
    """O = softmax(Q K^T / sqrt(D)) V per (batch, head); Q, O [B][S_q][H][D], K, V [B][S_kv][H_kv][D]
    (H_kv = 0: H; query head h reads K/V head h // (H // H_kv)), head dimension D = 1..256."""

    _args_type = AttnArgs
    _run_fn = "mtk_attn_run"

    def __init__(self, device: Device | None, B, H, S_q, S_kv, D=128, *, causal=False, dtype="f16", q_rows=0,
                 H_kv=0):
        self.desc = AttnDesc(B=B, H=H, S_q=S_q, S_kv=S_kv, D=D, causal=1 if causal else 0, dtype=_DT[dtype],
                             q_rows=q_rows, H_kv=H_kv)
        h = ctypes.c_void_p()
        _check(lib().mtk_attn_plan(device.handle if device else None, ctypes.byref(self.desc), ctypes.byref(h)))
        super().__init__(h)

    @staticmethod
    def args(Q, K, V, O, lse=None) -> AttnArgs:
        return AttnArgs(Q=_ptr(Q), K=_ptr(K), V=_ptr(V), O=_ptr(O), lse=_ptr(lse))

    def run(self, Q, K, V, O, lse=None):
        self._run(self.args(Q, K, V, O, lse))


class AttentionBwdPlan(_Plan):
    """dQ, dK, dV of the loss sum(dO * O) (Network.swift:313-402) from Q, K, V, the forward's O and
    lse, and dO; tensors [B][S][H][D] (K, V, dK, dV with H_kv heads), lse [B][H][S_q] fp32; needs a
    workspace (two per-query row terms)."""

    _args_type = AttnBwdArgs
    _run_fn = "mtk_attn_bwd_run"

    def __init__(self, device: Device | None, B, H, S_q, S_kv, D=128, *, causal=False, dtype="f16", H_kv=0):
        self.desc = AttnDesc(B=B, H=H, S_q=S_q, S_kv=S_kv, D=D, causal=1 if causal else 0, dtype=_DT[dtype], q_rows=0,
                             H_kv=H_kv)
        h = ctypes.c_void_p()
        _check(lib().mtk_attn_bwd_plan(device.handle if device else None, ctypes.byref(self.desc), ctypes.byref(h)))
        super().__init__(h)

    @staticmethod
    def args(Q, K, V, O, dO, lse, dQ, dK, dV, workspace) -> AttnBwdArgs:
        return AttnBwdArgs(Q=_ptr(Q), K=_ptr(K), V=_ptr(V), O=_ptr(O), dO=_ptr(dO), lse=_ptr(lse), dQ=_ptr(dQ),
                           dK=_ptr(dK), dV=_ptr(dV), workspace=_ptr(workspace))

    def run(self, Q, K, V, O, dO, lse, dQ, dK, dV, workspace):
        self._run(self.args(Q, K, V, O, dO, lse, dQ, dK, dV, workspace))


class PermutePlan(_Plan):
    """OIDHW -> DHWIO weight re-layout (WeightPermutationSession3D, ConvolutionShared.swift:1577-1674):
    dst[kd][kh][kw][c][o] = src[o][c][kd][kh][kw] for 16-bit elements."""

    _args_type = PermuteArgs
    _run_fn = "mtk_permute_run"

    def __init__(self, device: Device | None, O, C, KD, KH, KW):
        self.desc = PermuteDesc(O=O, C=C, KD=KD, KH=KH, KW=KW)
        h = ctypes.c_void_p()
        _check(lib().mtk_permute_plan(device.handle if device else None, ctypes.byref(self.desc), ctypes.byref(h)))
        super().__init__(h)

    @staticmethod
    def args(src, dst) -> PermuteArgs:
        return PermuteArgs(src=_ptr(src), dst=_ptr(dst))

    def run(self, src, dst):
        self._run(self.args(src, dst))


def permute_oidhw_to_dhwio(dev: Device, w) -> np.ndarray:
    """[O][C][KD][KH][KW] (or [O][C][KH][KW]) 16-bit weights -> [KD][KH][KW][C][O] on the GPU."""
    w = _bits(w)
    if w.ndim == 4:
        w = w.reshape(w.shape[0], w.shape[1], 1, w.shape[2], w.shape[3])
    O, C, KD, KH, KW = w.shape
    plan = PermutePlan(dev, O, C, KD, KH, KW)
    src = dev.upload(w)
    dst = dev.empty(w.nbytes)
    plan.run(src, dst)
    dev.sync()
    out = dev.download(dst, (KD, KH, KW, C, O), w.dtype)
    src.free()
    dst.free()
    return out


WEIGHTS_DHWIO, WEIGHTS_OIDHW = 0, 1
_WEIGHT_LAYOUTS = {"DHWIO": WEIGHTS_DHWIO, "OIDHW": WEIGHTS_OIDHW}


def conv_desc(dims, has_bias=False, rank=None, weight_layout="DHWIO") -> ConvDesc:
    """Descriptor from any object with the oracle's ConvDims field names (N, D, H, ..., PL, PR).

    rank defaults to 2 when the depth axis is trivial (D = KD = 1, no depth padding), else 3.
    weight_layout "OIDHW": the weights are [O][C][KD][KH][KW] and each run re-lays them out in the
    plan's workspace first (the reference's PermuteThenTensorOpSession3D)."""
    g = (lambda k, dflt=0: getattr(dims, k, dflt))
    if rank is None:
        rank = 2 if (g("D", 1) == 1 and g("KD", 1) == 1 and not g("PF") and not g("PBk")) else 3
    return ConvDesc(rank=rank, N=g("N"), D=g("D", 1), H=g("H"), W=g("W"), C=g("C"), O=g("O"), KD=g("KD", 1),
                    KH=g("KH"), KW=g("KW"), stride_d=g("SZ", 1), stride_h=g("SY", 1), stride_w=g("SX", 1),
                    dil_d=g("DZ", 1), dil_h=g("DY", 1), dil_w=g("DX", 1), pad_front=g("PF"), pad_back=g("PBk"),
                    pad_top=g("PT"), pad_bottom=g("PB"), pad_left=g("PL"), pad_right=g("PR"),
                    has_bias=1 if has_bias else 0, dtype=F16,
                    weight_layout=_WEIGHT_LAYOUTS[weight_layout])


class ConvPlan(_Plan):
    """Implicit-GEMM conv2d/conv3d (NDHWC x DHWIO -> NDHWC), one launch, f16 in, fp32 accumulate."""

    _args_type = ConvArgs
    _run_fn = "mtk_conv_run"

    def __init__(self, device: Device | None, desc: ConvDesc):
        self.desc = desc
        h = ctypes.c_void_p()
        _check(lib().mtk_conv_plan(device.handle if device else None, ctypes.byref(desc), ctypes.byref(h)))
        super().__init__(h)

    def out_shape(self):
        od, oh, ow = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _check(lib().mtk_conv_out_shape(ctypes.byref(self.desc), ctypes.byref(od), ctypes.byref(oh), ctypes.byref(ow)))
        d = self.desc
        return (d.N, od.value, oh.value, ow.value, d.O) if d.rank == 3 else (d.N, oh.value, ow.value, d.O)

    @staticmethod
    def args(x, w, bias, y, workspace=None) -> ConvArgs:
        return ConvArgs(x=_ptr(x), w=_ptr(w), bias=_ptr(bias), y=_ptr(y), workspace=_ptr(workspace))

    def run(self, x, w, bias, y, workspace=None):
        self._run(self.args(x, w, bias, y, workspace))


# ------------------------------------------------------------------ harness-level calls

def gemm(dev: Device, A, B, bias=None, *, trans_b=True, dtype="f16", split_k=1, tile=0,
         trans_a=False, split_mode="auto") -> np.ndarray:
    """matmul.run equivalent: upload, plan, run, read back C (same 16-bit dtype as the inputs).
    A is [M][K], or [K][M] with trans_a; B is [N][K] with trans_b, else [K][N]."""
    A, B = _bits(A), _bits(B)
    K, M = A.shape if trans_a else A.shape[::-1]
    N = B.shape[0] if trans_b else B.shape[1]
    plan = GemmPlan(dev, M, N, K, trans_b=trans_b, dtype=dtype, has_bias=bias is not None, split_k=split_k, tile=tile,
                    trans_a=trans_a, split_mode=split_mode)
    dA, dB = dev.upload(A), dev.upload(B)
    dbias = dev.upload(_bits(bias)) if bias is not None else None
    dC = dev.empty(M * N * 2)
    ws = dev.empty(plan.workspace_bytes) if plan.workspace_bytes else None
    plan.run(dA, dB, dbias, dC, ws)
    dev.sync()
    out = dev.download(dC, (M, N), A.dtype)
    for b in (dA, dB, dbias, dC, ws):
        if b is not None:
            b.free()
    return out


def attention(dev: Device, Q, K, V, *, causal=False, dtype="f16", q_rows=0, return_lse=False):
    """attention.run equivalent on [B][S][H][D] tensors (K and V may have fewer heads, dividing H);
    with return_lse, also the [B][H][S_q] fp32 row log-sum-exp the backward takes."""
    Q, K, V = _bits(Q), _bits(K), _bits(V)
    B, Sq, H, D = Q.shape
    plan = AttentionPlan(dev, B, H, Sq, K.shape[1], D, causal=causal, dtype=dtype, q_rows=q_rows, H_kv=K.shape[2])
    dQ, dK, dV = dev.upload(Q), dev.upload(K), dev.upload(V)
    dO = dev.empty(Q.nbytes)
    dl = dev.empty(B * H * Sq * 4) if return_lse else None
    plan.run(dQ, dK, dV, dO, dl)
    dev.sync()
    out = dev.download(dO, Q.shape, Q.dtype)
    lse = dev.download(dl, (B, H, Sq), np.float32) if return_lse else None
    for b in (dQ, dK, dV, dO, dl):
        if b is not None:
            b.free()
    return (out, lse) if return_lse else out


def attention_bwd(dev: Device, Q, K, V, O, dO, lse, *, causal=False, dtype="f16"):
    """(dQ, dK, dV) of the loss sum(dO * O) given the forward's O and lse (Network.swift:313-402)."""
    Q, K, V, O, dO = _bits(Q), _bits(K), _bits(V), _bits(O), _bits(dO)
    B, Sq, H, D = Q.shape
    plan = AttentionBwdPlan(dev, B, H, Sq, K.shape[1], D, causal=causal, dtype=dtype, H_kv=K.shape[2])
    bufs = [dev.upload(x) for x in (Q, K, V, O, dO, np.ascontiguousarray(lse, np.float32))]
    outs = [dev.empty(x.nbytes) for x in (Q, K, V)]
    ws = dev.empty(plan.workspace_bytes)
    plan.run(*bufs, *outs, ws)
    dev.sync()
    res = tuple(dev.download(o, x.shape, x.dtype) for o, x in zip(outs, (Q, K, V)))
    for b in bufs + outs + [ws]:
        b.free()
    return res


def conv(dev: Device, dims, x, w, bias=None, *, weight_layout="DHWIO") -> np.ndarray:
    """TensorOpSession*.run equivalent: one implicit-GEMM launch; returns the f16 output. With
    weight_layout "OIDHW", w is [O][C][KD][KH][KW] (rank 2: [O][C][KH][KW]) and the run re-lays it
    out first (PermuteThenTensorOpSession3D.run)."""
    desc = conv_desc(dims, has_bias=bias is not None, weight_layout=weight_layout)
    plan = ConvPlan(dev, desc)
    shape = plan.out_shape()
    dx, dw = dev.upload(_bits(x)), dev.upload(_bits(w))
    db = dev.upload(_bits(bias)) if bias is not None else None
    dy = dev.empty(int(np.prod(shape)) * 2)
    ws = dev.empty(plan.workspace_bytes) if plan.workspace_bytes else None
    plan.run(dx, dw, db, dy, ws)
    dev.sync()
    out = dev.download(dy, shape, np.float16)
    for b in (dx, dw, db, dy, ws):
        if b is not None:
            b.free()
    return out


def validate(actual, expected, abs_tol: float, dtype="f16") -> dict:
    """validateOutput metrics (ConvolutionShared.swift:5174-5246): max-abs error, mismatches above
    ``abs_tol``, plus the relative Frobenius error."""
    a = _bits(actual).reshape(-1)
    e = np.ascontiguousarray(expected, np.float32).reshape(-1)
    assert a.size == e.size
    v = Validation()
    _check(lib().mtk_validate_f16(a.ctypes.data_as(ctypes.c_void_p), _DT[dtype], e.ctypes.data_as(ctypes.c_void_p),
                                  a.size, abs_tol, ctypes.byref(v)))
    return {"rel_frobenius": v.rel_frobenius, "max_abs_error": v.max_abs_error, "mismatches": int(v.mismatches)}


__all__ = ["Device", "DeviceBuffer", "GemmPlan", "AttentionPlan", "ConvPlan", "conv_desc", "gemm", "attention",
           "conv", "validate", "MtkError", "lib", "SIGNATURES"]
