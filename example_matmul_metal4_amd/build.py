"""Build the gfx950 code objects and the C-ABI host library, in-tree.

    python -m example_matmul_metal4_amd.build

Outputs (under example_matmul_metal4_amd/lib/, git-ignored, shipped with the tree):
  mtk_<unit>.hsaco   one code object per csrc/<unit>.hip, `hipcc --genco --offload-arch=gfx950`
                     (replaces the reference's package.sh `xcrun metal` -> metallib step,
                     Sources/matmul/package.sh:1-3, and its run-time makeLibrary(source:) JIT)
  libmtk.so          host runtime (csrc/runtime.cpp, plus any host HIP units compiled by hipcc)
                     exporting include/mtk.h, linked to libamdhip64
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_UNITS = ["gemm_f16", "gemm_bf16", "conv", "attention", "attention_hd", "attention_bwd", "attention_bwd256", "attention_wide", "skinny",
             "permute", "util"]

HIPCC_FLAGS = [
    "--genco", "--offload-arch=gfx950", "-O3", "-std=c++17",
    # packed fp32 VALU ops stay off in every kernel (hardware issue on these boxes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return time.time() - t0


def hip_unit(unit: str) -> str:
    src = os.path.join(CSRC, unit + ".hip")
    out = os.path.join(LIB, f"mtk_{unit}.hsaco")
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc")] + HIPCC_FLAGS + [src, "-o", tmp])
    os.replace(tmp, out)
    return out


# Host sources compiled by hipcc into the library itself (host code plus a gfx950 device part).
HOST_HIP_UNITS: list[str] = ["scratch"]  # the static device scratch of mtk_gemm_run_noalloc


def host_hip_object(unit: str) -> str:
    out = os.path.join(LIB, f"{unit}.o")
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), "-c", "-fPIC", "--offload-arch=gfx950", "-O2", "-std=c++17",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          os.path.join(CSRC, unit + ".hip"), "-o", tmp])
    os.replace(tmp, out)
    return out


def host_lib() -> str:
    out = os.path.join(LIB, "libmtk.so")
    tmp = out + ".tmp"
    objs = [host_hip_object(u) for u in HOST_HIP_UNITS]
    cxx = shutil.which("g++") or "g++"
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", os.path.join(CSRC, "runtime.cpp")] + objs +
         [f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl", "-o", tmp])
    os.replace(tmp, out)
    return out


def build(units=None, verbose=True) -> list[str]:
    os.makedirs(LIB, exist_ok=True)
    units = [u for u in (units or HIP_UNITS) if os.path.exists(os.path.join(CSRC, u + ".hip"))]
    t0 = time.time()
    outs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, len(units) + 1)) as ex:
        futs = [ex.submit(hip_unit, u) for u in units] + [ex.submit(host_lib)]
        for f in futs:
            outs.append(f.result())
    if verbose:
        print(f"[build] {len(outs)} artefacts in {time.time() - t0:.1f}s -> {LIB}", flush=True)
    return outs


if __name__ == "__main__":
    build(sys.argv[1:] or None)
