"""The host runtime (csrc/runtime.cpp) built with AddressSanitizer and UndefinedBehaviorSanitizer
runs the C-ABI tests that need no GPU (tests/test_abi.py: descriptor validation, kernel-select of
dry plans, describe / work / destroy, validate, the no-device path) without a sanitizer report.
Host code only: the library's device part (the scratch object) is linked unchanged."""
import os
import shutil
import subprocess
import sys

import pytest

import example_matmul_metal4_amd as mtk

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _runtime(name):
    r = subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def test_dry_plan_abi_tests_under_asan_and_ubsan(tmp_path):
    scratch_obj = os.path.join(mtk.LIB_DIR, "scratch.o")
    asan = _runtime("libasan.so")
    if shutil.which("g++") is None or asan is None or not os.path.exists(scratch_obj):
        pytest.skip("needs g++ with libasan and a built library (python -m example_matmul_metal4_amd.build)")
    lib = tmp_path / "libmtk.so"
    subprocess.run(["g++", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
                    f"-I{ROCM}/include", os.path.join(mtk.PKG, "csrc", "runtime.cpp"), scratch_obj,
                    f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl", "-o", str(lib)],
                   check=True, capture_output=True)
    env = dict(os.environ, LD_PRELOAD=asan, MTK_LIBRARY=str(lib),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    # the child really maps the sanitized build
    probe = ("import example_matmul_metal4_amd as m; m.lib(); "
             "print(any(l.rstrip().endswith(m.LIB_PATH) for l in open('/proc/self/maps')))")
    r = subprocess.run([sys.executable, "-c", probe], env=env, capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "True", r.stdout + r.stderr
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                        os.path.join(ROOT, "tests", "test_abi.py")],
                       env=env, capture_output=True, text=True, cwd=ROOT, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in out
