"""mtk_init's code-object failures (the counterpart of the reference's makeLibrary failure path,
Sources/matmul/matmul.swift:364-370): a directory without code objects, a truncated code object and
a code object built for another kernel-argument version must each give MTK_ERR_MODULE with a
message naming the problem. All three fail while the host loads modules; no kernel runs. Each case
runs in a child process so that a loader problem cannot take the test session down with it."""
import json
import os
import shutil
import struct
import subprocess
import sys

import pytest

import example_matmul_metal4_amd as mtk

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import json, sys
sys.path.insert(0, sys.argv[1])
import example_matmul_metal4_amd as mtk
try:
    d = mtk.Device(0, code_object_dir=sys.argv[2])
    d.close()
    print(json.dumps({"status": 0, "message": ""}))
except mtk.MtkError as e:
    print(json.dumps({"status": e.status, "message": e.message}))
"""


def _init_in_child(co_dir):
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT, str(co_dir)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def _copy_code_objects(dst):
    for f in os.listdir(mtk.LIB_DIR):
        if f.endswith(".hsaco"):
            shutil.copy(os.path.join(mtk.LIB_DIR, f), dst / f)


def _symbol_file_offset(blob: bytes, name: str) -> int:
    """File offset of a defined symbol's bytes in an uncompressed offload bundle holding one
    little-endian ELF64 code object (section headers + .symtab)."""
    base = blob.index(b"\x7fELF")
    elf = blob[base:]
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, _ = struct.unpack_from("<HHH", elf, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    for sh in secs:
        if sh[1] != 2:  # SHT_SYMTAB
            continue
        strtab = secs[sh[6]]
        for off in range(sh[4], sh[4] + sh[5], sh[9]):
            st_name, _, _, st_shndx, st_value, _ = struct.unpack_from("<IBBHQQ", elf, off)
            end = elf.index(b"\0", strtab[4] + st_name)
            if elf[strtab[4] + st_name:end].decode() == name and 0 < st_shndx < shnum:
                sec = secs[st_shndx]
                return base + sec[4] + (st_value - sec[3])
    raise KeyError(name)


@pytest.mark.gpu
def test_empty_code_object_directory(tmp_path):
    r = _init_in_child(tmp_path)
    assert r["status"] == mtk.MTK_ERR_MODULE, r
    assert "no mtk_*.hsaco" in r["message"], r


@pytest.mark.gpu
def test_truncated_code_object(tmp_path):
    _copy_code_objects(tmp_path)
    victim = tmp_path / "mtk_util.hsaco"
    blob = victim.read_bytes()
    victim.write_bytes(blob[: blob.index(b"\x7fELF") + 200])  # bundle header + the start of the ELF header
    r = _init_in_child(tmp_path)
    assert r["status"] == mtk.MTK_ERR_MODULE, r
    assert "mtk_util.hsaco" in r["message"], r


@pytest.mark.gpu
def test_stale_kernel_argument_version(tmp_path):
    _copy_code_objects(tmp_path)
    victim = tmp_path / "mtk_util.hsaco"
    blob = bytearray(victim.read_bytes())
    at = _symbol_file_offset(bytes(blob), "mtk_kargs_version")
    have, = struct.unpack_from("<i", blob, at)
    struct.pack_into("<i", blob, at, have - 1)  # a build from an older kargs.h
    victim.write_bytes(bytes(blob))
    r = _init_in_child(tmp_path)
    assert r["status"] == mtk.MTK_ERR_MODULE, r
    assert f"kernel-argument version {have - 1}" in r["message"] and "rebuild" in r["message"], r


def test_symbol_patch_finds_the_version_on_cpu(tmp_path):
    # the patch above lands on the version the runtime checks (no GPU needed)
    blob = open(os.path.join(mtk.LIB_DIR, "mtk_util.hsaco"), "rb").read()
    at = _symbol_file_offset(blob, "mtk_kargs_version")
    import re
    src = open(os.path.join(os.path.dirname(mtk.__file__), "csrc", "kargs.h")).read()
    want = int(re.search(r"#define MTK_KARGS_VERSION (\d+)", src).group(1))
    assert struct.unpack_from("<i", blob, at)[0] == want
