"""Static checks on the built gfx950 code objects (CPU only: they disassemble this build's own
`example_matmul_metal4_amd/lib/mtk_*.hsaco`).

A 16-byte (or 12-byte) buffer store whose scalar offset is a register is taken by the compiler's
hazard check to need no wait states before its data registers are rewritten. On gfx950 a VALU
write of those registers in the very next instruction corrupted the stored data: a build of the
in-workgroup split-K kernel with such an instruction pair gave non-repeatable running sums in that
accumulator block. The kernels keep the scalar offset of such stores constant (the compiler then
inserts the wait states), and these tests keep it that way.
"""
import glob
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "example_matmul_metal4_amd", "lib")
LLVM = "/opt/rocm/llvm/bin"
BUNDLER = os.path.join(LLVM, "clang-offload-bundler")
OBJDUMP = os.path.join(LLVM, "llvm-objdump")

STORE = re.compile(r"^\s*(buffer|global)_store_dwordx[34]\s+(v\[\d+:\d+\])")
SGPR_SOFFSET_STORE = re.compile(r"^\s*buffer_store_dwordx[34]\s+v\[\d+:\d+\],\s*v\d+,\s*s\[\d+:\d+\],\s*s\d+\b")
VREG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")


def _regs(text):
    out = set()
    for m in VREG.finditer(text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _code_objects():
    return sorted(glob.glob(os.path.join(LIB, "mtk_*.hsaco")))


def _disassemble(path, tmp):
    elf = os.path.join(tmp, os.path.basename(path) + ".elf")
    subprocess.run([BUNDLER, "--unbundle", "--type=o", f"--input={path}", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--output={elf}"], check=True, capture_output=True)
    out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", elf], check=True, capture_output=True, text=True).stdout
    return [ln.split("//")[0].rstrip() for ln in out.splitlines()]


@pytest.fixture(scope="module")
def listings():
    if not (os.path.exists(BUNDLER) and os.path.exists(OBJDUMP)):
        pytest.skip("ROCm LLVM tools not found")
    objs = _code_objects()
    if not objs:
        pytest.skip("no built code objects (run __graft_entry__.build() first)")
    with tempfile.TemporaryDirectory() as tmp:
        return {os.path.basename(p): _disassemble(p, tmp) for p in objs}


def test_no_wide_buffer_store_with_register_soffset(listings):
    bad = [(name, ln.strip()) for name, lines in listings.items() for ln in lines if SGPR_SOFFSET_STORE.match(ln)]
    assert not bad, f"{len(bad)} 12/16-byte buffer stores with a register scalar offset, e.g. {bad[:3]}"


def test_no_store_data_rewrite_in_next_instruction(listings):
    bad = []
    for name, lines in listings.items():
        ins = [ln.strip() for ln in lines if ln.startswith("\t")]
        for k, ln in enumerate(ins[:-1]):
            m = STORE.match(ln)
            if not m:
                continue
            nxt = ins[k + 1]
            if not nxt.startswith("v_"):
                continue
            dst = nxt.split(None, 1)[1].split(",")[0] if " " in nxt else ""
            if _regs(dst) & _regs(m.group(2)):
                bad.append((name, ln, nxt))
    assert not bad, f"{len(bad)} stores whose data registers the next VALU instruction rewrites, e.g. {bad[:3]}"


def test_checker_finds_the_pattern():
    # the two checks above flag what they are meant to flag
    assert SGPR_SOFFSET_STORE.match("\tbuffer_store_dwordx4 v[182:185], v84, s[12:15], s60 offen nt sc1")
    assert not SGPR_SOFFSET_STORE.match("\tbuffer_store_dwordx4 v[80:83], v87, s[12:15], 0 offen nt sc1")
    m = STORE.match("\tbuffer_store_dwordx4 v[182:185], v84, s[12:15], s60 offen nt sc1")
    assert m and _regs("v185") & _regs(m.group(2))
    assert not _regs("v186") & _regs(m.group(2))
