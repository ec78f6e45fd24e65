"""C-ABI checks that need no GPU: the library loads, exports every entry point include/mtk.h
declares, refuses to start without a gfx950 device, and its kernel-select / descriptor
validation (dry plans, ctx = NULL) behaves as documented."""
import ctypes
import os
import re

import numpy as np
import pytest

import example_matmul_metal4_amd as mtk
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mtk.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mtk_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    return mtk.lib()


def test_exports_every_declared_symbol(L):
    syms = declared_symbols()
    assert len(syms) >= 25
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    # ...and the Python binding types every one of them
    assert set(syms) <= set(mtk.SIGNATURES), set(syms) - set(mtk.SIGNATURES)


def test_code_objects_hold_every_selectable_kernel():
    blobs = b"".join(open(os.path.join(mtk.LIB_DIR, f), "rb").read()
                     for f in os.listdir(mtk.LIB_DIR) if f.endswith(".hsaco"))
    names = [f"mtk_gemm_{dt}_{lay}_{t}x{t}_{v}" for dt in ("f16", "bf16") for lay in ("nt", "nn") for t in (128, 256)
             for v in ("d", "v1")]
    names += [f"mtk_gemm_{dt}_{lay}_{t}x{t}_d" for dt in ("f16", "bf16") for lay in ("tt", "tn") for t in (128, 256)]
    names += [f"mtk_gemm_{dt}_{lay}_{t}x{t}_s" for dt in ("f16", "bf16") for lay in ("nt", "nn", "tt", "tn")
              for t in (128, 256)]
    names += ["mtk_splitk_reduce_f16", "mtk_splitk_reduce_bf16", "mtk_fill_u16", "mtk_skinny_f16", "mtk_skinny_bf16",
              "mtk_skinny_f16_long", "mtk_skinny_bf16_long", "mtk_skinny_few_f16", "mtk_skinny_few_bf16"]
    names += [f"mtk_attn_fwd_{w}{dt}{c}" for w in ("", "pp_") for dt in ("f16", "bf16") for c in ("", "_causal")]
    names += [f"mtk_conv_f16_fast_{t}_d" for t in ("256x256", "128x128")]
    names += [f"mtk_conv_f16_gen_128x128_v{v}" for v in (8, 4, 1)]
    missing = [n for n in names if n.encode() not in blobs]
    assert not missing, missing


def _kargs_version_header():
    src = open(os.path.join(os.path.dirname(mtk.__file__), "csrc", "kargs.h")).read()
    return int(re.search(r"#define MTK_KARGS_VERSION (\d+)", src).group(1))


def _elf_symbol_bytes(elf: bytes, name: str, size: int) -> bytes:
    """Bytes of a defined symbol of a little-endian ELF64 file (section headers + .symtab)."""
    import struct
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, _ = struct.unpack_from("<HHH", elf, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    for sh in secs:
        if sh[1] != 2:  # SHT_SYMTAB
            continue
        strtab = secs[sh[6]]
        for off in range(sh[4], sh[4] + sh[5], sh[9]):
            st_name, st_info, st_other, st_shndx, st_value, st_size = struct.unpack_from("<IBBHQQ", elf, off)
            end = elf.index(b"\0", strtab[4] + st_name)
            if elf[strtab[4] + st_name:end].decode() == name and 0 < st_shndx < shnum:
                sec = secs[st_shndx]
                at = sec[4] + (st_value - sec[3])
                return elf[at:at + size]
    raise KeyError(name)


def test_code_objects_carry_the_kernel_argument_version(tmp_path):
    # The runtime refuses a code object whose mtk_kargs_version differs from its own; every build
    # output carries the version of the kargs.h it was compiled against.
    import subprocess
    want = _kargs_version_header()
    bundler = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "clang-offload-bundler")
    units = sorted(f for f in os.listdir(mtk.LIB_DIR) if f.endswith(".hsaco"))
    assert units
    for f in units:
        out = tmp_path / (f + ".co")
        subprocess.run([bundler, "--unbundle", "--type=o", f"--input={os.path.join(mtk.LIB_DIR, f)}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={out}"], check=True)
        got = int.from_bytes(_elf_symbol_bytes(out.read_bytes(), "mtk_kargs_version", 4), "little")
        assert got == want, (f, got, want)


def test_init_without_gpu_reports_no_device(L):
    n = ctypes.c_int(-1)
    st = L.mtk_device_count(ctypes.byref(n))
    if st == mtk.MTK_OK and n.value > 0:
        pytest.skip("a GPU is visible")
    h = ctypes.c_void_p()
    assert L.mtk_init(0, None, ctypes.byref(h)) == mtk.MTK_ERR_NO_DEVICE
    assert h.value is None
    assert L.mtk_last_error()
    with pytest.raises(mtk.MtkError) as e:
        mtk.Device()
    assert e.value.status == mtk.MTK_ERR_NO_DEVICE


def test_status_strings(L):
    for s in range(-7, 1):
        assert L.mtk_status_string(s).startswith(b"MTK_")


def test_gemm_kernel_select_dry():
    # config 2: 256 tiles fill the device, so split-K 4 runs in-workgroup (one kernel, one
    # running-sum slot per tile, partition ends staggered over 16 K-tiles); the two-pass schedule
    # (uniform partitions) on request
    p = mtk.GemmPlan(None, 4096, 4096, 4100, has_bias=True, split_k=4)
    d = p.describe()
    assert d.endswith("kernels: mtk_gemm_f16_nt_256x256_s") and "split_k=4" in d and "grid=256 " in d
    assert "k_stagger=16 " in d
    # each tile's running-sum slot: half of the fp32 tile (four of each wavefront's eight blocks)
    assert p.workspace_bytes == 256 * (256 * 256 * 4) // 2
    p = mtk.GemmPlan(None, 4096, 4096, 4100, has_bias=True, split_k=4, split_mode="two_pass")
    d = p.describe()
    assert d.endswith("kernels: mtk_gemm_f16_nt_256x256_d mtk_splitk_reduce_f16") and "grid=1024 " in d
    assert "k_stagger=0 " in d
    assert p.workspace_bytes == 4 * 4096 * 4096 * 4
    # explicit layouts: uniform, a given span, and the largest span that keeps every partition
    # non-empty (65 K-tiles, 17 per partition, the last one 14: span <= 28)
    for ks, want in ((-1, 0), (6, 6), (7, 6), (100, 28)):
        for mode in ("serial", "two_pass"):
            d = mtk.GemmPlan(None, 4096, 4096, 4100, split_k=4, split_mode=mode, k_stagger=ks).describe()
            assert f"k_stagger={want} " in d, (ks, mode, d)
    assert "k_stagger=0 " in mtk.GemmPlan(None, 4096, 4096, 4100, split_k=1, k_stagger=8).describe()
    # 3 K-tiles over 2 partitions (2 + 1): boundaries at K-tile 1 or 2; 2 K-tiles: no room at all
    assert "k_stagger=2 " in mtk.GemmPlan(None, 4096, 4096, 192, split_k=2, k_stagger=8).describe()
    assert "k_stagger=0 " in mtk.GemmPlan(None, 4096, 4096, 128, split_k=2, k_stagger=8).describe()
    # a small tile grid keeps the two-pass schedule (the partitions are the parallelism)
    assert "mtk_splitk_reduce_f16" in mtk.GemmPlan(None, 512, 512, 4100, split_k=4).describe()
    p = mtk.GemmPlan(None, 512, 512, 4100, split_k=4, split_mode="serial")
    # 128x128: one of each wavefront's four blocks in the slot
    assert p.describe().endswith("kernels: mtk_gemm_f16_nt_128x128_s") and p.workspace_bytes == 16 * (128 * 128 * 4) // 4
    assert "_tn_256x256_s" in mtk.GemmPlan(None, 4096, 4096, 512, split_k=2, trans_a=True, trans_b=False,
                                            dtype="bf16").describe()
    p = mtk.GemmPlan(None, 4096, 4096, 4100, has_bias=True, split_k=4)
    flops, byts = p.work()
    assert flops == 2 * 4096 * 4096 * 4100 and byts == 2 * (4096 * 4100 * 2 + 4096 * 4096 + 4096)
    p = mtk.GemmPlan(None, 256, 256, 256, trans_b=False)
    assert "mtk_gemm_f16_nn_128x128_d" in p.describe() and p.workspace_bytes == 0
    p = mtk.GemmPlan(None, 48, 40, 70, dtype="bf16", trans_b=True)
    assert "mtk_gemm_bf16_nt_128x128_d" in p.describe()
    p = mtk.GemmPlan(None, 48, 40, 71, dtype="bf16", trans_b=True)  # odd leading dimension: 2-byte rows
    assert "mtk_gemm_bf16_nt_128x128_v1" in p.describe()
    # the K tail is owned by exactly one split: 65 K-tiles over 4 splits -> 17 per split, 4 splits
    p = mtk.GemmPlan(None, 512, 512, 4100, split_k=4)
    assert "split_k=4 k_tiles/split=17" in p.describe()
    # decode shapes take the HBM-streaming kernel with the K partitions reduced on chip
    # (at most four 16-column groups per workgroup and split-K >= 4: one reduction at the end)
    p = mtk.GemmPlan(None, 16, 14336, 4096, dtype="bf16", has_bias=True, split_k=8)
    assert "mtk_skinny_few_bf16" in p.describe() and "split_k=8" in p.describe() and p.workspace_bytes == 0
    assert "kernels: mtk_skinny_bf16" in mtk.GemmPlan(None, 16, 16400, 4096, dtype="bf16", split_k=8).describe()
    assert "kernels: mtk_skinny_f16" in mtk.GemmPlan(None, 16, 14336, 1024, split_k=2).describe()
    assert "kernels: mtk_skinny_few_f16" in mtk.GemmPlan(None, 16, 16384, 2048, split_k=4).describe()
    assert "mtk_skinny_f16" not in mtk.GemmPlan(None, 17, 64, 64).describe()
    # partitions longer than 512 K: with K >= 2048 and two or more of them, the partial-writing
    # kernel with the same partition count (one workgroup per (partition, 64 columns)) and the
    # two-pass reduce; otherwise the long-partition kernel, which reloads A per pass on a persistent
    # grid (<= one workgroup per CU)
    p = mtk.GemmPlan(None, 8, 14336, 8192, split_k=4)
    assert "skinny partials M=8 N=14336 K=8192 split_k=4 k_tiles/split=32 grid=896 " in p.describe(), p.describe()
    assert p.describe().endswith("kernels: mtk_skinny_parts_f16 mtk_splitk_reduce_f16")
    assert p.workspace_bytes == 4 * 8 * 14336 * 4
    p = mtk.GemmPlan(None, 8, 14336, 8192, split_k=4, split_mode="serial")
    assert "mtk_skinny_f16_long" in p.describe() and "grid=256 " in p.describe()
    p = mtk.GemmPlan(None, 8, 14336, 1536, split_k=2)
    assert "mtk_skinny_f16_long" in p.describe() and p.workspace_bytes == 0
    p = mtk.GemmPlan(None, 8, 14336, 8192, split_k=1)
    assert "mtk_skinny_f16_long" in p.describe() and p.workspace_bytes == 0
    assert "grid=3 " in mtk.GemmPlan(None, 8, 40, 256, split_k=2).describe()
    # transpose.left: A [K][M] through the transposed-read policy; never the skinny path
    p = mtk.GemmPlan(None, 4096, 4096, 4100, has_bias=True, split_k=4, trans_a=True, split_mode="two_pass")
    assert "mtk_gemm_f16_tt_256x256_d" in p.describe() and "A[K][M]" in p.describe()
    assert "mtk_gemm_bf16_tn_128x128_d" in mtk.GemmPlan(None, 16, 64, 64, dtype="bf16", trans_a=True,
                                                          trans_b=False).describe()
    # split-K never produces an empty split
    p = mtk.GemmPlan(None, 64, 64, 100, split_k=8)
    assert "split_k=2 k_tiles/split=1" in p.describe()


def test_gemm_small_m_large_k_plan():
    # the reference's default run (matmul.swift:334): 16 < M <= 32 and long K go to the
    # partial-writing skinny kernel (one workgroup per (partition, 64 columns): 30 x 48) with the
    # requested 30 partitions of 42 K-tiles, then the two-pass reduce
    p = mtk.GemmPlan(None, 32, 3072, 80000, has_bias=True, split_k=30)
    d = p.describe()
    assert "skinny partials M=32 N=3072 K=80000 split_k=30 k_tiles/split=42 grid=1440 " in d, d
    assert d.endswith("kernels: mtk_skinny_parts_f16 mtk_splitk_reduce_f16")
    assert p.workspace_bytes == 30 * 32 * 3072 * 4
    # an explicit tile keeps the tile kernels (128x128: 24 tiles x 30 partitions)
    d = mtk.GemmPlan(None, 32, 3072, 80000, has_bias=True, split_k=30, tile=128).describe()
    assert "tile=128x128 split_k=30 k_tiles/split=42 " in d and "grid=720 " in d
    assert d.endswith("kernels: mtk_gemm_f16_nt_128x128_d mtk_splitk_reduce_f16")
    assert "tile=256x256" in mtk.GemmPlan(None, 32, 3072, 80000, split_k=30, tile=256).describe()
    # the in-workgroup schedule, split-K 1, short K, M <= 16 or transposed operands keep their kernels
    assert "mtk_gemm_f16_nt_128x128_s" in mtk.GemmPlan(None, 32, 3072, 8192, split_k=4, split_mode="serial").describe()
    assert "skinny" not in mtk.GemmPlan(None, 32, 3072, 80000, split_k=1).describe()
    assert "skinny" not in mtk.GemmPlan(None, 32, 3072, 1024, split_k=4).describe()
    assert "skinny partials M=16 N=3072 K=80000 split_k=8 " in mtk.GemmPlan(None, 16, 3072, 80000, split_k=8).describe()
    assert "skinny" not in mtk.GemmPlan(None, 32, 3072, 8192, split_k=4, trans_a=True).describe()
    # the plan's own split: about four workgroups per CU over 48 column blocks
    d = mtk.GemmPlan(None, 24, 3072, 16384, dtype="bf16", split_k=0).describe()
    assert "skinny partials M=24" in d and "mtk_skinny_parts_bf16" in d, d


@pytest.mark.parametrize("kw,status", [
    (dict(M=0, N=4, K=4), mtk.MTK_ERR_INVALID),
    (dict(M=4, N=4, K=-1), mtk.MTK_ERR_INVALID),
    (dict(M=4, N=4, K=8, lda=4), mtk.MTK_ERR_INVALID),
    (dict(M=4, N=4, K=8, ldc=2), mtk.MTK_ERR_INVALID),
    (dict(M=4, N=4, K=8, split_k=-2), mtk.MTK_ERR_INVALID),
    (dict(M=4, N=4, K=8, tile=64), mtk.MTK_ERR_INVALID),
    (dict(M=4, N=4, K=8, split_mode=3), mtk.MTK_ERR_INVALID),
    (dict(M=4, N=4, K=8, k_stagger=-2), mtk.MTK_ERR_INVALID),
    (dict(M=64, N=64, K=2048, split_k=8, split_mode="serial"), mtk.MTK_ERR_UNSUPPORTED),
    (dict(M=64, N=64, K=1024, lda=1025, split_k=2, split_mode="serial"), mtk.MTK_ERR_UNSUPPORTED),
    (dict(M=70000, N=4, K=20000), mtk.MTK_ERR_UNSUPPORTED),
    (dict(M=8, N=4, K=8, trans_a=True, lda=6), mtk.MTK_ERR_INVALID),        # lda < M
    (dict(M=7, N=4, K=8, trans_a=True), mtk.MTK_ERR_UNSUPPORTED),           # odd lda for A [K][M]
])
def test_gemm_descriptor_validation(kw, status):
    M, N, K = kw.pop("M"), kw.pop("N"), kw.pop("K")
    with pytest.raises(mtk.MtkError) as e:
        mtk.GemmPlan(None, M, N, K, **kw)
    assert e.value.status == status and e.value.message


def test_gemm_bad_dtype(L):
    d = mtk.GemmDesc(M=4, N=4, K=4, dtype=7)
    h = ctypes.c_void_p()
    assert L.mtk_gemm_plan(None, ctypes.byref(d), ctypes.byref(h)) == mtk.MTK_ERR_INVALID
    assert b"dtype" in L.mtk_last_error()


def test_dry_plan_refuses_to_run():
    p = mtk.GemmPlan(None, 64, 64, 64)
    with pytest.raises(mtk.MtkError) as e:
        p.run(0x1000, 0x1000, None, 0x1000)
    assert e.value.status == mtk.MTK_ERR_INVALID


def test_conv_kernel_select_and_shapes():
    d = oracle.ConvDims.conv2d(N=8, H=128, W=128, C=256, O=256, PT=1, PB=1, PL=1, PR=1)
    p = mtk.ConvPlan(None, mtk.conv_desc(d, has_bias=True))
    assert "mtk_conv_f16_fast_256x256_d" in p.describe()
    assert p.out_shape() == (8, 128, 128, 256)
    assert p.work()[0] == d.flops() == 154618822656
    d3 = oracle.ConvDims.conv3d(N=1, D=16, H=64, W=64, C=128, O=128, PF=1, PBk=1, PT=1, PB=1, PL=1, PR=1)
    p = mtk.ConvPlan(None, mtk.conv_desc(d3))
    assert "mtk_conv_f16_fast_128x128_d" in p.describe() and p.out_shape() == (1, 16, 64, 64, 128)
    assert p.work()[0] == d3.flops() == 57982058496
    # OIDHW weights: re-laid out in the workspace, then the same convolution (two kernels)
    p = mtk.ConvPlan(None, mtk.conv_desc(d3, weight_layout="OIDHW"))
    assert p.describe().endswith("kernels: mtk_permute_oidhw_dhwio_v8 mtk_conv_f16_fast_128x128_d")
    assert p.workspace_bytes == 27 * 128 * 128 * 2
    # the reference's case lists: every output shape agrees with the oracle's formulas
    import json
    cases = json.load(open(os.path.join(ROOT, "tests", "golden", "cases.json")))
    for kind, spec in cases.items():
        for c in spec["cases"]:
            dims = oracle.ConvDims.conv2d(**c) if "2d" in kind else oracle.ConvDims.conv3d(**c)
            p = mtk.ConvPlan(None, mtk.conv_desc(dims))
            shape = p.out_shape()
            assert shape[1:-1] == ((dims.OH, dims.OW) if len(shape) == 4 else (dims.OD, dims.OH, dims.OW))
            assert "gen_128x128" in p.describe()


@pytest.mark.parametrize("field,value,status", [
    ("rank", 4, mtk.MTK_ERR_INVALID), ("C", 0, mtk.MTK_ERR_INVALID), ("stride_h", 0, mtk.MTK_ERR_INVALID),
    ("pad_left", -1, mtk.MTK_ERR_INVALID), ("KH", 40, mtk.MTK_ERR_UNSUPPORTED), ("H", 1, mtk.MTK_ERR_INVALID),
    ("dtype", mtk.BF16, mtk.MTK_ERR_INVALID), ("pad_front", 1, mtk.MTK_ERR_INVALID),
])
def test_conv_descriptor_validation(field, value, status):
    desc = mtk.conv_desc(oracle.ConvDims.conv2d(N=1, H=5, W=5, C=4, O=8))
    setattr(desc, field, value)
    with pytest.raises(mtk.MtkError) as e:
        mtk.ConvPlan(None, desc)
    assert e.value.status == status


def test_attention_select_and_validation():
    # config 5 -> the 256-row ping-pong kernel, causal -> 128 rows; either on request
    p = mtk.AttentionPlan(None, 2, 32, 4096, 4096, 128, causal=True)
    assert p.describe().endswith("kernels: mtk_attn_fwd_f16_causal") and "rows/wg=128 grid=2048" in p.describe()
    pc = mtk.AttentionPlan(None, 2, 32, 4096, 4096, 128, causal=True, q_rows=256)
    assert pc.describe().endswith("kernels: mtk_attn_fwd_pp_f16_causal") and "rows/wg=256 grid=1024" in pc.describe()
    p256 = mtk.AttentionPlan(None, 2, 32, 4096, 4096, 128)
    assert p256.describe().endswith("kernels: mtk_attn_fwd_pp_f16") and "rows/wg=256 grid=1024" in p256.describe()
    assert mtk.AttentionPlan(None, 2, 32, 4096, 4096, 128, q_rows=128).describe().endswith("kernels: mtk_attn_fwd_f16")
    assert mtk.AttentionPlan(None, 1, 4, 1000, 1000, 128, dtype="bf16").describe().endswith("kernels: mtk_attn_fwd_bf16")
    with pytest.raises(mtk.MtkError) as e:
        mtk.AttentionPlan(None, 1, 1, 16, 16, 128, q_rows=64)
    assert e.value.status == mtk.MTK_ERR_INVALID
    flops = p.work()[0]
    assert flops == 4 * 2 * 32 * 128 * (4096 * 4097 // 2)
    assert mtk.AttentionPlan(None, 2, 32, 4096, 4096, 128).work()[0] == 549755813888
    # head dimensions (the reference's K, any value: attention.swift:398): padded kernel families
    for D, fam in ((64, "d64_"), (8, "d64_"), (96, ""), (136, "d256_"), (256, "d256_"), (1, "g64_"), (100, "g128_"),
                   (255, "g256_")):
        p = mtk.AttentionPlan(None, 1, 2, 300, 300, D)
        assert p.describe().endswith(f"kernels: mtk_attn_fwd_{fam}f16"), (D, p.describe())
        assert p.work()[0] == 4 * 2 * D * 300 * 300
    assert mtk.AttentionPlan(None, 2, 32, 4096, 4096, 64, causal=True).describe().endswith("mtk_attn_fwd_d64_f16_causal")
    # D = 64 exactly: the ping-pong kernel for non-causal grids that fill the device, as at D = 128
    p64 = mtk.AttentionPlan(None, 2, 32, 4096, 4096, 64)
    assert p64.describe().endswith("kernels: mtk_attn_fwd_pp_d64_f16") and "rows/wg=256 grid=1024" in p64.describe()
    assert mtk.AttentionPlan(None, 2, 32, 4096, 4096, 64, q_rows=128).describe().endswith("kernels: mtk_attn_fwd_d64_f16")
    assert mtk.AttentionPlan(None, 1, 2, 300, 300, 64, causal=True, q_rows=256, dtype="bf16").describe().endswith(
        "kernels: mtk_attn_fwd_pp_d64_bf16_causal")
    for D, q_rows, status in ((257, 0, mtk.MTK_ERR_UNSUPPORTED), (0, 0, mtk.MTK_ERR_UNSUPPORTED),
                              (56, 256, mtk.MTK_ERR_UNSUPPORTED), (96, 256, mtk.MTK_ERR_UNSUPPORTED)):
        with pytest.raises(mtk.MtkError) as e:
            mtk.AttentionPlan(None, 1, 1, 16, 16, D, q_rows=q_rows)
        assert e.value.status == status
    for D in (60, 264, 0):  # the backward: multiples of 8 up to 256
        with pytest.raises(mtk.MtkError) as e:
            mtk.AttentionBwdPlan(None, 1, 1, 16, 16, D)
        assert e.value.status == mtk.MTK_ERR_UNSUPPORTED
    # D <= 128: 128-key dK/dV and 256-query dQ workgroups (laid out for 64 up to D = 64); D > 128:
    # 64 keys / 64 queries per workgroup
    b = mtk.AttentionBwdPlan(None, 1, 2, 256, 200, 64)
    assert "grids=32/4/2 " in b.describe() + " " and b.describe().endswith(
        "kernels: mtk_attn_bwd_pre_f16 mtk_attn_bwd_dkdv_d64_f16 mtk_attn_bwd_dq_d64_f16")
    assert mtk.AttentionBwdPlan(None, 1, 2, 256, 200, 72, dtype="bf16", causal=True).describe().endswith(
        "kernels: mtk_attn_bwd_pre_bf16 mtk_attn_bwd_dkdv_bf16_causal mtk_attn_bwd_dq_bf16_causal")
    b = mtk.AttentionBwdPlan(None, 1, 2, 256, 200, 256, causal=True)
    assert "grids=32/8/8 " in b.describe() + " " and b.describe().endswith(
        "kernels: mtk_attn_bwd_pre_f16 mtk_attn_bwd256_dkdv_f16_causal mtk_attn_bwd256_dq_f16_causal")
    with pytest.raises(mtk.MtkError) as e:
        mtk.AttentionPlan(None, 0, 1, 16, 16, 128)
    assert e.value.status == mtk.MTK_ERR_INVALID


def test_attention_grouped_kv_heads_plan():
    # H_kv (the reference's Hk) defaults to H; must divide H; the dK/dV grid runs per K/V head
    assert "H=8 H_kv=8 " in mtk.AttentionPlan(None, 1, 8, 512, 512, 128).describe()
    p = mtk.AttentionPlan(None, 1, 8, 512, 512, 128, H_kv=2)
    assert "H=8 H_kv=2 " in p.describe() and "rows/wg=128 grid=32" in p.describe()  # per query head
    assert p.work()[0] == mtk.AttentionPlan(None, 1, 8, 512, 512, 128).work()[0]
    b = mtk.AttentionBwdPlan(None, 2, 8, 512, 300, 128, H_kv=2)
    assert "grids=512/12/32" in b.describe()  # pre: 2*512*8/16, dkdv: 3 key blocks * 2 * 2, dq: 2 * 2 * 8
    assert b.workspace_bytes == 2 * (2 * 8 * 512 * 4)  # D * scale and the base-2 lse per query row
    for hkv in (3, -1, 16):
        for plan in (mtk.AttentionPlan, mtk.AttentionBwdPlan):
            with pytest.raises(mtk.MtkError) as e:
                plan(None, 1, 8, 64, 64, 128, H_kv=hkv)
            assert e.value.status == mtk.MTK_ERR_INVALID


def test_validate_helper_matches_numpy():
    rng = np.random.default_rng(0)
    e = rng.standard_normal(1000).astype(np.float32)
    a = (e + rng.standard_normal(1000).astype(np.float32) * 1e-3).astype(np.float16)
    r = mtk.validate(a, e, abs_tol=2e-3)
    af = a.astype(np.float64)
    assert abs(r["max_abs_error"] - np.abs(af - e).max()) < 1e-12
    assert r["mismatches"] == int((np.abs(af - e) > 2e-3).sum())
    assert abs(r["rel_frobenius"] - oracle.rel_frobenius(af, e)) < 1e-12
    b = oracle.from_f32(e, "bf16")
    rb = mtk.validate(b, e, abs_tol=0.0, dtype="bf16")
    assert abs(rb["max_abs_error"] - np.abs(oracle.to_f32(b, "bf16") - e).max()) < 1e-12
