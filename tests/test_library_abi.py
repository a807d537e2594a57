"""CPU checks of the C-ABI boundary: libtcrv_hip.so loads without a GPU,
exports exactly the symbols include/tcrv_hip.h declares, and rejects bad
arguments before any launch (host logic only; no kernel runs here)."""
import os
import re
import subprocess

import pytest

import tcrv_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tcrv_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"TCRV_HIP_API\s+[\w\s\*]*?\b(tcrv_hip_\w+)\s*\(", text)))


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", tcrv_hip.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    return sorted({line.split()[-1] for line in out.splitlines()
                   if line.split() and line.split()[-1].startswith("tcrv_")})


def test_library_is_built():
    assert os.path.exists(tcrv_hip.LIB_PATH), "run __graft_entry__.build()"


def test_exports_exactly_the_header():
    decl = declared_symbols()
    assert len(decl) >= 15
    assert exported_symbols() == decl


def test_binding_covers_the_header():
    bound = set(tcrv_hip.SIGNATURES) | set(tcrv_hip.STRING_FUNCS) | set(tcrv_hip.SIZE_FUNCS)
    assert bound == set(declared_symbols())


def test_loads_and_reports_version_without_gpu():
    tcrv_hip.load()
    assert tcrv_hip.version().startswith("tcrv_hip")
    assert tcrv_hip.status_string(0) == "ok"
    assert "aligned" in tcrv_hip.status_string(tcrv_hip.ERR_MISALIGNED)


@pytest.mark.parametrize("name,args,want", [
    # null pointers
    ("tcrv_hip_add_f32", (0, 16, 32, 8, 0), tcrv_hip.ERR_NULL_POINTER),
    ("tcrv_hip_q8_0_q8_0_gemm", (64, 0, 256, 512, 80, 2, 2, 80, 2, 0), tcrv_hip.ERR_NULL_POINTER),
    # misalignment (fake device addresses: rejected before any launch)
    ("tcrv_hip_add_f32", (2, 16, 32, 8, 0), tcrv_hip.ERR_MISALIGNED),
    ("tcrv_hip_dequantize_row_q8_0", (257, 256, 64, 0), tcrv_hip.ERR_MISALIGNED),
    ("tcrv_hip_dequantize_row_q8_0", (256, 258, 64, 0), tcrv_hip.ERR_MISALIGNED),
    ("tcrv_hip_dequantize_row_q4_0", (257, 256, 64, 0), tcrv_hip.ERR_MISALIGNED),
    ("tcrv_hip_dequantize_row_q4_0", (256, 258, 64, 0), tcrv_hip.ERR_MISALIGNED),
    ("tcrv_hip_dequantize_row_q4_0", (0, 256, 64, 0), tcrv_hip.ERR_NULL_POINTER),
    ("tcrv_hip_q8_0_q8_0_gemm", (64, 256, 257, 512, 80, 2, 2, 80, 2, 0), tcrv_hip.ERR_MISALIGNED),
    ("tcrv_hip_q8_0_q8_0_gemm", (64, 256, 256, 512, 81, 2, 2, 80, 2, 0), tcrv_hip.ERR_MISALIGNED),
    ("tcrv_hip_q8_0_q8_0_block_dot_rows", (64, 256, 256, 69, 512, 68, 2, 0),
     tcrv_hip.ERR_MISALIGNED),
    # bad strides / output row stride
    ("tcrv_hip_q8_0_q8_0_gemm", (64, 256, 256, 512, 66, 2, 2, 80, 2, 0), tcrv_hip.ERR_BAD_SIZE),
    ("tcrv_hip_q8_0_q8_0_gemm", (64, 256, 256, 512, 80, 2, 2, 80, 1, 0), tcrv_hip.ERR_BAD_SIZE),
    ("tcrv_hip_q4_0_q8_0_block_dot_rows", (64, 256, 256, 24, 512, 80, 3, 0),
     tcrv_hip.ERR_BAD_SIZE),
    ("tcrv_hip_gemv_q4_0_q8_0", (64, 256, 512, 34, 1024, 3, 0), tcrv_hip.ERR_BAD_SIZE),
    # the tiled Q8_0 GEMM's 32-bit chunk offsets: at most 1 973 789 blocks (n/32)
    ("tcrv_hip_q8_0_q8_0_gemm_tiles", (1973790 * 32, 256, 512, 1024, 256, 2, 2, 0),
     tcrv_hip.ERR_TOO_LARGE),
])
def test_argument_errors_before_launch(name, args, want):
    assert tcrv_hip.call(name, *args, check=False) == want


@pytest.mark.parametrize("name,args", [
    ("tcrv_hip_q8_0_q8_0_gemm", (64, 256, 256, 512, 80, 0, 2, 80, 2, 0)),
    ("tcrv_hip_q8_0_q8_0_gemm", (64, 256, 256, 512, 80, 2, 0, 80, 2, 0)),
    ("tcrv_hip_q4_0_q8_0_block_sums", (16, 256, 256, 18, 512, 34, 4, 0)),
    ("tcrv_hip_add_f32", (256, 256, 256, 0, 0)),
])
def test_empty_problems_are_no_ops(name, args):
    assert tcrv_hip.call(name, *args, check=False) == tcrv_hip.OK


def test_noalloc_gemm_refuses_shapes_beyond_its_scratch():
    """Checked before any HIP call (fake addresses: nothing may run)."""
    assert tcrv_hip.q8_0_q8_0_gemm_noalloc_max_bytes() == 64 << 20
    nb = 241  # 4096 x 4096 x K 7712: 67.1 MB of GEMM tiles
    st = tcrv_hip.call("tcrv_hip_q8_0_q8_0_gemm_noalloc", nb * 32, 0x1000, 0x2000, 0x3000,
                       nb * 34, 4096, 4096, nb * 34, 4096, 0, check=False)
    assert st == tcrv_hip.ERR_SCRATCH_LIMIT
    assert "scratch" in tcrv_hip.status_string(st)


def test_repack_gemm_argument_checks():
    """Misaligned operands and null pointers are refused before any launch
    (the addresses are fake: nothing may run); empty groups write nothing."""
    call = lambda *a: tcrv_hip.call("tcrv_hip_repack_gemm_q4_0_q8_0", *a, 0, check=False)
    assert call(64, 0x1000, 0x2002, 0x3000, 4, 16, 16) == tcrv_hip.ERR_MISALIGNED
    assert call(64, 0x1000, 0x2000, 0x3002, 4, 16, 16) == tcrv_hip.ERR_MISALIGNED
    assert call(64, 0, 0x2000, 0x3000, 4, 16, 16) == tcrv_hip.ERR_NULL_POINTER
    assert call(64, 0x1000, 0x2000, 0x3000, 3, 16, 16) == tcrv_hip.OK   # no full activation group
    assert call(64, 0x1000, 0x2000, 0x3000, 4, 15, 16) == tcrv_hip.OK   # no full weight group


def test_repack_gemm_rejects_overlapping_rows():
    """Each group writes 4 activation rows at stride bs: a stride shorter than
    the written row is refused before anything runs."""
    st = tcrv_hip.call("tcrv_hip_repack_gemm_q4_0_q8_0", 64, 0x1000, 0x2000, 0x3000, 4, 32, 31, 0,
                       check=False)
    assert st == tcrv_hip.ERR_BAD_SIZE
