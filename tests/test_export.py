"""The host half of the export: tcrv_hip_export_function (libtcrv_hip_route)
and the tcrv_hip_export tool that turns a manifest of selected variants into
the generated C++ of their tcrv_emitc_<kernel>_<variant> functions
(name derivation RVVToEmitC.cpp:167-172; parameters the fixtures'
runtime_abi_value declarations).  CPU only: generation and compilation; the
generated functions run on the GPU in tests/test_harness.py."""
import os
import re
import subprocess

import pytest

import tcrv_hip

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
TOOL = os.path.join(ROOT, "tianchen-rv_amd", "tcrv_hip_export")
MANIFEST = os.path.join(HERE, "harness", "emitc_fixtures.manifest")
PROTOTYPES = os.path.join(HERE, "harness", "emitc_fixture_prototypes.h")
INCLUDE = os.path.join(ROOT, "include")


def manifest_variants():
    rows = []
    for line in open(MANIFEST):
        line = line.split("#", 1)[0].split()
        if line:
            rows.append(line)
    return rows


@pytest.fixture(scope="module")
def generated(tmp_path_factory):
    if not os.path.exists(TOOL):
        pytest.fail("run __graft_entry__.build()")
    out = tmp_path_factory.mktemp("gen")
    cpp, hdr = out / "tcrv_emitc_fixtures.cpp", out / "tcrv_emitc_fixtures.h"
    subprocess.run([TOOL, MANIFEST, str(cpp), str(hdr)], check=True)
    return out, cpp.read_text(), hdr.read_text()


def test_every_fixture_variant_is_exported_by_its_derived_name(generated):
    _, cpp, hdr = generated
    rows = manifest_variants()
    assert len(rows) == 13
    for op, kernel, variant, *_ in rows:
        name = f"tcrv_emitc_{kernel}_{variant}"
        assert re.search(r'extern "C" int ' + name + r"\(", cpp), name
        assert re.search(r'extern "C" int ' + name + r"\([^)]*\);", hdr), name
        # each definition forwards to the op's libtcrv_hip entry
        row = tcrv_hip.load_route().tcrv_hip_route_find(op.encode())
        assert row >= 0, op
        entry = tcrv_hip.load_route().tcrv_hip_route_entry(row).decode()
        body = cpp.split(name + "(", 1)[1].split("}", 1)[0]
        assert f"return {entry}(" in body and body.rstrip().endswith("stream);")


def test_generated_unit_compiles_with_gxx(generated):
    out, _, _ = generated
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-fPIC",
                    "-I" + INCLUDE, "-c", str(out / "tcrv_emitc_fixtures.cpp"), "-o",
                    str(out / "x.o")], check=True)
    syms = subprocess.run(["nm", "--defined-only", str(out / "x.o")], capture_output=True,
                          text=True, check=True).stdout
    assert sum(1 for ln in syms.splitlines() if " T tcrv_emitc_" in ln) == 13


def test_generated_prototypes_match_the_fixtures(generated):
    """The fixtures' prototypes (written by hand from their runtime_abi_value
    declarations) and the generated ones in one translation unit: g++ rejects
    two extern "C" declarations of one name with different parameters."""
    out, _, _ = generated
    tu = out / "check.cpp"
    tu.write_text('#include "tcrv_emitc_fixtures.h"\n#include "emitc_fixture_prototypes.h"\n')
    subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I" + str(out),
                    "-I" + os.path.dirname(PROTOTYPES), str(tu)], check=True)
    # and a planted mismatch (two parameters swapped) is rejected
    bad = out / "bad_prototypes.h"
    text = open(PROTOTYPES).read().replace("size_t nblocks, const uint8_t *src",
                                           "const uint8_t *src, size_t nblocks")
    bad.write_text(text)
    tu.write_text('#include "tcrv_emitc_fixtures.h"\n#include "bad_prototypes.h"\n')
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I" + str(out), str(tu)],
                       capture_output=True, text=True)
    assert r.returncode != 0 and "conflicting declaration" in r.stderr


def test_binary_export_bakes_in_kind_and_element():
    st, text = tcrv_hip.export_function("tcrv_rvv.binary", "k", "v",
                                        (tcrv_hip.BINARY_MUL, tcrv_hip.ELEM["u16"]))
    assert st == tcrv_hip.OK
    assert ("extern \"C\" int tcrv_emitc_k_v(const uint16_t *lhs, const uint16_t *rhs, "
            "uint16_t *out, size_t n, void *stream)") in text
    assert "tcrv_hip_binary(TCRV_HIP_BINARY_MUL, TCRV_HIP_ELEM_U16, lhs, rhs, out, n, stream)" \
        in text
    st, text = tcrv_hip.export_function("tcrv_rvv.binary", "k", "v",
                                        (tcrv_hip.BINARY_ADD, tcrv_hip.ELEM["f64"]),
                                        tcrv_hip.EXPORT_DECLARATION)
    assert st == tcrv_hip.OK
    assert text == ('extern "C" int tcrv_emitc_k_v(const double *lhs, const double *rhs, '
                    "double *out, size_t n, void *stream);\n")


def test_gemm_tile_export_bakes_in_activation_cols():
    st, text = tcrv_hip.export_function("tcrv_rvv.q4_0_q8_0_gemm_tile", "k", "v", (8,))
    assert st == tcrv_hip.OK
    assert "tcrv_hip_q4_0_q8_0_gemm_tile(n, s, vx, vy, by, 8 /* m */, stream)" in text


@pytest.mark.parametrize("op,attrs,form,want", [
    ("tcrv_rvv.no_such_op", (), 0, tcrv_hip.ERR_UNSUPPORTED),
    ("tcrv_rvv.binary", (), 0, tcrv_hip.ERR_BAD_SIZE),              # kind and element missing
    ("tcrv_rvv.binary", (0,), 0, tcrv_hip.ERR_BAD_SIZE),
    ("tcrv_rvv.binary", (3, 4), 0, tcrv_hip.ERR_BAD_SIZE),          # kind outside the grid
    ("tcrv_rvv.binary", (0, 9), 0, tcrv_hip.ERR_BAD_SIZE),          # element outside the grid
    ("tcrv_rvv.q4_0_q8_0_gemm_tile", (), 0, tcrv_hip.ERR_BAD_SIZE),
    ("tcrv_rvv.q4_0_q8_0_gemm_tile", (0,), 0, tcrv_hip.ERR_BAD_SIZE),
    ("tcrv_rvv.quantize_row_q8_0", (), 2, tcrv_hip.ERR_BAD_SIZE),   # unknown form
])
def test_export_rejects(op, attrs, form, want):
    st, text = tcrv_hip.export_function(op, "k", "v", attrs, form)
    assert st == want and text is None


def test_export_truncates_to_the_buffer():
    import ctypes
    lib = tcrv_hip.load_route()
    need = ctypes.c_size_t()
    buf = ctypes.create_string_buffer(16)
    st = lib.tcrv_hip_export_function(b"tcrv_rvv.quantize_row_q8_0", b"k", b"v", None, 0, 0,
                                      buf, 16, ctypes.byref(need))
    assert st == tcrv_hip.OK and len(buf.value) == 15 and need.value > 16


@pytest.mark.parametrize("line,msg", [
    ("tcrv_rvv.no_such_op k v", "no route row for tcrv_rvv.no_such_op"),
    ("tcrv_rvv.binary k v kind=add", "bad attributes for tcrv_rvv.binary"),
    ("tcrv_rvv.binary k v kind=div elem=i32", "unknown attribute: kind=div"),
    ("tcrv_rvv.q4_0_q8_0_gemm_tile k v activation_cols=0", "not a positive integer"),
    ("tcrv_rvv.quantize_row_q8_0 k", "expected <op> <kernel> <variant>"),
])
def test_tool_reports_the_bad_manifest_line(tmp_path, line, msg):
    man = tmp_path / "m.manifest"
    man.write_text("# comment\n\n" + line + "\n")
    r = subprocess.run([TOOL, str(man), str(tmp_path / "o.cpp"), str(tmp_path / "o.h")],
                       capture_output=True, text=True)
    assert r.returncode == 1
    assert f"{man}:3: " in r.stderr and msg in r.stderr
