"""The host-side HIP provider (libtcrv_hip_route.so, include/tcrv_hip_route.h):
the typed-fact selection, the op-identity route table against the C-ABI header
and library, and (-m gpu) routed contractions against the oracle."""
import os
import re
import subprocess

import numpy as np
import pytest

import tcrv_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIP_HEADER = os.path.join(ROOT, "include", "tcrv_hip.h")
ROUTE_HEADER = os.path.join(ROOT, "include", "tcrv_hip_route.h")

# The reference's runtime-ABI role spellings (stringifyRuntimeABIParameterRole,
# include/TianChenRV/Support/RuntimeABI.h:82-) that the hot-path fixtures use.
REFERENCE_ROLES = {
    "lhs-input-buffer", "rhs-input-buffer", "output-buffer", "runtime-element-count",
    "lhs-input-stride", "rhs-input-stride", "output-stride", "source-byte-stride",
    "destination-byte-stride", "rhs-scalar-value", "accumulator-input-buffer",
}
# Values that are not runtime-ABI parameters in the reference but arguments of
# the HIP entry: op attributes and the element type.
NON_ABI = {("tcrv_rvv.q4_0_q8_0_gemm_tile", "m"): "op-attribute",
           ("tcrv_rvv.binary", "kind"): "op-attribute",
           ("tcrv_rvv.binary", "elem"): "element-type"}


# Route rows with no reference op, keyed by the ggml function they restate.
GGML_ONLY = {"ggml.dequantize_row_q8_0", "ggml.dequantize_row_q4_0"}


def header_params(entry):
    """Parameter names of `entry` as declared in include/tcrv_hip.h."""
    text = open(HIP_HEADER).read()
    m = re.search(r"TCRV_HIP_API\s+int\s+" + entry + r"\s*\(([^;]*?)\)\s*;", text, re.S)
    assert m, f"{entry} not declared in tcrv_hip.h"
    names = []
    for part in m.group(1).split(","):
        part = part.strip()
        names.append(re.findall(r"(\w+)\s*$", part)[0])
    return names


def test_route_library_exports_its_header():
    path = tcrv_hip.ROUTE_LIB_PATH
    assert os.path.exists(path), "run __graft_entry__.build()"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines()
                       if ln.split() and ln.split()[-1].startswith("tcrv_")})
    declared = sorted(set(re.findall(r"TCRV_HIP_API\s+[\w\s\*]*?\b(tcrv_hip_(?:route|export)_\w+)\s*\(",
                                     open(ROUTE_HEADER).read())))
    assert exported == declared
    assert set(tcrv_hip.ROUTE_SIGNATURES) == set(declared)


def test_schedule_registry_is_consistent():
    """Every registry row names an op of the route table; each (op, regime,
    knob) has distinct candidate values and exactly one default; a selectable
    row names an entry the C-ABI header declares and libtcrv_hip exports; the
    registry stores no timings (bench.py measures them)."""
    ops = {r["op"] for r in tcrv_hip.route_table()}
    rows = tcrv_hip.route_schedules()
    assert rows
    hip_text = open(HIP_HEADER).read()
    exported = subprocess.run(["nm", "-D", "--defined-only", tcrv_hip.LIB_PATH],
                              capture_output=True, text=True, check=True).stdout
    groups = {}
    for r in rows:
        assert r["op"] in ops, r
        assert r["m_regime"] in (-1, tcrv_hip.M_DECODE, tcrv_hip.M_PREFILL), r
        assert r["measured_us"] == -1 and r["reason"], r
        if r["entry"]:
            assert re.search(r"TCRV_HIP_API\s+int\s+" + r["entry"] + r"\s*\(", hip_text), r
            assert re.search(r"\b" + r["entry"] + r"\b", exported), r
        groups.setdefault((r["op"], r["m_regime"], r["knob"]), []).append(r)
    for key, cands in groups.items():
        values = [c["value"] for c in cands]
        assert len(set(values)) == len(values), key
        assert sum(1 for c in cands if c["is_default"]) == 1, key
        assert len({c["entry"] for c in cands}) == 1, key  # a knob is selectable or not


SCHEDULES = os.path.join(ROOT, "profiles", "schedules.json")


def test_schedule_defaults_match_the_recorded_measurement():
    """profiles/schedules.json is bench.py --only schedules' record (one MI355X):
    every selectable candidate timed at the reference shapes.  At the
    4096-row reference shape the registry's default is the fastest candidate
    (within 1 %); up to 2048 rows the plain entry's rule (2 rows per wave) is."""
    import json
    with open(SCHEDULES) as f:
        rec = json.load(f)
    meas = rec["schedules"]
    sel = [r for r in tcrv_hip.route_schedules() if r["entry"]]
    assert sel
    for (op, regime, knob) in {(r["op"], r["m_regime"], r["knob"]) for r in sel}:
        cands = [r for r in sel if (r["op"], r["m_regime"], r["knob"]) == (op, regime, knob)]
        default = next(r["value"] for r in cands if r["is_default"])
        for rows, want in ((4096, default), (2048, 2)):
            got = {m["value"]: m["us"] for m in meas
                   if (m["op"], m["m_regime"], m["knob"], m["rows"]) == (op, regime, knob, rows)}
            assert set(got) == {r["value"] for r in cands}, (knob, rows)
            assert got[want] <= 1.01 * min(got.values()), (knob, rows, got)


def test_schedule_default_lookup():
    d = tcrv_hip.route_schedule_default
    assert d("tcrv_rvv.q4_0_q8_0_gemm", tcrv_hip.M_DECODE, "rows_per_wave") == (tcrv_hip.OK, 4)
    assert d("tcrv_rvv.q8_0_q8_0_gemm", tcrv_hip.M_PREFILL, "k_chunk_blocks") == (tcrv_hip.OK, 6)
    for regime in (tcrv_hip.M_DECODE, tcrv_hip.M_PREFILL):  # not regime-specific
        assert d("tcrv_rvv.quantize_row_q8_0", regime, "blocks_per_lane_group") == (tcrv_hip.OK, 2)
    assert d("tcrv_rvv.q4_0_q8_0_gemm", tcrv_hip.M_PREFILL, "rows_per_wave")[0] == \
        tcrv_hip.ERR_UNSUPPORTED
    assert d("tcrv_rvv.q4_0_q8_0_gemm", tcrv_hip.M_DECODE, "no_such_knob")[0] == \
        tcrv_hip.ERR_UNSUPPORTED
    assert d("tcrv_rvv.no_such_op", tcrv_hip.M_DECODE, "rows_per_wave")[0] == \
        tcrv_hip.ERR_UNSUPPORTED


@pytest.mark.parametrize("quant,regime,layout,algo,entry", [
    ("q4_0", tcrv_hip.M_DECODE, "plain", "decode_gemv", "tcrv_hip_q4_0_q8_0_gemm"),
    ("q8_0", tcrv_hip.M_DECODE, "plain", "decode_gemv", "tcrv_hip_q8_0_q8_0_gemm"),
    ("q4_0", tcrv_hip.M_PREFILL, "plain", "mfma_gemm", "tcrv_hip_q4_0_q8_0_gemm"),
    ("q8_0", tcrv_hip.M_PREFILL, "plain", "mfma_gemm", "tcrv_hip_q8_0_q8_0_gemm"),
    ("q4_0", tcrv_hip.M_DECODE, "x16", "repack_gemv", "tcrv_hip_repack_gemv_q4_0_q8_0"),
    ("q8_0", tcrv_hip.M_DECODE, "x16", "repack_gemv", "tcrv_hip_repack_gemv_q8_0_q8_0"),
    ("q4_0", tcrv_hip.M_PREFILL, "x16", "repack_gemm", "tcrv_hip_repack_gemm_q4_0_q8_0"),
    ("q8_0", tcrv_hip.M_PREFILL, "x16", "decline", None),
    ("q4_K", tcrv_hip.M_DECODE, "plain", "decline", None),
    ("q4_K", tcrv_hip.M_PREFILL, "plain", "decline", None),
    ("q4_K", tcrv_hip.M_DECODE, "x16", "decline", None),
])
def test_selection_from_typed_facts(quant, regime, layout, algo, entry):
    got_algo, reason, got_entry = tcrv_hip.route_select(quant, regime, layout)
    assert (got_algo, got_entry) == (algo, entry)
    assert reason.startswith("hip-") and " " not in reason
    # the audit token names the fact that carried the decision
    if algo == "decline":
        assert "decline" in reason
    if layout == "x16" and algo != "decline":
        assert "x16" in reason
    if quant != "q4_K":
        assert quant in reason


def test_audit_tokens_are_distinct_per_outcome():
    seen = {}
    for quant in ("q4_0", "q8_0"):
        for regime in (tcrv_hip.M_DECODE, tcrv_hip.M_PREFILL):
            for layout in ("plain", "x16"):
                algo, reason, entry = tcrv_hip.route_select(quant, regime, layout)
                if algo != "decline":
                    assert seen.setdefault(reason, (quant, algo)) == (quant, algo)


def test_selection_rejects_values_outside_the_enums():
    lib = tcrv_hip.load_route()
    import ctypes
    a = ctypes.c_int(-7)
    for facts in ((3, 0, 0), (-1, 0, 0), (0, 2, 0), (0, 0, 2)):
        assert lib.tcrv_hip_route_select(*facts, ctypes.byref(a), None, None) == \
            tcrv_hip.ERR_BAD_SIZE
        assert a.value == -7  # untouched


@pytest.mark.parametrize("kind", [tcrv_hip.BINARY_ADD, tcrv_hip.BINARY_SUB, tcrv_hip.BINARY_MUL])
@pytest.mark.parametrize("elem", list(tcrv_hip.ELEM))
def test_route_binary_typed_facts(kind, elem):
    st, entry, reason = tcrv_hip.route_binary(kind, elem)
    assert st == tcrv_hip.OK and entry == "tcrv_hip_binary"
    assert reason == ("hip-binary-float-ieee" if elem in ("f32", "f64")
                      else "hip-binary-integer-wrapping")


@pytest.mark.parametrize("kind,elem", [(3, 0), (-1, 0), (0, 9), (0, -1)])
def test_route_binary_declines_outside_the_grid(kind, elem):
    st, entry, reason = tcrv_hip.route_binary(kind, elem)
    assert st == tcrv_hip.ERR_UNSUPPORTED and entry is None and reason.startswith("hip-decline")


@pytest.mark.parametrize("nc,regime", [(0, 0), (1, 0), (2, 1), (4096, 1)])
def test_m_regime_from_shape(nc, regime):
    assert tcrv_hip.load_route().tcrv_hip_route_m_regime(nc) == regime


def test_route_table_matches_the_c_abi():
    rows = tcrv_hip.route_table()
    assert len(rows) >= 10
    exported = set(tcrv_hip.SIGNATURES) | set(tcrv_hip.STRING_FUNCS)
    lib = tcrv_hip.load_route()
    for row in rows:
        assert row["op"].startswith("tcrv_rvv.") or row["op"] in GGML_ONLY
        assert row["entry"] in exported
        names = [p[0] for p in row["params"]]
        # the entry takes the op's runtime-ABI parameters in order, then the stream
        assert header_params(row["entry"]) == names + ["stream"], row["entry"]
        for c_name, c_type, role in row["params"]:
            # the gemm tile's column count and the binary op's kind are op
            # attributes in the reference (activation_cols, RVVOps.td:4048-4133;
            # kind, :3217-3243), arguments here, as is the element type
            if (row["op"], c_name) in NON_ABI:
                assert role == NON_ABI[(row["op"], c_name)]
                continue
            assert role in REFERENCE_ROLES, (row["op"], c_name, role)
            assert c_type in ("size_t", "int32_t") or c_type.endswith("*")
        assert lib.tcrv_hip_route_find(row["op"].encode()) == rows.index(row)
    assert lib.tcrv_hip_route_find(b"tcrv_rvv.q4_K_q8_K_block_dot") == -1
    assert lib.tcrv_hip_route_find(None) == -1


def test_route_table_keeps_the_reference_gemm_abi():
    rows = {r["op"]: r for r in tcrv_hip.route_table()}
    gemm = rows["tcrv_rvv.q4_0_q8_0_gemm"]["params"]
    # rvv-to-emitc-q4-0-q8-0-gemm.mlir:23-31
    assert [p[0] for p in gemm] == ["n", "s", "vx", "vy", "by", "nr", "nc", "bx", "bs"]
    assert rows["tcrv_rvv.q8_0_q8_0_gemm"]["params"] == gemm
    rgemm = rows["tcrv_rvv.repack_gemm_q4_0_q8_0"]["params"]
    # rvv-to-emitc-repack-gemm-q4-0-q8-0.mlir:22-28
    assert [p[0] for p in rgemm] == ["n", "s", "vx", "vy", "nr", "nc", "bs"]
    core = rows["tcrv_rvv.packed_i4_offset_binary_x_i8_product"]["params"]
    # rvv-to-emitc-packed-i4-offset-binary-x-i8-product-reduce.mlir:22-27
    assert [p[0] for p in core] == ["w", "qlo", "qhi", "acc", "out", "n"]
    assert core[3] == ("acc", "const int32_t *", "accumulator-input-buffer")
    binary = rows["tcrv_rvv.binary"]["params"]
    # the reference's (lhs, rhs, out, n) after the two typed facts
    assert [p[0] for p in binary] == ["kind", "elem", "lhs", "rhs", "out", "n"]
    assert not any(op.startswith("tcrv_rvv.binary.") for op in rows)  # no names with facts in them
    dot = rows["tcrv_rvv.q4_0_q8_0_block_dot"]["params"]
    # the ggml vec_dot ABI, rvv-to-emitc-q4-0-q8-0-block-dot.mlir:24-31
    assert [p[0] for p in dot] == ["n", "s", "bs", "vx", "bx", "vy", "by", "nrc"]
    assert dot[7] == ("nrc", "int32_t", "rhs-scalar-value")


@pytest.mark.parametrize("quant,layout,nr,nc,bs", [
    ("q4_K", "plain", 16, 1, 1),   # no kernel for the format
    ("q8_0", "x16", 32, 8, 8),     # Q8_0 x16 prefill: no repack GEMM in the reference
    ("q4_0", "x16", 32, 8, 8),     # Q4_0 x16 prefill: the repack GEMM's own ABI differs
    ("q4_0", "x16", 32, 6, 8),     # ... with a partial 4-row activation group
    ("q4_0", "x16", 24, 1, 1),     # x16 decode with a partial 16-row group
    ("q8_0", "x16", 32, 1, 4),     # x16 decode into a strided output
])
def test_declined_contractions_touch_nothing(quant, layout, nr, nc, bs):
    # fake, unmapped addresses: a launch would fault, so the status proves none happened
    st, _ = tcrv_hip.route_contraction(quant, layout, 256, 0x1000, 0x2000, 0x3000, 272, nr, nc,
                                       272, bs, stream=0, check=False)
    assert st == tcrv_hip.ERR_UNSUPPORTED


@pytest.mark.gpu
def test_routed_contractions_match_the_oracle(oracle, dev):
    import torch

    import synth
    from gpu_util import assert_f32_parity, empty_dev, from_dev, to_dev

    # decode, plain Q4_0 rows -> the GEMV
    n, nr = 1024, 512
    w = synth.q4_0_matrix(nr, n, 1006, 0.02)
    x = synth.q8_0_matrix(1, n, 1007, 1.0)
    s = empty_dev(nr, torch.float32, dev)
    _, algo = tcrv_hip.route_contraction("q4_0", "plain", n, s, to_dev(w, dev), to_dev(x, dev),
                                         x.shape[1], nr, 1, w.shape[1], 1)
    assert algo == "decode_gemv"
    assert_f32_parity(from_dev(s), oracle.gemm_q4_0(n, w, x, x.shape[1], nr, 1, w.shape[1], 1, 8),
                      what="routed q4_0 decode")

    # prefill, plain Q8_0 rows -> the MFMA GEMM
    n, nr, nc = 512, 160, 96
    w8 = synth.q8_0_matrix(nr, n, 1009, 0.02)
    a8 = synth.q8_0_matrix(nc, n, 1008, 1.0)
    s = empty_dev(nr * nc, torch.float32, dev)
    _, algo = tcrv_hip.route_contraction("q8_0", "plain", n, s, to_dev(w8, dev), to_dev(a8, dev),
                                         a8.shape[1], nr, nc, w8.shape[1], nc)
    assert algo == "mfma_gemm"
    assert_f32_parity(from_dev(s), oracle.gemm_q8_0(n, w8, a8, a8.shape[1], nr, nc, w8.shape[1],
                                                    nc, 8), what="routed q8_0 prefill")

    # decode over x16 weights -> the repacked GEMV (its own fold)
    n, nr = 512, 64
    nb = n // 32
    for quant, mat, pack, ref, xbytes in (
            ("q4_0", synth.q4_0_matrix, oracle.pack_q4_0x16, oracle.repack_gemv_q4_0, 288),
            ("q8_0", synth.q8_0_matrix, oracle.pack_q8_0x16, oracle.repack_gemv_q8_0, 544)):
        plain = mat(nr, n, 1006, 0.02)
        blk = plain.shape[1] // nb
        # 16 rows x nb blocks per group -> per block index, the 16 rows' blocks
        src = plain.reshape(nr // 16, 16, nb, blk).transpose(0, 2, 1, 3).reshape(-1)
        packed = pack(np.ascontiguousarray(src), nr // 16 * nb)
        x = synth.q8_0_matrix(1, n, 1007, 1.0).reshape(-1)
        s = empty_dev(nr, torch.float32, dev)
        _, algo = tcrv_hip.route_contraction(quant, "x16", n, s, to_dev(packed, dev),
                                             to_dev(x, dev), 0, nr, 1, 0, 1)
        assert algo == "repack_gemv"
        assert packed.size == nr // 16 * nb * xbytes
        assert_f32_parity(from_dev(s), ref(n, packed, x, nr), what=f"routed {quant} x16")

    # prefill over x16 Q4_0 weights: the selection names the repack GEMM, which
    # the caller runs in its own ABI (x4 activations, output activation-row
    # major); the GEMM-ABI call refuses it and writes nothing
    nc = 8
    plain = synth.q4_0_matrix(nr, n, 1006, 0.02)
    src = plain.reshape(nr // 16, 16, nb, 18).transpose(0, 2, 1, 3).reshape(-1)
    packed = oracle.pack_q4_0x16(np.ascontiguousarray(src), nr // 16 * nb)
    a8 = synth.q8_0_matrix(nc, n, 1008, 1.0)
    ax4 = oracle.pack_q8_0x4(a8, nc, nb, a8.shape[1])
    s = to_dev(np.full(nc * nr, -5.0, np.float32), dev)
    st, algo = tcrv_hip.route_contraction("q4_0", "x16", n, s, to_dev(packed, dev),
                                          to_dev(ax4, dev), 0, nr, nc, 0, nr, check=False)
    assert (st, algo) == (tcrv_hip.ERR_UNSUPPORTED, "repack_gemm")
    assert np.all(from_dev(s) == -5.0)
    algo, _, entry = tcrv_hip.route_select("q4_0", tcrv_hip.M_PREFILL, "x16")
    assert (algo, entry) == ("repack_gemm", "tcrv_hip_repack_gemm_q4_0_q8_0")
    tcrv_hip.repack_gemm_q4_0_q8_0(n, s, to_dev(packed, dev), to_dev(ax4, dev), nc, nr, nr)
    assert_f32_parity(from_dev(s), oracle.repack_gemm_q4_0(n, packed, ax4, nc, nr, nr),
                      what="selected q4_0 x16 prefill entry")
