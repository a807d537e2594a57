"""ctypes binding of libtcrv_hip.so, the gfx950 runtime library.

The entry points keep the reference's emitted-kernel ABI (parameter roles and
order of ``tcrv_emitc_<kernel>_<variant>``, lib/Conversion/RVV/RVVToEmitC.cpp:
134-145, :258-268) and take caller-owned DEVICE pointers plus a HIP stream.
PyTorch is used only as the device-memory and stream allocator: tensors are
passed by ``data_ptr()``.

Loading fails loudly (``TcrvHipError``) when the library is missing: there is
no CPU fallback anywhere in this module.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
# TCRV_HIP_LIB selects another build of the library (same C-ABI).
LIB_PATH = os.environ.get("TCRV_HIP_LIB") or os.path.join(HERE, "libtcrv_hip.so")

QK = 32
Q8_0_BLOCK_BYTES = 34
Q4_0_BLOCK_BYTES = 18
Q4_0X16_BLOCK_BYTES = 288

OK = 0
ERR_NULL_POINTER = -1
ERR_BAD_SIZE = -2
ERR_MISALIGNED = -3
ERR_TOO_LARGE = -4
ERR_UNSUPPORTED = -5
ERR_SCRATCH_LIMIT = -6

BINARY_ADD, BINARY_SUB, BINARY_MUL = 0, 1, 2
ELEM = {"i8": 0, "u8": 1, "i16": 2, "u16": 3, "i32": 4, "u32": 5, "i64": 6, "f32": 7, "f64": 8}


class TcrvHipError(RuntimeError):
    """A libtcrv_hip call returned a non-zero status, or the library is absent."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_sz = ctypes.c_size_t
_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_int = ctypes.c_int

# name -> argtypes (all return int status, except the string getters)
SIGNATURES = {
    "tcrv_hip_stream_synchronize": [_p],
    "tcrv_hip_add_f32": [_p, _p, _p, _sz, _p],
    "tcrv_hip_add_i32": [_p, _p, _p, _sz, _p],
    "tcrv_hip_binary": [_int, _int, _p, _p, _p, _sz, _p],
    "tcrv_hip_dequantize_row_q8_0": [_p, _p, _sz, _p],
    "tcrv_hip_dequantize_row_q4_0": [_p, _p, _sz, _p],
    "tcrv_hip_quantize_row_q8_0": [_sz, _p, _p, _p],
    "tcrv_hip_q8_0_q8_0_block_dot": [_sz, _p, _p, _p, _p],
    "tcrv_hip_q8_0_q8_0_block_dot_rows": [_sz, _p, _p, _sz, _p, _sz, _sz, _p],
    "tcrv_hip_q4_0_q8_0_block_dot": [_sz, _p, _sz, _p, _sz, _p, _sz, _i32, _p],
    "tcrv_hip_q4_0_q8_0_block_dot_rows": [_sz, _p, _p, _sz, _p, _sz, _sz, _p],
    "tcrv_hip_q8_0_q8_0_block_sums": [_sz, _p, _p, _sz, _p, _sz, _sz, _p],
    "tcrv_hip_q4_0_q8_0_block_sums": [_sz, _p, _p, _sz, _p, _sz, _sz, _p],
    "tcrv_hip_q4_0_q8_0_gemm": [_sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _p],
    "tcrv_hip_q4_0_q8_0_gemm_tile": [_sz, _p, _p, _p, _sz, _sz, _p],
    "tcrv_hip_gemv_q4_0_q8_0": [_sz, _p, _p, _sz, _p, _sz, _p],
    "tcrv_hip_gemv_q4_0_q8_0_shaped": [_sz, _p, _p, _sz, _p, _sz, _i32, _p],
    "tcrv_hip_q8_0_q8_0_gemm": [_sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _p],
    "tcrv_hip_pack_q4_0_to_q4_0x16": [_sz, _p, _p, _p],
    "tcrv_hip_pack_q8_0_to_q8_0x16": [_sz, _p, _p, _p],
    "tcrv_hip_repack_gemv_q4_0_q8_0": [_sz, _p, _p, _p, _sz, _p],
    "tcrv_hip_repack_gemv_q8_0_q8_0": [_sz, _p, _p, _p, _sz, _p],
    "tcrv_hip_repack_gemm_q4_0_q8_0": [_sz, _p, _p, _p, _sz, _sz, _sz, _p],
    "tcrv_hip_pack_q8_0_to_q8_0x4": [_sz, _sz, _p, _sz, _p, _p],
    "tcrv_hip_pack_q4_0_to_soa": [_sz, _sz, _p, _sz, _p, _p],
    "tcrv_hip_gemv_q4_0_soa_q8_0": [_sz, _p, _p, _p, _sz, _p],
    "tcrv_hip_packed_i4_offset_binary_x_i8_product_reduce": [_p, _p, _p, _p, _p, _sz, _p],
    "tcrv_hip_pack_q8_0_to_gemm_tiles": [_sz, _sz, _p, _sz, _p, _p],
    "tcrv_hip_q8_0_q8_0_gemm_tiles": [_sz, _p, _p, _p, _sz, _sz, _sz, _p],
    "tcrv_hip_q8_0_q8_0_gemm_ws": [_sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _p, _sz, _p],
    "tcrv_hip_q8_0_q8_0_gemm_noalloc": [_sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _p],
    "tcrv_hip_pack_q4_0_to_gemm_tiles": [_sz, _sz, _p, _sz, _p, _p],
    "tcrv_hip_q4_0_q8_0_gemm_tiles": [_sz, _p, _p, _p, _sz, _sz, _sz, _p],
    "tcrv_hip_q4_0_q8_0_gemm_ws": [_sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _p, _sz, _p],
}
# size queries (return size_t)
SIZE_FUNCS = {"tcrv_hip_gemm_tiles_bytes": [_sz, _sz],
              "tcrv_hip_q8_0_q8_0_gemm_workspace_bytes": [_sz, _sz, _sz],
              "tcrv_hip_q4_0_q8_0_gemm_workspace_bytes": [_sz, _sz, _sz],
              "tcrv_hip_q8_0_q8_0_gemm_noalloc_max_bytes": []}
STRING_FUNCS = {"tcrv_hip_status_string": [_int], "tcrv_hip_version": []}

_lib: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads libtcrv_hip.so once; raises TcrvHipError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise TcrvHipError(
            ERR_UNSUPPORTED,
            f"libtcrv_hip.so not found at {path}: run __graft_entry__.build() "
            "(make -C tianchen-rv_amd); there is no CPU fallback")
    # PyTorch-ROCm ships its own libamdhip64.  Importing torch first makes the
    # library bind to that same HIP runtime (one runtime per process, so torch's
    # streams and device pointers are valid here); loading the library first
    # maps the system runtime beside torch's, and the second runtime to
    # initialise finds no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _int
    for name, argtypes in STRING_FUNCS.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p
    for name, argtypes in SIZE_FUNCS.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _sz
    _lib = lib
    return lib


def status_string(status: int) -> str:
    return load().tcrv_hip_status_string(status).decode()


def version() -> str:
    return load().tcrv_hip_version().decode()


def _check(name: str, status: int) -> int:
    if status != OK:
        raise TcrvHipError(status, f"{name} failed: {status} ({status_string(status)})")
    return status


def _ptr(t) -> int:
    """Device address of a torch tensor (or an int address / None)."""
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    if not t.is_cuda:
        raise TcrvHipError(ERR_UNSUPPORTED, "libtcrv_hip takes device tensors only")
    return t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def call(name: str, *args, check: bool = True) -> int:
    """Raw call by symbol name; tensor arguments are passed as device addresses."""
    fn = getattr(load(), name)
    conv = []
    for a, t in zip(args, fn.argtypes):
        conv.append(_ptr(a) if t is _p else a)
    status = fn(*conv)
    return _check(name, status) if check else status


# ---------------------------------------------------------------------------
# Typed wrappers in the reference's parameter order (plus a stream).
# ---------------------------------------------------------------------------

def add_f32(lhs, rhs, out, n: Optional[int] = None, stream=None):
    n = lhs.numel() if n is None else n
    return call("tcrv_hip_add_f32", lhs, rhs, out, n, _stream(stream))


def add_i32(lhs, rhs, out, n: Optional[int] = None, stream=None):
    n = lhs.numel() if n is None else n
    return call("tcrv_hip_add_i32", lhs, rhs, out, n, _stream(stream))


def binary(kind: int, elem: str, lhs, rhs, out, n: Optional[int] = None, stream=None):
    """tcrv_rvv.binary: kind BINARY_ADD/SUB/MUL, elem a key of ELEM."""
    n = lhs.numel() if n is None else n
    return call("tcrv_hip_binary", kind, ELEM[elem], lhs, rhs, out, n, _stream(stream))


def dequantize_row_q8_0(vx, y, n: int, stream=None):
    return call("tcrv_hip_dequantize_row_q8_0", vx, y, n, _stream(stream))


def dequantize_row_q4_0(vx, y, n: int, stream=None):
    return call("tcrv_hip_dequantize_row_q4_0", vx, y, n, _stream(stream))


def quantize_row_q8_0(n: int, x, vy, stream=None):
    return call("tcrv_hip_quantize_row_q8_0", n, x, vy, _stream(stream))


def packed_i4_offset_binary_x_i8_product_reduce(w, qlo, qhi, acc, out, n: int, stream=None):
    return call("tcrv_hip_packed_i4_offset_binary_x_i8_product_reduce", w, qlo, qhi, acc, out, n,
                _stream(stream))


def q8_0_q8_0_block_dot(n: int, s, vx, vy, stream=None):
    return call("tcrv_hip_q8_0_q8_0_block_dot", n, s, vx, vy, _stream(stream))


def q8_0_q8_0_block_dot_rows(n: int, s, vx, bx: int, vy, by: int, nrows: int, stream=None):
    return call("tcrv_hip_q8_0_q8_0_block_dot_rows", n, s, vx, bx, vy, by, nrows,
                _stream(stream))


def q4_0_q8_0_block_dot(n: int, s, bs: int, vx, bx: int, vy, by: int, nrc: int, stream=None):
    return call("tcrv_hip_q4_0_q8_0_block_dot", n, s, bs, vx, bx, vy, by, nrc,
                _stream(stream))


def q4_0_q8_0_block_dot_rows(n: int, s, vx, bx: int, vy, by: int, nrows: int, stream=None):
    return call("tcrv_hip_q4_0_q8_0_block_dot_rows", n, s, vx, bx, vy, by, nrows,
                _stream(stream))


def q8_0_q8_0_block_sums(n: int, sumi, vx, bx: int, vy, by: int, nrows: int, stream=None):
    return call("tcrv_hip_q8_0_q8_0_block_sums", n, sumi, vx, bx, vy, by, nrows,
                _stream(stream))


def q4_0_q8_0_block_sums(n: int, sumi, vx, bx: int, vy, by: int, nrows: int, stream=None):
    return call("tcrv_hip_q4_0_q8_0_block_sums", n, sumi, vx, bx, vy, by, nrows,
                _stream(stream))


def q4_0_q8_0_gemm(n: int, s, vx, vy, by: int, nr: int, nc: int, bx: int, bs: int,
                   stream=None):
    return call("tcrv_hip_q4_0_q8_0_gemm", n, s, vx, vy, by, nr, nc, bx, bs, _stream(stream))


def q4_0_q8_0_gemm_tile(n: int, s, vx, vy, by: int, m: int, stream=None):
    return call("tcrv_hip_q4_0_q8_0_gemm_tile", n, s, vx, vy, by, m, _stream(stream))


def gemv_q4_0_q8_0(n: int, s, vx, bx: int, vy, nr: int, stream=None):
    return call("tcrv_hip_gemv_q4_0_q8_0", n, s, vx, bx, vy, nr, _stream(stream))


def gemv_q4_0_q8_0_shaped(n: int, s, vx, bx: int, vy, nr: int, rows_per_wave: int, stream=None,
                          check: bool = True):
    return call("tcrv_hip_gemv_q4_0_q8_0_shaped", n, s, vx, bx, vy, nr, rows_per_wave,
                _stream(stream), check=check)


def q8_0_q8_0_gemm(n: int, s, vx, vy, by: int, nr: int, nc: int, bx: int, bs: int,
                   stream=None):
    return call("tcrv_hip_q8_0_q8_0_gemm", n, s, vx, vy, by, nr, nc, bx, bs, _stream(stream))


def pack_q4_0_to_q4_0x16(nblocks: int, src, dst, stream=None):
    return call("tcrv_hip_pack_q4_0_to_q4_0x16", nblocks, src, dst, _stream(stream))


def pack_q8_0_to_q8_0x16(nblocks: int, src, dst, stream=None):
    return call("tcrv_hip_pack_q8_0_to_q8_0x16", nblocks, src, dst, _stream(stream))


def repack_gemv_q4_0_q8_0(n: int, s, vx, vy, nc: int, stream=None):
    return call("tcrv_hip_repack_gemv_q4_0_q8_0", n, s, vx, vy, nc, _stream(stream))


def repack_gemv_q8_0_q8_0(n: int, s, vx, vy, nc: int, stream=None):
    return call("tcrv_hip_repack_gemv_q8_0_q8_0", n, s, vx, vy, nc, _stream(stream))


def repack_gemm_q4_0_q8_0(n: int, s, vx, vy, nr: int, nc: int, bs: int, stream=None):
    return call("tcrv_hip_repack_gemm_q4_0_q8_0", n, s, vx, vy, nr, nc, bs, _stream(stream))


def pack_q8_0_to_q8_0x4(nrows: int, nb: int, src, by: int, dst, stream=None):
    return call("tcrv_hip_pack_q8_0_to_q8_0x4", nrows, nb, src, by, dst, _stream(stream))


def pack_q4_0_to_soa(nrows: int, nb: int, src, bx: int, dst, stream=None):
    return call("tcrv_hip_pack_q4_0_to_soa", nrows, nb, src, bx, dst, _stream(stream))


def gemv_q4_0_soa_q8_0(n: int, s, vx, vy, nr: int, stream=None):
    return call("tcrv_hip_gemv_q4_0_soa_q8_0", n, s, vx, vy, nr, _stream(stream))


def gemm_tiles_bytes(nrows: int, nb: int) -> int:
    return load().tcrv_hip_gemm_tiles_bytes(nrows, nb)


def pack_q8_0_to_gemm_tiles(nrows: int, nb: int, src, bx: int, dst, stream=None):
    return call("tcrv_hip_pack_q8_0_to_gemm_tiles", nrows, nb, src, bx, dst, _stream(stream))


def q8_0_q8_0_gemm_tiles(n: int, s, tx, ty, nr: int, nc: int, bs: int, stream=None):
    return call("tcrv_hip_q8_0_q8_0_gemm_tiles", n, s, tx, ty, nr, nc, bs, _stream(stream))


def q8_0_q8_0_gemm_workspace_bytes(n: int, nr: int, nc: int) -> int:
    return load().tcrv_hip_q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)


def q8_0_q8_0_gemm_ws(n: int, s, vx, vy, by: int, nr: int, nc: int, bx: int, bs: int, ws,
                      ws_bytes: int, stream=None):
    return call("tcrv_hip_q8_0_q8_0_gemm_ws", n, s, vx, vy, by, nr, nc, bx, bs, ws, ws_bytes,
                _stream(stream))


def q8_0_q8_0_gemm_noalloc_max_bytes() -> int:
    return load().tcrv_hip_q8_0_q8_0_gemm_noalloc_max_bytes()


def q8_0_q8_0_gemm_noalloc(n: int, s, vx, vy, by: int, nr: int, nc: int, bx: int, bs: int,
                           stream=None, check: bool = True):
    """tcrv_hip_q8_0_q8_0_gemm_ws with the library's fixed device scratch as the
    workspace (no allocation); returns the status when check is False."""
    return call("tcrv_hip_q8_0_q8_0_gemm_noalloc", n, s, vx, vy, by, nr, nc, bx, bs,
                _stream(stream), check=check)


def pack_q4_0_to_gemm_tiles(nrows: int, nb: int, src, bx: int, dst, stream=None):
    return call("tcrv_hip_pack_q4_0_to_gemm_tiles", nrows, nb, src, bx, dst, _stream(stream))


def q4_0_q8_0_gemm_tiles(n: int, s, tx, ty, nr: int, nc: int, bs: int, stream=None):
    return call("tcrv_hip_q4_0_q8_0_gemm_tiles", n, s, tx, ty, nr, nc, bs, _stream(stream))


def q4_0_q8_0_gemm_workspace_bytes(n: int, nr: int, nc: int) -> int:
    return load().tcrv_hip_q4_0_q8_0_gemm_workspace_bytes(n, nr, nc)


def q4_0_q8_0_gemm_ws(n: int, s, vx, vy, by: int, nr: int, nc: int, bx: int, bs: int, ws,
                      ws_bytes: int, stream=None):
    return call("tcrv_hip_q4_0_q8_0_gemm_ws", n, s, vx, vy, by, nr, nc, bx, bs, ws, ws_bytes,
                _stream(stream))


def synchronize(stream=None):
    return call("tcrv_hip_stream_synchronize", _stream(stream))


# ---------------------------------------------------------------------------
# libtcrv_hip_route.so: the host-side provider (include/tcrv_hip_route.h).
# ---------------------------------------------------------------------------
ROUTE_LIB_PATH = os.path.join(HERE, "libtcrv_hip_route.so")

QUANT = {"q4_0": 0, "q8_0": 1, "q4_K": 2}
M_DECODE, M_PREFILL = 0, 1
LAYOUT = {"plain": 0, "x16": 1}
ALGO = {0: "decline", 1: "decode_gemv", 2: "repack_gemv", 3: "mfma_gemm", 4: "repack_gemm"}

_cs = ctypes.c_char_p


class Schedule(ctypes.Structure):
    """tcrv_hip_schedule (include/tcrv_hip_route.h)."""
    _fields_ = [("op", _cs), ("m_regime", _int), ("kernel", _cs), ("knob", _cs),
                ("value", ctypes.c_int64), ("is_default", _int), ("entry", _cs),
                ("measured_us", ctypes.c_double), ("reason", _cs)]


ROUTE_SIGNATURES = {
    "tcrv_hip_route_select": ([_int, _int, _int, ctypes.POINTER(_int), ctypes.POINTER(_cs),
                               ctypes.POINTER(_cs)], _int),
    "tcrv_hip_route_m_regime": ([_sz], _int),
    "tcrv_hip_route_binary": ([_int, _int, ctypes.POINTER(_cs), ctypes.POINTER(_cs)], _int),
    "tcrv_hip_route_contraction": ([_int, _int, _sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _p,
                                    ctypes.POINTER(_int)], _int),
    "tcrv_hip_route_count": ([], _sz),
    "tcrv_hip_route_op": ([_sz], _cs),
    "tcrv_hip_route_entry": ([_sz], _cs),
    "tcrv_hip_route_param_count": ([_sz], _sz),
    "tcrv_hip_route_param": ([_sz, _sz, ctypes.POINTER(_cs), ctypes.POINTER(_cs),
                              ctypes.POINTER(_cs)], _int),
    "tcrv_hip_route_find": ([_cs], ctypes.c_long),
    "tcrv_hip_route_schedule_count": ([], _sz),
    "tcrv_hip_route_schedule": ([_sz, ctypes.POINTER(Schedule)], _int),
    "tcrv_hip_route_schedule_default": ([_cs, _int, _cs, ctypes.POINTER(ctypes.c_int64)], _int),
    "tcrv_hip_export_function": ([_cs, _cs, _cs, ctypes.POINTER(ctypes.c_int64), _sz, _int,
                                  ctypes.c_char_p, _sz, ctypes.POINTER(_sz)], _int),
    "tcrv_hip_export_prologue": ([], _cs),
}

EXPORT_DEFINITION, EXPORT_DECLARATION = 0, 1

_route: Optional[ctypes.CDLL] = None


def load_route(path: str = ROUTE_LIB_PATH) -> ctypes.CDLL:
    """Loads the route provider (after libtcrv_hip itself, so both share one
    HIP runtime); raises TcrvHipError if it is not built."""
    global _route
    if _route is not None:
        return _route
    load()
    if not os.path.exists(path):
        raise TcrvHipError(ERR_UNSUPPORTED, f"libtcrv_hip_route.so not found at {path}: run "
                           "__graft_entry__.build()")
    lib = ctypes.CDLL(path)
    for name, (argtypes, restype) in ROUTE_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _route = lib
    return lib


def route_select(quant: str, m_regime: int, layout: str):
    """(algorithm name, audit token, entry symbol or None) for typed facts."""
    lib = load_route()
    algo, reason, entry = _int(), _cs(), _cs()
    st = lib.tcrv_hip_route_select(QUANT[quant], m_regime, LAYOUT[layout], ctypes.byref(algo),
                                   ctypes.byref(reason), ctypes.byref(entry))
    _check("tcrv_hip_route_select", st)
    return ALGO[algo.value], reason.value.decode(), entry.value.decode() if entry.value else None


def route_binary(kind: int, elem: str):
    """(status, entry symbol or None, audit token) for tcrv_rvv.binary's typed
    facts: kind BINARY_ADD/SUB/MUL, elem a key of ELEM."""
    lib = load_route()
    entry, reason = _cs(), _cs()
    st = lib.tcrv_hip_route_binary(kind, ELEM[elem] if isinstance(elem, str) else elem,
                                   ctypes.byref(entry), ctypes.byref(reason))
    return st, entry.value.decode() if entry.value else None, reason.value.decode()


def route_table():
    """The op-identity route table: [{op, entry, params: [(c_name, c_type, role)]}]."""
    lib = load_route()
    rows = []
    for i in range(lib.tcrv_hip_route_count()):
        params = []
        for j in range(lib.tcrv_hip_route_param_count(i)):
            c_name, c_type, role = _cs(), _cs(), _cs()
            _check("tcrv_hip_route_param", lib.tcrv_hip_route_param(
                i, j, ctypes.byref(c_name), ctypes.byref(c_type), ctypes.byref(role)))
            params.append((c_name.value.decode(), c_type.value.decode(), role.value.decode()))
        rows.append({"op": lib.tcrv_hip_route_op(i).decode(),
                     "entry": lib.tcrv_hip_route_entry(i).decode(), "params": params})
    return rows


def route_schedules():
    """The schedule registry: one dict per (op, regime, knob, candidate value)."""
    lib = load_route()
    rows = []
    for i in range(lib.tcrv_hip_route_schedule_count()):
        r = Schedule()
        _check("tcrv_hip_route_schedule", lib.tcrv_hip_route_schedule(i, ctypes.byref(r)))
        rows.append({"op": r.op.decode(), "m_regime": r.m_regime, "kernel": r.kernel.decode(),
                     "knob": r.knob.decode(), "value": r.value, "is_default": bool(r.is_default),
                     "entry": r.entry.decode() if r.entry else None,
                     "measured_us": r.measured_us, "reason": r.reason.decode()})
    return rows


def route_schedule_default(op: str, m_regime: int, knob: str):
    """(status, the default value of `knob` for (op, m_regime) or None)."""
    v = ctypes.c_int64()
    st = load_route().tcrv_hip_route_schedule_default(op.encode(), m_regime, knob.encode(),
                                                      ctypes.byref(v))
    return st, (v.value if st == OK else None)


def export_function(op: str, kernel: str, variant: str, attrs=(), form: int = EXPORT_DEFINITION):
    """(status, C++ text) of the exported tcrv_emitc_<kernel>_<variant> for
    one selected variant of `op`; attrs are the baked-in op facts ({kind,
    element} for tcrv_rvv.binary, {activation_cols} for the GEMM tile)."""
    lib = load_route()
    arr = (ctypes.c_int64 * max(1, len(attrs)))(*attrs)
    need = _sz()
    st = lib.tcrv_hip_export_function(op.encode(), kernel.encode(), variant.encode(), arr,
                                      len(attrs), form, None, 0, ctypes.byref(need))
    if st != OK:
        return st, None
    buf = ctypes.create_string_buffer(need.value)
    st = lib.tcrv_hip_export_function(op.encode(), kernel.encode(), variant.encode(), arr,
                                      len(attrs), form, buf, need.value, None)
    return st, buf.value.decode()


def export_prologue() -> str:
    return load_route().tcrv_hip_export_prologue().decode()


def route_contraction(quant: str, layout: str, n: int, s, vx, vy, by: int, nr: int, nc: int,
                      bx: int, bs: int, stream=None, check: bool = True):
    """Runs a contraction (reference GEMM ABI) on the routed kernel; returns
    (status, algorithm name)."""
    lib = load_route()
    algo = _int(-1)
    st = lib.tcrv_hip_route_contraction(QUANT[quant], LAYOUT[layout], n, _ptr(s), _ptr(vx),
                                        _ptr(vy), by, nr, nc, bx, bs,
                                        _stream(stream) if stream != 0 else 0,
                                        ctypes.byref(algo))
    if check:
        _check("tcrv_hip_route_contraction", st)
    return st, ALGO.get(algo.value)
