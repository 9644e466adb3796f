"""ctypes view of the CPU oracle (oracle/exl3_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product path
(plugins_amd/, libexl3_mi355x.so) never imports this module.

Half values are numpy uint16 arrays holding binary16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "libexl3_oracle.so")

CB_MUL1 = 0
CB_MCG = 1
CB_SPEC1 = 2
CB_PAIR1 = 3
CB_STD1 = 4
# the shipped codebook tables (sx/codebook_tables.zig:99-104)
TAB_PAIR1_W16_V1 = 0
TAB_SPEC1_W15 = 1
TAB_SPEC1_W16 = 2
TAB_STD1 = 3
TABLE_NAMES = {TAB_PAIR1_W16_V1: "pair1-w16-v1", TAB_SPEC1_W15: "spec1-w15",
               TAB_SPEC1_W16: "spec1-w16", TAB_STD1: "std1"}


def spec1(table: int) -> int:
    """The `codebook` argument of spec1 decoded with `table`."""
    return CB_SPEC1 | ((table + 1) << 8)

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_int = ctypes.c_int

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "exl3o_h2f": (ctypes.c_float, [ctypes.c_uint16]),
            "exl3o_f2h": (ctypes.c_uint16, [ctypes.c_float]),
            "exl3o_d2h": (ctypes.c_uint16, [ctypes.c_double]),
            "exl3o_bit_end": (_u32, [_u32, _u32]),
            "exl3o_decode_mul1": (ctypes.c_uint16, [ctypes.c_uint16]),
            "exl3o_decode_mcg": (ctypes.c_uint16, [ctypes.c_uint16]),
            "exl3o_mul1_table": (None, [_u16p]),
            "exl3o_table_info": (_int, [_int, ctypes.POINTER(_u32), ctypes.POINTER(_u32),
                                        ctypes.POINTER(_u32)]),
            "exl3o_table_row": (_int, [_int, _u32, ctypes.POINTER(_u32)]),
            "exl3o_decode_hash_mask": (ctypes.c_uint16, [ctypes.c_uint16, _u32, _u32]),
            "exl3o_decode_pair1": (None, [ctypes.c_uint16, ctypes.POINTER(_u32),
                                          ctypes.POINTER(ctypes.c_uint16)]),
            "exl3o_unpack_tile": (None, [_u16p, _u32, _u16p]),
            "exl3o_unpack_tile_bitwise": (None, [_u16p, _u32, _u16p]),
            "exl3o_tile_perm": (None, [_u16p]),
            "exl3o_decode_tile": (None, [_u16p, _u32, _int, _u32, _u16p]),
            "exl3o_reconstruct_inner": (None, [_u16p, _sz, _sz, _u32, _int, _u32, _u16p]),
            "exl3o_reconstruct_public": (None, [_u16p, _u16p, _u16p, _sz, _sz, _u32, _int, _u32, _u16p]),
            "exl3o_hadamard128_dense": (None, [_f32p]),
            "exl3o_hadamard128_butterfly": (None, [_f32p]),
            "exl3o_prepare": (None, [_f32p, _u16p, _sz, _sz, _int, _u16p]),
            "exl3o_inner": (None, [_u16p, _u16p, _sz, _sz, _sz, _u32, _int, _u32, _u16p]),
            "exl3o_finish": (None, [_u16p, _u16p, _sz, _sz, _int, _u16p]),
            "exl3o_project": (None, [_f32p, _u16p, _u16p, _u16p, _sz, _sz, _sz, _u32, _int, _u32, _int, _u16p]),
            "exl3o_route_topk": (None, [_f32p, _sz, _sz, _sz, _i32p, _f32p]),
            "exl3o_moe_swiglu": (None, [_f32p, _sz, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p,
                                        _u16p, _i32p, _f32p, _sz, _sz, _sz, _u32, _int, _u32,
                                        ctypes.c_float, _f32p]),
            "exl3o_synth_plane": (None, [ctypes.c_uint64, _sz, _u16p]),
            "exl3o_set_threads": (None, [_int]),
            "exl3o_get_threads": (_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a).view(np.uint16) if np.asarray(a).dtype == np.int16
                                else np.asarray(a, dtype=np.uint16))


def set_threads(n: int) -> None:
    lib().exl3o_set_threads(int(n))


def threads() -> int:
    return int(lib().exl3o_get_threads())


def bit_end(n: int, t: int) -> int:
    return int(lib().exl3o_bit_end(n, t))


def decode_mul1(cw: int) -> int:
    return int(lib().exl3o_decode_mul1(cw))


def decode_mcg(cw: int) -> int:
    return int(lib().exl3o_decode_mcg(cw))


def mul1_table() -> np.ndarray:
    out = np.empty(65536, np.uint16)
    lib().exl3o_mul1_table(out)
    return out


def table_info(table: int):
    """(n_lo, rows, fields) of a shipped table, or None."""
    n_lo, rows, fields = _u32(), _u32(), _u32()
    if not lib().exl3o_table_info(table, ctypes.byref(n_lo), ctypes.byref(rows), ctypes.byref(fields)):
        return None
    return n_lo.value, rows.value, fields.value


def table_row(table: int, n: int):
    """The table's row for rate n as a 4-tuple, or None."""
    row = (_u32 * 4)()
    if not lib().exl3o_table_row(table, n, row):
        return None
    return tuple(int(v) for v in row)


def decode_hash_mask(cw: int, mult: int, mask: int) -> int:
    return int(lib().exl3o_decode_hash_mask(cw, mult, mask))


def decode_pair1(cw: int, row) -> tuple:
    r = (_u32 * 4)(*row)
    out = (ctypes.c_uint16 * 2)()
    lib().exl3o_decode_pair1(cw, r, out)
    return int(out[0]), int(out[1])


def mcg_table() -> np.ndarray:
    return np.array([decode_mcg(c) for c in range(65536)], np.uint16)


def unpack_tile(words, n: int, bitwise: bool = False) -> np.ndarray:
    out = np.empty(256, np.uint16)
    w = _u16(words)
    (lib().exl3o_unpack_tile_bitwise if bitwise else lib().exl3o_unpack_tile)(w, n, out)
    return out


def tile_perm() -> np.ndarray:
    out = np.empty(256, np.uint16)
    lib().exl3o_tile_perm(out)
    return out


def decode_tile(words, n: int, codebook: int = CB_MUL1, window: int = 16) -> np.ndarray:
    out = np.empty(256, np.uint16)
    lib().exl3o_decode_tile(_u16(words), n, codebook, window, out)
    return out


def reconstruct_inner(trellis, in_f: int, out_f: int, n: int, codebook: int = CB_MUL1,
                      window: int = 16) -> np.ndarray:
    out = np.empty((in_f, out_f), np.uint16)
    lib().exl3o_reconstruct_inner(_u16(trellis).reshape(-1), in_f, out_f, n, codebook, window, out)
    return out


def reconstruct_public(trellis, suh, svh, in_f: int, out_f: int, n: int, codebook: int = CB_MUL1,
                       window: int = 16) -> np.ndarray:
    out = np.empty((in_f, out_f), np.uint16)
    lib().exl3o_reconstruct_public(_u16(trellis).reshape(-1), _u16(suh), _u16(svh), in_f, out_f, n,
                                   codebook, window, out)
    return out


def hadamard128(v, dense: bool = True) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(v, np.float32).copy())
    (lib().exl3o_hadamard128_dense if dense else lib().exl3o_hadamard128_butterfly)(a)
    return a


def prepare(x, suh, dense: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    rows, in_f = x.reshape(-1, x.shape[-1]).shape
    out = np.empty((rows, in_f), np.uint16)
    lib().exl3o_prepare(x.reshape(rows, in_f), _u16(suh), rows, in_f, int(dense), out)
    return out


def inner(trellis, xp, in_f: int, out_f: int, n: int, codebook: int = CB_MUL1,
          window: int = 16) -> np.ndarray:
    xp = _u16(xp).reshape(-1, in_f)
    rows = xp.shape[0]
    out = np.empty((rows, out_f), np.uint16)
    lib().exl3o_inner(_u16(trellis).reshape(-1), xp, rows, in_f, out_f, n, codebook, window, out)
    return out


def finish(z, svh, dense: bool = False) -> np.ndarray:
    z = _u16(z)
    out_f = z.shape[-1]
    z = z.reshape(-1, out_f)
    out = np.empty_like(z)
    lib().exl3o_finish(z, _u16(svh), z.shape[0], out_f, int(dense), out)
    return out


def project(x, trellis, suh, svh, in_f: int, out_f: int, n: int, codebook: int = CB_MUL1,
            window: int = 16, dense: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, np.float32)).reshape(-1, in_f)
    out = np.empty((x.shape[0], out_f), np.uint16)
    lib().exl3o_project(x, _u16(trellis).reshape(-1), _u16(suh), _u16(svh), x.shape[0], in_f, out_f,
                        n, codebook, window, int(dense), out)
    return out


def route_topk(logits, k: int):
    logits = np.ascontiguousarray(np.asarray(logits, np.float32))
    rows, experts = logits.shape
    inds = np.empty((rows, k), np.int32)
    scores = np.empty((rows, k), np.float32)
    lib().exl3o_route_topk(logits, rows, experts, k, inds, scores)
    return inds, scores


def moe_swiglu(x, gate, up, down, inds, scores, hidden: int, inter: int, n: int,
               codebook: int = CB_MUL1, window: int = 16, limit: float = 0.0) -> np.ndarray:
    """gate/up/down: (trellis [E, ...], suh [E, dim], svh [E, dim]) in the pack's tile order."""
    x = np.ascontiguousarray(np.asarray(x, np.float32)).reshape(-1, hidden)
    inds = np.ascontiguousarray(np.asarray(inds, np.int32))
    scores = np.ascontiguousarray(np.asarray(scores, np.float32))
    topk = inds.shape[-1]
    y = np.empty((x.shape[0], hidden), np.float32)
    g, u, d = gate, up, down
    lib().exl3o_moe_swiglu(x, x.shape[0], _u16(g[0]).reshape(-1), _u16(g[1]).reshape(-1), _u16(g[2]).reshape(-1),
                           _u16(u[0]).reshape(-1), _u16(u[1]).reshape(-1), _u16(u[2]).reshape(-1),
                           _u16(d[0]).reshape(-1), _u16(d[1]).reshape(-1), _u16(d[2]).reshape(-1),
                           inds.reshape(-1), scores.reshape(-1), topk, hidden, inter, n, codebook, window,
                           float(limit), y)
    return y


def synth_plane(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint16)
    lib().exl3o_synth_plane(seed, count, out)
    return out


def h2f(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def f2h(x) -> np.ndarray:
    """f32 -> f16 bits, nearest-even (numpy's cast rounds to nearest-even too)."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)
