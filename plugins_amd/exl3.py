"""Python host mirror of the EXL3 quant-plugin boundary (include/exl3_mi355x.h).

The reference's host code is Zig calling the quant plugin table through its
C ABI (turboexl3_qwen38/overlay/mlx_serve/abi/quant.zig:24-108, filled by
turboexl3_ds41/plugin.zig:28-43; paths relative to /root/reference/plugins/).
This module binds the same entries of libexl3_mi355x.so with ctypes, under
the reference's names (claims, validate, bill, open, close, load_tensor,
load_bank, release, matmul, moe, swiglu) and with the same meaning: each
returns a Verdict (code, why) and refuses by name instead of falling back.

PyTorch supplies device memory and the HIP stream handle only; every
computation runs in the library's HIP kernels.  If the library is not built,
loading fails loudly (no CPU path exists here).
"""
from __future__ import annotations

import ctypes
import json
import os
from ctypes import (CFUNCTYPE, POINTER, Structure, c_bool, c_char_p, c_int, c_int32, c_int64,
                    c_size_t, c_uint32, c_uint64, c_void_p)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libexl3_mi355x.so")

# Verdict codes (kit Verdict: ok, unsupported, failed, too_large)
OK, UNSUPPORTED, FAILED, TOO_LARGE = 0, 1, 2, 3
# Claim values
CLAIM_NO, CLAIM_BY_MODE, CLAIM_BY_MARKER = 0, 1, 2
# mlx-c dtype numbering
DT_BOOL, DT_U8, DT_U16, DT_U32, DT_U64, DT_I8, DT_I16, DT_I32, DT_I64 = range(9)
DT_F16, DT_F32, DT_F64, DT_BF16 = 9, 10, 11, 12
MAX_DIMS = 4


class Str(Structure):
    _fields_ = [("ptr", c_char_p), ("len", c_size_t)]

    @classmethod
    def of(cls, s) -> "Str":
        b = s.encode() if isinstance(s, str) else (s or b"")
        return cls(b, len(b))


class Verdict(Structure):
    _fields_ = [("code", c_int32), ("why", c_char_p)]

    def is_ok(self) -> bool:
        return self.code == OK

    @property
    def reason(self) -> str:
        return (self.why or b"").decode()

    def __repr__(self) -> str:
        return f"Verdict(code={self.code}, why={self.reason!r})"


class Array(Structure):
    _fields_ = [("data", c_void_p), ("dtype", c_int32), ("ndim", c_int32),
                ("shape", c_int64 * MAX_DIMS), ("owned", c_uint32), ("_pad", c_uint32)]

    def dims(self) -> tuple:
        return tuple(self.shape[i] for i in range(self.ndim))


class Weight(Structure):
    _fields_ = [("w", Array), ("scales", Array), ("biases", Array), ("side", Array),
                ("flags", c_uint32), ("_pad", c_uint32), ("priv", c_void_p)]


class HostTensor(Structure):
    _fields_ = [("data", c_void_p), ("dtype", c_int32), ("ndim", c_int32),
                ("shape", c_int64 * MAX_DIMS)]


TENSOR_FN = CFUNCTYPE(c_int, c_void_p, Str, POINTER(HostTensor))
FILE_BYTES_FN = CFUNCTYPE(c_uint64, c_void_p, Str)


class Source(Structure):
    _fields_ = [("self", c_void_p), ("tensor", TENSOR_FN)]


class PackDir(Structure):
    _fields_ = [("self", c_void_p), ("file_bytes", FILE_BYTES_FN)]


class LoadCtx(Structure):
    _fields_ = [("size", c_uint32), ("device", c_int32), ("block_json", Str),
                ("config_json", Str), ("source", POINTER(Source)), ("dir", POINTER(PackDir)),
                ("stream", c_void_p), ("state", c_void_p)]


class SwigluOpts(Structure):
    _fields_ = [("size", c_uint32), ("limit", c_int32), ("verify_rows", c_bool)]


class ArraySpan(Structure):
    _fields_ = [("ptr", POINTER(Array)), ("len", c_size_t)]


class U32Span(Structure):
    _fields_ = [("ptr", POINTER(c_uint32)), ("len", c_size_t)]


class U8Span(Structure):
    _fields_ = [("ptr", POINTER(ctypes.c_uint8)), ("len", c_size_t)]


class WeightSpan(Structure):
    _fields_ = [("ptr", POINTER(Weight)), ("len", c_size_t)]


class LinearParts(Structure):
    """`LinearParts` (quant.zig:111-128), the split entries' options."""
    _fields_ = [("size", c_uint32), ("dtype", c_int32), ("side", c_void_p), ("inner", c_bool),
                ("prepared", c_bool), ("held", Array), ("rows", U32Span), ("parts", ArraySpan)]


class SharedSwiglu(Structure):
    """`SharedSwiglu` (quant.zig:183-197): the gated shared expert's options."""
    _fields_ = [("size", c_uint32), ("gate", POINTER(Weight)), ("up", POINTER(Weight)),
                ("down", POINTER(Weight)), ("sigtab", Array), ("logit", Array),
                ("gate_vec", Array), ("logits", Array), ("k", c_uint32)]


# The QuantTable's entries in the reference's order (quant.zig:24-107).
TABLE_ENTRIES = ("claims", "validate", "bill", "open", "close", "load_tensor", "load_bank",
                 "release", "matmul", "moe", "register_kernels", "swiglu", "linear_split",
                 "linear_finish", "linear_prepared", "linear_pieces", "linear_piece", "attn_in",
                 "attn_prep", "linear_prepared_idx", "gated_out", "merged_gated_out", "q_planes",
                 "indexer", "swiglu_shared", "resident", "resident_pending", "unrotate",
                 "linear_joined")


class QuantTable(Structure):
    _fields_ = [("size", c_uint32), ("version", c_uint32), ("name", Str)] + \
        [(e, c_void_p) for e in TABLE_ENTRIES]


# Every symbol include/exl3_mi355x.h declares, with its ctypes signature.
SIGNATURES = {
    "exl3_claims": (c_int32, [Str, Str]),
    "exl3_claims_qwen38": (c_int32, [Str, Str]),
    "exl3_validate": (Verdict, [Str, Str, POINTER(PackDir)]),
    "exl3_bill": (c_uint64, [Str, Str, c_uint64]),
    "exl3_open": (Verdict, [POINTER(LoadCtx)]),
    "exl3_close": (None, [POINTER(LoadCtx)]),
    "exl3_load_tensor": (Verdict, [POINTER(LoadCtx), Str, c_uint32, POINTER(Weight)]),
    "exl3_load_bank": (Verdict, [POINTER(LoadCtx), Str, c_uint32, POINTER(Weight)]),
    "exl3_release": (None, [POINTER(Weight)]),
    "exl3_matmul": (Verdict, [POINTER(Weight), Array, c_void_p, POINTER(Array)]),
    "exl3_matmul_shared": (Verdict, [POINTER(POINTER(Weight)), c_uint32, Array, c_void_p, POINTER(Array)]),
    "exl3_moe": (Verdict, [POINTER(Weight), Array, Array, Array, c_bool, c_void_p, POINTER(Array)]),
    "exl3_swiglu": (Verdict, [POINTER(Weight), POINTER(Weight), POINTER(Weight), Array, Array, Array,
                              POINTER(SwigluOpts), c_void_p, POINTER(Array)]),
    "exl3_quant_table_get": (POINTER(QuantTable), []),
    "exl3_quant_table_qwen38_get": (POINTER(QuantTable), []),
    "exl3_array_free": (None, [POINTER(Array)]),
    "exl3_weight_wrap": (Verdict, [Array, Array, Array, Str, c_int32, POINTER(Weight)]),
    "exl3_decode_matrix": (Verdict, [POINTER(Weight), c_int32, Array, c_void_p]),
    "exl3_prepare": (Verdict, [POINTER(Weight), Array, Array, c_void_p]),
    "exl3_finish": (Verdict, [POINTER(Weight), Array, Array, c_void_p]),
    "exl3_inner": (Verdict, [POINTER(Weight), Array, Array, c_void_p]),
    "exl3_version": (c_char_p, []),
    "exl3_safetensors_open": (c_void_p, [POINTER(c_char_p), c_uint32, POINTER(Verdict)]),
    "exl3_safetensors_close": (None, [c_void_p]),
    "exl3_pack_dir_open": (c_void_p, [c_char_p]),
    "exl3_pack_dir_close": (None, [c_void_p]),
    "exl3_matmul_path": (c_char_p, [POINTER(Weight), c_int64]),
    "exl3_swiglu_path": (c_char_p, [POINTER(Weight), POINTER(Weight), POINTER(Weight), c_int64, c_int32,
                                    c_bool]),
    "exl3_scratch_release": (Verdict, [c_int32, c_void_p]),
    "exl3_stream_status": (Verdict, [c_int32, c_void_p]),
    "exl3_set_splitk_poll_bound": (None, [c_int32]),
    "exl3_set_splitk_test_drop": (None, [c_int32]),
    "exl3_self_check": (Verdict, [c_int32]),
    "exl3_set_self_check_fault": (None, [c_char_p]),
    "exl3_matmul_noalloc": (Verdict, [POINTER(Weight), Array, c_void_p, Array]),
    "exl3_linear_split": (Verdict, [POINTER(Weight), Array, POINTER(LinearParts), c_void_p,
                                    POINTER(Array)]),
    "exl3_linear_finish": (Verdict, [POINTER(Weight), POINTER(LinearParts), c_void_p, POINTER(Array)]),
    "exl3_linear_prepared": (Verdict, [POINTER(Weight), Array, POINTER(LinearParts), c_void_p,
                                       POINTER(Array)]),
    "exl3_linear_pieces": (Verdict, [POINTER(Weight), POINTER(LinearParts), c_void_p, POINTER(Array)]),
    "exl3_linear_piece": (Verdict, [POINTER(Weight), Array, POINTER(LinearParts), c_void_p,
                                    POINTER(Array)]),
    "exl3_swiglu_shared": (Verdict, [POINTER(Weight), POINTER(Weight), POINTER(Weight), Array, Array,
                                     Array, POINTER(SharedSwiglu), c_void_p, POINTER(Array)]),
    "exl3_resident": (Verdict, [WeightSpan, c_uint64, c_void_p, POINTER(c_uint64)]),
    "exl3_resident_pending": (c_uint64, []),
    "exl3_unrotate": (Verdict, [WeightSpan, U8Span, c_int32, c_void_p, POINTER(c_bool)]),
    "exl3_linear_joined": (Verdict, [WeightSpan, Array, c_void_p, POINTER(Array)]),
}

_lib = None


class Exl3Error(RuntimeError):
    def __init__(self, verdict: Verdict, what: str = ""):
        self.code = verdict.code
        self.why = verdict.reason
        super().__init__(f"{what}: {self.why} (code {self.code})" if what else self.why)


def lib():
    """The loaded libexl3_mi355x.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m plugins_amd.build` "
                               "(the EXL3 path has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(v: Verdict, what: str = "") -> None:
    if v.code != OK:
        raise Exl3Error(v, what)


# ------------------------------------------------------------ torch glue

def _torch():
    import torch
    return torch


def dtype_of(t) -> int:
    torch = _torch()
    table = {torch.float16: DT_F16, torch.bfloat16: DT_BF16, torch.float32: DT_F32,
             torch.int16: DT_I16, torch.int32: DT_I32, torch.uint8: DT_U8, torch.int64: DT_I64,
             torch.float64: DT_F64, torch.bool: DT_BOOL}
    for name, code in (("uint16", DT_U16), ("uint32", DT_U32)):
        if hasattr(torch, name):
            table[getattr(torch, name)] = code
    if t.dtype not in table:
        raise TypeError(f"no ABI dtype for {t.dtype}")
    return table[t.dtype]


def array(t, dtype: int | None = None) -> Array:
    """An Array descriptor over a contiguous device tensor (None: empty)."""
    a = Array()
    if t is None:
        return a
    if not t.is_contiguous():
        raise ValueError("the ABI takes dense row-major arrays")
    if t.dim() > MAX_DIMS:
        raise ValueError("too many dims")
    a.data = t.data_ptr()
    a.dtype = dtype_of(t) if dtype is None else dtype
    a.ndim = t.dim()
    for i, s in enumerate(t.shape):
        a.shape[i] = s
    return a


def stream_handle(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


# --------------------------------------------------------- table entries

def claims(block_json: str, config_json: str = "{}") -> int:
    """turboexl3_ds41's claim rule (the default table's)."""
    return int(lib().exl3_claims(Str.of(block_json), Str.of(config_json)))


def claims_qwen38(block_json: str, config_json: str = "{}") -> int:
    """turboexl3_qwen38's claim rule (the qwen38 table's)."""
    return int(lib().exl3_claims_qwen38(Str.of(block_json), Str.of(config_json)))


def validate(block_json: str, config_json: str = "{}", dir: PackDir | None = None) -> Verdict:
    return lib().exl3_validate(Str.of(block_json), Str.of(config_json),
                               ctypes.byref(dir) if dir is not None else None)


def bill(block_json: str, model_dir: str, stored: int) -> int:
    return int(lib().exl3_bill(Str.of(block_json), Str.of(model_dir), stored))


def quant_table(qwen38: bool = False) -> QuantTable:
    """The exported table: ds41's claim rule, or with qwen38 the table under
    its own name that claims as turboexl3_qwen38 does."""
    get = lib().exl3_quant_table_qwen38_get if qwen38 else lib().exl3_quant_table_get
    return get().contents


def version() -> str:
    return lib().exl3_version().decode()


class DictSource:
    """A weight source over host arrays (numpy) keyed by tensor name: the
    reference's `Source` (`ctx.source.tensor(name)`) for tests and tools."""

    _DT = {"float16": DT_F16, "int16": DT_I16, "uint16": DT_U16, "float32": DT_F32,
           "bfloat16": DT_BF16, "int32": DT_I32, "uint32": DT_U32}

    def __init__(self, tensors: dict):
        import numpy as np
        self.tensors = {k: np.ascontiguousarray(v) for k, v in tensors.items()}
        self._fn = TENSOR_FN(self._lookup)
        self.struct = Source(None, self._fn)

    def _lookup(self, _self, name: Str, out) -> int:
        key = ctypes.string_at(name.ptr, name.len).decode()
        a = self.tensors.get(key)
        if a is None:
            return 0
        t = out.contents
        t.data = a.ctypes.data
        t.dtype = self._DT[str(a.dtype)]
        t.ndim = a.ndim
        for i, s in enumerate(a.shape):
            t.shape[i] = s
        return 1


class SafetensorsSource:
    """A weight source over a pack's safetensors files (exl3_safetensors_open):
    the library maps the files and hands out host views; the same interface as
    DictSource for Loader."""

    def __init__(self, paths):
        if isinstance(paths, (str, os.PathLike)):
            paths = [paths]
        enc = [os.fsencode(p) for p in paths]
        arr = (c_char_p * len(enc))(*enc)
        self.verdict = Verdict()
        self.handle = lib().exl3_safetensors_open(arr, len(enc), ctypes.byref(self.verdict))
        if not self.handle:
            raise OSError(f"exl3_safetensors_open: {self.verdict}")
        self.struct = ctypes.cast(self.handle, POINTER(Source)).contents

    def tensor(self, name: str):
        """The host view of `name` (dtype code, shape, data address), or None."""
        t = HostTensor()
        if not self.struct.tensor(self.struct.self, Str.of(name), ctypes.byref(t)):
            return None
        return t.dtype, tuple(t.shape[i] for i in range(t.ndim)), t.data

    def close(self) -> None:
        if self.handle:
            lib().exl3_safetensors_close(self.handle)
            self.handle = None
            self.struct = None


class PackDirectory:
    """A PackDir over a directory (exl3_pack_dir_open): file_bytes(name)."""

    def __init__(self, root):
        self.handle = lib().exl3_pack_dir_open(os.fsencode(root))
        if not self.handle:
            raise OSError(f"not a directory: {root}")
        self.struct = ctypes.cast(self.handle, POINTER(PackDir)).contents

    def file_bytes(self, name: str) -> int:
        return int(self.struct.file_bytes(self.struct.self, Str.of(name)))

    def close(self) -> None:
        if self.handle:
            lib().exl3_pack_dir_close(self.handle)
            self.handle = None
            self.struct = None


class Loader:
    """open / load_tensor / load_bank / close over a weight source
    (turboexl3_ds41/plugin.zig:52-185)."""

    def __init__(self, block_json: str, source: DictSource, config_json: str = "{}", device: int = 0,
                 stream=None):
        self.source = source
        self._keep = (Str.of(block_json), Str.of(config_json))
        self.ctx = LoadCtx()
        self.ctx.size = ctypes.sizeof(LoadCtx)
        self.ctx.device = device
        self.ctx.block_json = self._keep[0]
        self.ctx.config_json = self._keep[1]
        self.ctx.source = ctypes.pointer(source.struct)
        self.ctx.stream = stream_handle(stream) if stream is not None else None
        self.opened = lib().exl3_open(ctypes.byref(self.ctx))

    def load_tensor(self, name: str, in_dim: int = 0) -> tuple[Verdict, Weight]:
        w = Weight()
        v = lib().exl3_load_tensor(ctypes.byref(self.ctx), Str.of(name), in_dim, ctypes.byref(w))
        return v, w

    def load_bank(self, name: str, in_dim: int = 0) -> tuple[Verdict, Weight]:
        w = Weight()
        v = lib().exl3_load_bank(ctypes.byref(self.ctx), Str.of(name), in_dim, ctypes.byref(w))
        return v, w

    def close(self) -> None:
        lib().exl3_close(ctypes.byref(self.ctx))


def release(w: Weight) -> None:
    lib().exl3_release(ctypes.byref(w))


# The shipped codebook tables a spec1 / std1 / pair1 block names, with the
# digests it must carry (sushi_ds41/src/sushi/exl3/codebook_tables.zig:99-104).
TABLE_DIGESTS = {"pair1-w16-v1": "c089b4eb", "spec1-w15": "37f72431", "spec1-w16": "753ffa03",
                 "std1": "c5dba171"}


def quant_block(codebook: str = "mul1", window: int = 16, table: str | None = None,
                digest: str | None = None) -> str:
    """An EXL3 quantization block; the table codebooks name their table (std1
    and pair1 default to their one table) and its digest (default: the
    shipped table's)."""
    b = {"format": "exl3", "codebook": codebook, "window": window}
    if table is None:
        table = {"std1": "std1", "pair1": "pair1-w16-v1"}.get(codebook)
    if table is not None:
        b["codebook_table"] = table
        b["codebook_digest"] = digest if digest is not None else TABLE_DIGESTS.get(table, "")
    return json.dumps(b)


def wrap(trellis, suh, svh, codebook: str = "mul1", window: int = 16, device: int = 0,
         table: str | None = None, digest: str | None = None) -> Weight:
    """A Weight over device tensors (the library borrows their memory).  The
    returned Weight holds references to the three tensors, so the memory it
    points at stays allocated for as long as the Weight object lives, even
    when the caller passed temporaries (a freed block could otherwise be
    handed to the next allocation, or returned to the driver by
    torch.cuda.empty_cache(), which torch.cuda.graph() calls on entry).
    spec1 / std1 / pair1 decode with the row of `table` for the weight's rate."""
    w = Weight()
    block = quant_block(codebook, window, table, digest)
    tdt = DT_U16 if str(trellis.dtype) in ("torch.int16", "torch.uint16") else dtype_of(trellis)
    check(lib().exl3_weight_wrap(array(trellis, tdt), array(suh), array(svh), Str.of(block), device,
                                 ctypes.byref(w)), "weight_wrap")
    w._keep = (trellis, suh, svh)
    return w


def _out_tensor(like, last: int, dtype=None):
    torch = _torch()
    return torch.empty(*like.shape[:-1], last, dtype=dtype or like.dtype, device=like.device)


def matmul(w: Weight, x, out=None, stream=None):
    """x @ W^T through the library (QuantTable.matmul).  `out` is written if
    given, else allocated with torch (the library never owns it here)."""
    out_f = w.biases.shape[w.biases.ndim - 1]
    y = out if out is not None else _out_tensor(x, out_f)
    a = array(y)
    check(lib().exl3_matmul(ctypes.byref(w), array(x), stream_handle(stream), ctypes.byref(a)),
          "matmul")
    return y


def matmul_shared(ws, x, outs=None, stream=None):
    """Several linears reading the same rows in one launch (outs[i] = x @ W_i^T)."""
    n = len(ws)
    ptrs = (POINTER(Weight) * n)(*[ctypes.pointer(w) for w in ws])
    ys = outs if outs is not None else [_out_tensor(x, w.biases.shape[w.biases.ndim - 1]) for w in ws]
    arr = (Array * n)(*[array(y) for y in ys])
    check(lib().exl3_matmul_shared(ptrs, n, array(x), stream_handle(stream), arr), "matmul_shared")
    return ys


def moe(bank: Weight, x, lhs=None, rhs=None, sorted_: bool = False, stream=None) -> Verdict:
    a = Array()
    return lib().exl3_moe(ctypes.byref(bank), array(x), array(lhs), array(rhs), sorted_,
                          stream_handle(stream), ctypes.byref(a))


def swiglu(gate: Weight, up: Weight, down: Weight, x, inds=None, scores=None, limit: int = 0,
           verify_rows: bool = False, out=None, stream=None):
    """Routed (or, with inds None, dense) SwiGLU experts (QuantTable.swiglu)."""
    y = out if out is not None else _torch().empty_like(x)
    opts = SwigluOpts(ctypes.sizeof(SwigluOpts), int(limit), bool(verify_rows))
    a = array(y)
    check(lib().exl3_swiglu(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down), array(x),
                            array(inds), array(scores), ctypes.byref(opts), stream_handle(stream),
                            ctypes.byref(a)), "swiglu")
    return y


def swiglu_shared(gate: Weight, up: Weight, down: Weight, x, shared, inds=None, scores=None,
                  logit=None, gate_vec=None, logits=None, k: int = 0, out=None, stream=None):
    """QuantTable.swiglu_shared: routed experts plus sigmoid(logit) * the shared
    expert (shared = (gate, up, down) Weights), in the routed launches.  Routes
    from inds/scores, or from the router's `logits` with `k`; the logit given
    per row or computed from `gate_vec`."""
    y = out if out is not None else _torch().empty_like(x)
    o = SharedSwiglu()
    o.size = ctypes.sizeof(SharedSwiglu)
    o.gate, o.up, o.down = (ctypes.pointer(w) for w in shared)
    o.logit = array(logit)
    o.gate_vec = array(gate_vec)
    o.logits = array(logits)
    o.k = k
    a = array(y)
    check(lib().exl3_swiglu_shared(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down),
                                   array(x), array(inds), array(scores), ctypes.byref(o),
                                   stream_handle(stream), ctypes.byref(a)), "swiglu_shared")
    return y


def decode_matrix(w: Weight, expert: int = 0, stream=None):
    torch = _torch()
    in_f = w.scales.shape[w.scales.ndim - 1]
    out_f = w.biases.shape[w.biases.ndim - 1]
    dev = torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(in_f, out_f, dtype=torch.float16, device=dev)
    check(lib().exl3_decode_matrix(ctypes.byref(w), expert, array(out), stream_handle(stream)),
          "decode_matrix")
    return out


def prepare(w: Weight, x, stream=None):
    torch = _torch()
    xp = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    check(lib().exl3_prepare(ctypes.byref(w), array(x), array(xp), stream_handle(stream)), "prepare")
    return xp


def finish(w: Weight, z, dtype=None, stream=None):
    torch = _torch()
    y = torch.empty(z.shape, dtype=dtype or torch.float16, device=z.device)
    check(lib().exl3_finish(ctypes.byref(w), array(z), array(y), stream_handle(stream)), "finish")
    return y


def inner(w: Weight, xp, stream=None):
    torch = _torch()
    out_f = w.biases.shape[w.biases.ndim - 1]
    z = torch.empty(*xp.shape[:-1], out_f, dtype=torch.float16, device=xp.device)
    check(lib().exl3_inner(ctypes.byref(w), array(xp), array(z), stream_handle(stream)), "inner")
    return z


_hip = None


def _hip_runtime():
    """The HIP runtime the library itself links (for copying its arrays)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpyAsync.argtypes = [c_void_p, c_void_p, c_size_t, c_int32, c_void_p]
        _hip.hipMemcpyAsync.restype = c_int32
    return _hip


def take(a: Array, stream=None):
    """A torch tensor holding the contents of an array the library allocated
    (owned = 1); the library's array is freed.  The copy is ordered on
    `stream` (the stream the library's work was recorded on)."""
    torch = _torch()
    dts = {DT_F16: torch.float16, DT_BF16: torch.bfloat16, DT_F32: torch.float32}
    t = torch.empty([a.shape[i] for i in range(a.ndim)], dtype=dts[a.dtype],
                    device=torch.device("cuda", torch.cuda.current_device()))
    st = stream if stream is not None else torch.cuda.current_stream()
    rc = _hip_runtime().hipMemcpyAsync(t.data_ptr(), a.data, t.numel() * t.element_size(), 3,
                                       st.cuda_stream)
    st.synchronize()
    lib().exl3_array_free(ctypes.byref(a))
    if rc != 0:
        raise RuntimeError(f"hipMemcpyAsync failed ({rc})")
    return t


def linear_parts(dtype: int = DT_F16, side=None, inner: bool = False, prepared: bool = False,
                 held: Array | None = None, rows=None, parts=None) -> LinearParts:
    o = LinearParts()
    o.size = ctypes.sizeof(LinearParts)
    o.dtype = dtype
    o.side = side.cuda_stream if side is not None else None
    o.inner = inner
    o.prepared = prepared
    if held is not None:
        o.held = held
    if rows is not None:
        buf = (c_uint32 * len(rows))(*rows)
        o.rows = U32Span(buf, len(rows))
        o._rows = buf
    if parts is not None:
        arr = (Array * len(parts))(*[array(z) for z in parts])
        o.parts = ArraySpan(arr, len(parts))
        o._parts = arr
    return o


def linear_split(w: Weight, x, inner: bool = False, side=None, stream=None):
    """QuantTable.linear_split: y (or, inner, z f16) with the work after x's
    prepare on `side`; returns a torch copy of the library's output."""
    o = linear_parts(dtype_of(x), side=side, inner=inner)
    a = Array()
    check(lib().exl3_linear_split(ctypes.byref(w), array(x), ctypes.byref(o),
                                  stream_handle(stream), ctypes.byref(a)), "linear_split")
    return take(a, side if side is not None else stream)


def linear_finish(w: Weight, zs, dtype: int = DT_F16, stream=None):
    """QuantTable.linear_finish over inner products zs (row order)."""
    o = linear_parts(dtype, parts=list(zs))
    a = Array()
    check(lib().exl3_linear_finish(ctypes.byref(w), ctypes.byref(o), stream_handle(stream),
                                   ctypes.byref(a)), "linear_finish")
    return take(a, stream)


def linear_prepared(w: Weight, xp, dtype: int = DT_F16, stream=None):
    """QuantTable.linear_prepared: y of rows already prepared (f16)."""
    o = linear_parts(dtype)
    a = Array()
    check(lib().exl3_linear_prepared(ctypes.byref(w), array(xp), ctypes.byref(o),
                                     stream_handle(stream), ctypes.byref(a)), "linear_prepared")
    return take(a, stream)


def linear_pieces(w: Weight, rows, dtype: int = DT_F16, stream=None) -> tuple[Verdict, Array]:
    o = linear_parts(dtype, rows=list(rows))
    a = Array()
    v = lib().exl3_linear_pieces(ctypes.byref(w), ctypes.byref(o), stream_handle(stream),
                                 ctypes.byref(a))
    return v, a


def linear_piece(w: Weight, x, held: Array, prepared: bool = False, stream=None):
    o = linear_parts(DT_F16, prepared=prepared, held=held)
    a = Array()
    check(lib().exl3_linear_piece(ctypes.byref(w), array(x), ctypes.byref(o),
                                  stream_handle(stream), ctypes.byref(a)), "linear_piece")
    return take(a, stream)


def _weight_span(ws) -> tuple[WeightSpan, object]:
    arr = (Weight * len(ws))(*ws)
    return WeightSpan(arr, len(ws)), arr


def resident(ws, room: int = 0, stream=None) -> int:
    """QuantTable.resident: admits the weights' decoded matrices (held from each
    one's first prefill-width matmul on); returns the bytes they take.  An
    empty list drops every kept matrix."""
    span, keep = _weight_span(list(ws))
    n = c_uint64(0)
    check(lib().exl3_resident(span, room, stream_handle(stream), ctypes.byref(n)), "resident")
    del keep
    return n.value


def resident_pending() -> int:
    """QuantTable.resident_pending: bytes admitted and not held yet."""
    return lib().exl3_resident_pending()


def unrotate(ws, sizes, act: int = DT_F16, stream=None) -> list[bool]:
    """QuantTable.unrotate: each group of sizes[g] weights (one input) joined
    as one public matrix in `act`; returns took[g]."""
    span, keep = _weight_span(list(ws))
    sz = (ctypes.c_uint8 * len(sizes))(*sizes)
    took = (c_bool * max(1, len(sizes)))()
    check(lib().exl3_unrotate(span, U8Span(sz, len(sizes)), act, stream_handle(stream), took),
          "unrotate")
    del keep
    return [bool(took[i]) for i in range(len(sizes))]


def linear_joined(ws, x, stream=None):
    """QuantTable.linear_joined: x times an un-rotated group's joined matrix."""
    span, keep = _weight_span(list(ws))
    a = Array()
    check(lib().exl3_linear_joined(span, array(x), stream_handle(stream), ctypes.byref(a)),
          "linear_joined")
    del keep
    return take(a, stream)


def matmul_path(w: Weight, rows: int) -> str:
    return lib().exl3_matmul_path(ctypes.byref(w), rows).decode()


def swiglu_path(gate: Weight, up: Weight, down: Weight, rows: int, topk: int = 0,
                verify_rows: bool = False) -> str:
    """The kernel path a swiglu of `rows` rows takes (exl3_swiglu_path)."""
    return lib().exl3_swiglu_path(ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down), rows,
                                  topk, bool(verify_rows)).decode()


class Linear:
    """One EXL3 linear on device tensors: trellis [in/16, out/16, n] (int16 or
    uint16 bits), suh f16 [in], svh f16 [out].  Keeps the tensors alive for the
    borrowed Weight."""

    def __init__(self, trellis, suh, svh, codebook: str = "mul1", window: int = 16,
                 table: str | None = None):
        self.tensors = (trellis, suh, svh)
        self.weight = wrap(trellis, suh, svh, codebook, window, trellis.device.index or 0, table)
        self.in_features = suh.shape[-1]
        self.out_features = svh.shape[-1]

    def __call__(self, x, out=None, stream=None):
        return matmul(self.weight, x, out=out, stream=stream)

    def __del__(self):
        try:
            if self.weight.priv:
                release(self.weight)
        except Exception:
            pass


def scratch_release(device: int = 0, stream=None) -> None:
    """Frees the library's scratch for (device, stream) (exl3_scratch_release):
    call once no graph captured on the stream will be replayed again."""
    check(lib().exl3_scratch_release(device, stream_handle(stream)), "scratch_release")


def stream_status(device: int = 0, stream=None) -> Verdict:
    """exl3_stream_status: synchronizes the stream and reports (FAILED) whether a
    split-K wait gave up since the last check; resets the slots if so."""
    return lib().exl3_stream_status(device, stream_handle(stream))
