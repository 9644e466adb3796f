"""A Qwen3-8B-shaped decoder decode step around the EXL3 linears.

36 layers, hidden 4096, 32 query / 8 KV heads of 128,
SwiGLU intermediate 12288, vocab 151936; RMSNorm (with per-head q/k norm),
rotate-half RoPE, f16 attention over an f16 KV cache, EXL3 K=4 mul1 weights for
every linear including lm_head; random-initialised weights and caches (no
checkpoints here).  The reference's model plugin runs the same step on MLX
(turboexl3_qwen38/src/direct/attn.zig:133-141, attn_core.zig, linear.zig:65-85,
model.zig; paths relative to /root/reference/plugins/), its linears through the
quant table this library exports.

Every operation runs in libexl3_mi355x.so: the linears through exl3d_linears
(the EXL3 GEMV with the step's norms, SwiGLU and residual adds fused into its
prepare and finish), embedding and attention through the other exl3d_*
harness entries (include/exl3_decoder.h).  PyTorch only allocates the
buffers and supplies the stream.
"""
from __future__ import annotations

import ctypes
import math
from ctypes import c_float, c_int, c_size_t, c_void_p
from dataclasses import dataclass

from . import exl3 as X

HEAD_DIM = 128


@dataclass
class Qwen3Config:
    layers: int = 36
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    inter: int = 12288
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1e6
    k_bits: int = 4

    @property
    def q_dim(self) -> int:
        return self.heads * HEAD_DIM

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * HEAD_DIM


_DEC_SIGS = {
    "exl3d_embed": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "exl3d_linears": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p, c_float, c_void_p,
                              c_void_p, c_void_p, c_void_p, c_void_p]),
    "exl3d_add_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_float,
                                  c_void_p]),
    "exl3d_qk_norm_rope": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                   c_int, c_int, c_float, c_float, c_void_p, c_void_p, c_void_p,
                                   c_int, c_void_p]),
    "exl3d_attn_scratch_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "exl3d_attn_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                  c_float, c_void_p, c_void_p, c_size_t, c_void_p]),
    "exl3d_attn_decode_rope": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_int, c_int, c_int, c_float, c_float, c_void_p, c_void_p,
                                       c_int, c_float, c_void_p, c_void_p, c_size_t, c_void_p]),
    "exl3d_attn_splits": (c_int, [c_int, c_int, c_int]),
    "exl3d_attn_heads_per_kv": (c_int, []),
    "exl3d_attn_o": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                             c_int, c_float, c_float, c_void_p, c_void_p, c_int, c_float, c_void_p,
                             c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "exl3d_silu_mul": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
}
_dec = None


def dec_lib():
    """libexl3_mi355x.so with the exl3d_* signatures set."""
    global _dec
    if _dec is None:
        L = X.lib()
        for name, (res, args) in _DEC_SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _dec = L
    return _dec


def _ck(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: HIP error {rc}")


def _p(t) -> int:
    return t.data_ptr()


# ------------------------------------------------------------------ ops

def embed(ids, table, h, ssq=None, stream=None):
    B, H = h.shape
    _ck(dec_lib().exl3d_embed(_p(ids), B, _p(table), H, _p(h), _p(ssq) if ssq is not None else None,
                              X.stream_handle(stream)), "embed")


def linears(ws, x, outs=None, norm_w=None, nssq=None, eps=0.0, up=None, res=None, res_ssq=None,
            stream=None):
    """exl3d_linears: the EXL3 linears ws on x with the decode step's fusions
    (RMSNorm of an f32 residual x, SwiGLU with up, residual finish into res)."""
    n = len(ws)
    wp = (ctypes.POINTER(X.Weight) * n)(*[ctypes.pointer(w) for w in ws])
    op = (c_void_p * n)(*[_p(t) for t in outs]) if outs is not None else None
    opt = lambda t: _p(t) if t is not None else None  # noqa: E731
    rc = dec_lib().exl3d_linears(ctypes.cast(wp, c_void_p), n, _p(x), x.shape[0], opt(norm_w),
                                 opt(nssq), eps, opt(up), opt(res), opt(res_ssq),
                                 ctypes.cast(op, c_void_p) if op is not None else None,
                                 X.stream_handle(stream))
    if rc == -1:
        raise RuntimeError("linears: weights or shapes refused")
    _ck(rc, "linears")


def add_rmsnorm(h, add, w, out, eps, stream=None):
    B, H = h.shape
    _ck(dec_lib().exl3d_add_rmsnorm(_p(h), _p(add) if add is not None else None, _p(w), _p(out), B, H,
                                    eps, X.stream_handle(stream)), "add_rmsnorm")


def qk_norm_rope(q, k, v, qn, kn, pos, qout, kcache, vcache, eps, theta, stream=None):
    B = q.shape[0]
    nq, nkv, tmax = q.shape[1] // HEAD_DIM, k.shape[1] // HEAD_DIM, kcache.shape[2]
    _ck(dec_lib().exl3d_qk_norm_rope(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(pos), B, nq, nkv, eps,
                                     theta, _p(qout), _p(kcache), _p(vcache), tmax,
                                     X.stream_handle(stream)), "qk_norm_rope")


def attn_scratch_bytes(B, nq, nkv, tmax) -> int:
    return int(dec_lib().exl3d_attn_scratch_bytes(B, nq, nkv, tmax))


def attn_decode(q, kcache, vcache, pos, out, scratch, stream=None):
    B = q.shape[0]
    nq, nkv, tmax = q.shape[1] // HEAD_DIM, kcache.shape[1], kcache.shape[2]
    _ck(dec_lib().exl3d_attn_decode(_p(q), _p(kcache), _p(vcache), _p(pos), B, nq, nkv, tmax,
                                    1.0 / math.sqrt(HEAD_DIM), _p(out), _p(scratch),
                                    scratch.numel() * scratch.element_size(),
                                    X.stream_handle(stream)), "attn_decode")


def attn_decode_rope(q, k, v, qn, kn, pos, kcache, vcache, out, scratch, eps, theta, stream=None):
    """q/k norm + RoPE + KV append + attention in one launch (raw q, k, v)."""
    B = q.shape[0]
    nq, nkv, tmax = q.shape[1] // HEAD_DIM, kcache.shape[1], kcache.shape[2]
    _ck(dec_lib().exl3d_attn_decode_rope(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(pos), B, nq, nkv,
                                         eps, theta, _p(kcache), _p(vcache), tmax,
                                         1.0 / math.sqrt(HEAD_DIM), _p(out), _p(scratch),
                                         scratch.numel() * scratch.element_size(),
                                         X.stream_handle(stream)), "attn_decode_rope")


def attn_o(q, k, v, qn, kn, pos, kcache, vcache, o, res, res_ssq, att, scratch, eps, theta,
           stream=None):
    """exl3d_attn_o: attn_decode_rope, then res += att @ o^T (residual finish,
    res_ssq its sums of squares per 128 columns); at rows that fit one
    prepare batch o's prepare combines the attention's splits (att is then
    not written)."""
    B = q.shape[0]
    nq, nkv, tmax = q.shape[1] // HEAD_DIM, kcache.shape[1], kcache.shape[2]
    rc = dec_lib().exl3d_attn_o(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(pos), B, nq, nkv, eps, theta,
                                _p(kcache), _p(vcache), tmax, 1.0 / math.sqrt(HEAD_DIM),
                                ctypes.byref(o), _p(res), _p(res_ssq), _p(att), _p(scratch),
                                scratch.numel() * scratch.element_size(), X.stream_handle(stream))
    if rc == -1:
        raise RuntimeError("attn_o: weight or shapes refused")
    _ck(rc, "attn_o")


def silu_mul(g, u, out, stream=None):
    _ck(dec_lib().exl3d_silu_mul(_p(g), _p(u), _p(out), out.numel(), X.stream_handle(stream)),
        "silu_mul")


# ------------------------------------------------------------------ model

def random_linear(torch, i: int, o: int, k_bits: int, gen):
    """An EXL3 linear with uniform-random trellis words, suh +-1 and
    svh f16(+-U[0.5, 1.5] * 0.02) (BASELINE's synthetic packing)."""
    n = 16 * k_bits
    t = torch.randint(-32768, 32768, (i // 16, o // 16, n), dtype=torch.int32, device="cuda",
                      generator=gen).to(torch.int16)
    suh = (torch.randint(0, 2, (i,), device="cuda", generator=gen) * 2 - 1).to(torch.float16)
    sgn = torch.randint(0, 2, (o,), device="cuda", generator=gen) * 2 - 1
    mag = torch.rand(o, device="cuda", generator=gen) + 0.5
    svh = (sgn * mag * 0.02).to(torch.float16)
    return X.Linear(t, suh, svh)


class Qwen3Decoder:
    """Weights, KV caches and step buffers for `batch` sequences whose caches
    hold `ctx` random positions; step() decodes one token per sequence."""

    def __init__(self, cfg: Qwen3Config, batch: int, ctx: int, seed: int = 0, max_new: int = 16):
        import torch
        self.torch = torch
        self.cfg, self.B = cfg, batch
        self.tmax = ctx + max_new
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        H, dev = cfg.hidden, "cuda"

        def norm_w(n):
            return (1.0 + 0.1 * torch.randn(n, device=dev, generator=g)).to(torch.float16)

        self.embed_table = (torch.randn(cfg.vocab, H, device=dev, generator=g)).to(torch.float16)
        self.layers = []
        for _ in range(cfg.layers):
            L = {
                "q": random_linear(torch, H, cfg.q_dim, cfg.k_bits, g),
                "k": random_linear(torch, H, cfg.kv_dim, cfg.k_bits, g),
                "v": random_linear(torch, H, cfg.kv_dim, cfg.k_bits, g),
                "o": random_linear(torch, cfg.q_dim, H, cfg.k_bits, g),
                "gate": random_linear(torch, H, cfg.inter, cfg.k_bits, g),
                "up": random_linear(torch, H, cfg.inter, cfg.k_bits, g),
                "down": random_linear(torch, cfg.inter, H, cfg.k_bits, g),
                "in_norm": norm_w(H), "post_norm": norm_w(H),
                "q_norm": norm_w(HEAD_DIM), "k_norm": norm_w(HEAD_DIM),
                "kc": torch.randn(batch, cfg.kv_heads, self.tmax, HEAD_DIM, device=dev,
                                  generator=g).to(torch.float16),
                "vc": torch.randn(batch, cfg.kv_heads, self.tmax, HEAD_DIM, device=dev,
                                  generator=g).to(torch.float16),
            }
            self.layers.append(L)
        self.final_norm = norm_w(H)
        self.lm_head = random_linear(torch, H, cfg.vocab, cfg.k_bits, g)
        B = batch
        f16 = torch.float16
        self.h = torch.empty(B, H, dtype=torch.float32, device=dev)
        self.ssq = torch.empty(B, H // 128, dtype=torch.float32, device=dev)
        self.g = torch.empty(B, cfg.inter, dtype=f16, device=dev)
        self.u = torch.empty(B, cfg.inter, dtype=f16, device=dev)
        self.q = torch.empty(B, cfg.q_dim, dtype=f16, device=dev)
        self.k = torch.empty(B, cfg.kv_dim, dtype=f16, device=dev)
        self.v = torch.empty(B, cfg.kv_dim, dtype=f16, device=dev)
        self.att = torch.empty(B, cfg.q_dim, dtype=f16, device=dev)
        self.logits = torch.empty(B, cfg.vocab, dtype=f16, device=dev)
        nbytes = attn_scratch_bytes(B, cfg.heads, cfg.kv_heads, self.tmax)
        # zeroed once: the attention leaves its arrival tickets zero
        self.scratch = torch.zeros((nbytes + 3) // 4, dtype=torch.float32, device=dev)
        self.ids = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.full((B,), ctx, dtype=torch.int32, device=dev)

    def weight_bytes(self) -> int:
        """Packed EXL3 bytes one step reads (every linear once)."""
        c = self.cfg
        per = (c.hidden * (c.q_dim + 2 * c.kv_dim) + c.q_dim * c.hidden + 3 * c.hidden * c.inter)
        return (c.layers * per + c.hidden * c.vocab) * c.k_bits // 8

    def kv_bytes(self) -> int:
        """KV cache bytes one step's attention reads (keys 0 .. pos per row)."""
        c = self.cfg
        rows = int(self.pos.sum().item()) + self.B
        return c.layers * 2 * c.kv_heads * HEAD_DIM * 2 * rows

    def step(self, stream=None):
        """One decode step: logits [B, vocab] for tokens self.ids at positions
        self.pos (the caches take their k, v at row pos).

        Five launches a layer: q+k+v with the input RMSNorm of the residual h
        in their prepare; attention with q/k norm, RoPE and the KV append;
        o, whose prepare combines the attention's key splits and whose
        finish adds into h (and leaves h's sums of squares per 128 columns
        for the next norm); gate+up with the post-attention RMSNorm in their
        prepare; down with the SwiGLU in its prepare and its finish adding
        into h.  Rows beyond one prepare batch (batch 16) add the
        attention's combine launch and norm / SwiGLU launches."""
        c = self.cfg
        embed(self.ids, self.embed_table, self.h, self.ssq, stream)
        for L in self.layers:
            linears([L["q"].weight, L["k"].weight, L["v"].weight], self.h,
                    outs=[self.q, self.k, self.v], norm_w=L["in_norm"], nssq=self.ssq, eps=c.eps,
                    stream=stream)
            attn_o(self.q, self.k, self.v, L["q_norm"], L["k_norm"], self.pos, L["kc"], L["vc"],
                   L["o"].weight, self.h, self.ssq, self.att, self.scratch, c.eps, c.theta,
                   stream)
            linears([L["gate"].weight, L["up"].weight], self.h, outs=[self.g, self.u],
                    norm_w=L["post_norm"], nssq=self.ssq, eps=c.eps, stream=stream)
            linears([L["down"].weight], self.g, up=self.u, res=self.h, res_ssq=self.ssq,
                    stream=stream)
        linears([self.lm_head.weight], self.h, outs=[self.logits], norm_w=self.final_norm,
                nssq=self.ssq, eps=c.eps, stream=stream)
        return self.logits
