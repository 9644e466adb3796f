"""Seeded synthetic EXL3 weights and activations shared by the tests and the
benchmark (the shapes and distributions of BASELINE.json's configs): trellis
words uniform u16 (any bitstream decodes validly), suh random +-1, svh =
f16(+-1 * U[0.5, 1.5] * 0.02), activations f16 ~ N(0, 1)."""
from __future__ import annotations

import numpy as np


# 1/sqrt(128) as the kernels and the oracle hold it (f32)
HAD_SCALE = float(np.float32(0.08838834764831845))


def linear(rng: np.random.Generator, in_f: int, out_f: int, n: int, experts: int | None = None):
    lead = () if experts is None else (experts,)
    trellis = rng.integers(0, 65536, lead + (in_f // 16, out_f // 16, n), dtype=np.uint16)
    suh = np.where(rng.random(lead + (in_f,)) < 0.5, -1.0, 1.0).astype(np.float16).view(np.uint16)
    sv = np.where(rng.random(lead + (out_f,)) < 0.5, -1.0, 1.0) * rng.uniform(0.5, 1.5, lead + (out_f,)) * 0.02
    svh = sv.astype(np.float16).view(np.uint16)
    return trellis, suh, svh


def activations(rng: np.random.Generator, rows: int, in_f: int) -> np.ndarray:
    return rng.standard_normal((rows, in_f)).astype(np.float16)


def h2f(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def hadamard(n: int = 128) -> np.ndarray:
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def public_weight(w_inner_f16_bits, suh, svh) -> np.ndarray:
    """W^T = diag(suh) H W_inner H diag(svh) in float64 (the dense effective
    weight, sushi_ds41/src/sushi/exl3/expert_exl3.zig:440-488), with H the
    orthonormal 128-point Hadamard per block."""
    W = h2f(w_inner_f16_bits).astype(np.float64)
    in_f, out_f = W.shape
    H = hadamard(128) / np.sqrt(128.0)
    Wr = np.einsum("bij,bjo->bio", np.broadcast_to(H, (in_f // 128, 128, 128)), W.reshape(in_f // 128, 128, out_f))
    Wr = Wr.reshape(in_f, out_f)
    Wr = (Wr.reshape(in_f, out_f // 128, 128) @ H).reshape(in_f, out_f)
    return h2f(suh).astype(np.float64)[:, None] * Wr * h2f(svh).astype(np.float64)[None, :]


def public_matmul(x, w_inner_f16_bits, suh, svh) -> np.ndarray:
    """x @ W_public in float64 with W_public = diag(suh) H W_inner H diag(svh)
    applied factor by factor (the same product as public_weight, without
    forming the dense matrix): ((x * suh) H) W_inner H * svh, H the
    orthonormal 128-point Hadamard per block (symmetric)."""
    H = hadamard(128) / np.sqrt(128.0)
    x64 = np.asarray(x, np.float64) * h2f(suh).astype(np.float64)
    rows, in_f = x64.shape
    xh = (x64.reshape(rows, in_f // 128, 128) @ H).reshape(rows, in_f)
    z = xh @ h2f(w_inner_f16_bits).astype(np.float64)
    out_f = z.shape[1]
    zh = (z.reshape(rows, out_f // 128, 128) @ H).reshape(rows, out_f)
    return zh * h2f(svh).astype(np.float64)


def row_rel(a, b) -> np.ndarray:
    """Relative Frobenius error of each row of a against b."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b, axis=-1) / np.maximum(np.linalg.norm(b, axis=-1), 1e-30)


def rel_fro(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
