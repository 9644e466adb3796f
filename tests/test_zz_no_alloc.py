"""exl3_matmul_noalloc (the allocation-free matmul) through the C ABI against
exl3_matmul: the same kernels, so the outputs agree bit for bit, on two calls
in a row with the second smaller, at GEMV sizes (split-K slots) and GEMM sizes
(prepared rows and split-K planes); a call beyond the array's 64 MiB is
refused before any launch; captured into a HIP graph (the callers it is
for) its replays equal the eager result; a split-K wait that gives up inside
it is reported by exl3_stream_status, which resets the array; and for a
weight admitted by exl3_resident it keeps the trellis kernels (exl3_matmul
takes the dense GEMM over the held matrix above 16 rows)."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from plugins_amd import exl3 as X  # noqa: E402
from tests import _synth as S  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def linear(rng, in_f, out_f, n=64):
    t, u, v = S.linear(rng, in_f, out_f, n)
    return X.Linear(torch.from_numpy(t.view(np.int16)).to(DEV),
                    torch.from_numpy(u.view(np.float16)).to(DEV),
                    torch.from_numpy(v.view(np.float16)).to(DEV))


def noalloc(lin, x, out, stream=None):
    return X.lib().exl3_matmul_noalloc(ctypes.byref(lin.weight), X.array(x),
                                      X.stream_handle(stream), X.array(out))


def both(lin, x):
    """exl3_matmul's result and exl3_matmul_noalloc's, into separate buffers."""
    want = torch.empty(*x.shape[:-1], lin.out_features, dtype=x.dtype, device=DEV)
    X.check(X.lib().exl3_matmul(ctypes.byref(lin.weight), X.array(x),
                                X.stream_handle(None), ctypes.byref(X.array(want))), "matmul")
    got = torch.full_like(want, float("nan"))
    X.check(noalloc(lin, x, got), "matmul_noalloc")
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("first,second", [
    # GEMV (split-K slots): q/o at 8 rows, then a narrower linear at 1 row
    ((4096, 4096, 8), (512, 256, 1)),
    # GEMM (prepared rows; small grids also split k): 300 rows, then 17
    ((4096, 4096, 300), (2048, 1024, 17)),
    # GEMM then GEMV on the same array
    ((12288, 4096, 64), (4096, 12288, 2)),
])
def test_noalloc_matches_matmul_twice(first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    for in_f, out_f, rows in (first, second):
        lin = linear(rng, in_f, out_f)
        x = torch.from_numpy(S.activations(rng, rows, in_f)).to(DEV)
        got, want = both(lin, x)
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got, want), (in_f, out_f, rows)
    assert X.stream_status(0).is_ok()


def test_noalloc_refuses_beyond_its_array():
    rng = np.random.default_rng(3)
    lin = linear(rng, 12288, 256)
    # 4096 rows x 12288 x 2 bytes of prepared rows = 96 MiB > 56 MiB of staging
    x = torch.zeros(4096, 12288, dtype=torch.float16, device=DEV)
    out = torch.full((4096, 256), 7.0, dtype=torch.float16, device=DEV)
    v = noalloc(lin, x, out)
    assert v.code == X.TOO_LARGE and "no-alloc" in v.reason
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was launched
    # no output buffer given: refused (the entry never allocates one)
    v2 = X.lib().exl3_matmul_noalloc(ctypes.byref(lin.weight), X.array(x[:1]), None, X.Array())
    assert v2.code == X.FAILED and "caller's output" in v2.reason


def test_noalloc_in_a_graph():
    rng = np.random.default_rng(5)
    lin = linear(rng, 4096, 4096)
    x = torch.from_numpy(S.activations(rng, 1, 4096)).to(DEV)
    got, want = both(lin, x)  # the first call on the device ran eagerly
    cap = torch.cuda.Stream()
    out = torch.empty(1, 4096, dtype=torch.float16, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap, capture_error_mode="thread_local"):
        X.check(noalloc(lin, x, out, cap), "matmul_noalloc")
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        # eager work between replays on the same array
        g2, w2 = both(lin, x)
        assert torch.equal(g2, w2)


def test_noalloc_give_up_is_reported_and_reset():
    """The array's status word: a split-K wait that gives up in a no-alloc
    call (forced from the host: the splits other than the last skip their
    stores, the wait's bound is 8 polls) is reported by exl3_stream_status,
    which refills the array's slots; later calls equal exl3_matmul again."""
    rng = np.random.default_rng(17)
    lin = linear(rng, 4096, 4096)  # 8 splits at batch 1
    x = torch.from_numpy(S.activations(rng, 1, 4096)).to(DEV)
    got, want = both(lin, x)
    assert torch.equal(got, want)
    assert X.stream_status(0).is_ok()
    out = torch.empty_like(want)
    try:
        X.lib().exl3_set_splitk_poll_bound(8)
        X.lib().exl3_set_splitk_test_drop(1)
        X.check(noalloc(lin, x, out), "matmul_noalloc")
        v = X.stream_status(0)
    finally:
        X.lib().exl3_set_splitk_test_drop(0)
        X.lib().exl3_set_splitk_poll_bound(-1)
    assert v.code == X.FAILED and "did not arrive" in v.reason
    assert torch.isnan(out.float()).all()
    assert X.stream_status(0).is_ok()
    for rows in (1, 3):
        xr = torch.from_numpy(S.activations(rng, rows, 4096)).to(DEV)
        g2, w2 = both(lin, xr)
        assert torch.equal(g2, w2)
    assert X.stream_status(0).is_ok()


def test_noalloc_keeps_trellis_kernels_for_resident_weights():
    """A weight that holds a matrix through exl3_resident (n = 50, a rate
    without the prefill GEMM): exl3_matmul above 16 rows takes the dense GEMM
    over it; the no-alloc entry keeps the trellis kernels, equal bit for bit
    to exl3_matmul of the weight before it was admitted, and within the
    matmul bar of the resident result.  At a GEMM rate (n = 64) nothing is
    held and the two entries stay equal bit for bit."""
    rng = np.random.default_rng(23)
    lin = linear(rng, 1024, 512, n=50)
    lin64 = linear(rng, 1024, 512, n=64)
    x = torch.from_numpy(S.activations(rng, 64, 1024)).to(DEV)
    got0, want0 = both(lin, x)
    assert torch.equal(got0, want0)
    X.resident([lin.weight, lin64.weight])
    try:
        got, want_res = both(lin, x)
        assert torch.equal(got, want0)  # trellis kernels, as before admission
        g64, w64 = got.double(), want_res.double()
        assert float(torch.linalg.norm(g64 - w64) / torch.linalg.norm(w64)) < 1e-3
        a, b = both(lin64, x)
        assert torch.equal(a, b)
    finally:
        X.resident([])
