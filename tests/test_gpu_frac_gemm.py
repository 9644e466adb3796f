"""The prefill GEMM at the half-integer rates n = 24 and 40 (K 1.5, 2.5:
turboexl3_ds41/src/bank/frac.zig:1-21, where the reference's turboexl3 runs
such tiles through its prefill GEMM as it runs integer ones), through the C
ABI: every row against the float64 product with the decoded weight (the
oracle's decode, bit-exact to the reference's), the oracle's projection for
the matmul bar, and the GEMV on the same rows (paths relative to
/root/reference/plugins/)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from plugins_amd import exl3 as X  # noqa: E402
from tests import _synth as S  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV)


def dev_f16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16) if a.dtype == np.uint16
                            else np.ascontiguousarray(a, np.float16)).to(DEV)


FORMS = {"mul1": ("mul1", None, O.CB_MUL1), "mcg": ("mcg", None, O.CB_MCG),
         "spec1-w15": ("spec1", "spec1-w15", O.spec1(O.TAB_SPEC1_W15)),
         "pair1": ("pair1", "pair1-w16-v1", O.CB_PAIR1)}


@pytest.mark.parametrize("rows", [17, 256, 300, 2048])
@pytest.mark.parametrize("n", [24, 40])
@pytest.mark.parametrize("form", ["mul1", "mcg", "spec1-w15", "pair1"])
def test_frac_gemm_every_row(form, n, rows):
    cb, table, ocb = FORMS[form]
    rng = np.random.default_rng(7000 + n + rows)
    in_f, out_f = 512, 384
    t, u, v = S.linear(rng, in_f, out_f, n)
    lin = X.Linear(dev_u16(t), dev_f16(u), dev_f16(v), cb, 16, table)
    assert X.matmul_path(lin.weight, rows) == "gemm"
    x = S.activations(rng, rows, in_f)
    y = lin(dev_f16(x)).float().cpu().numpy()
    w_inner = O.reconstruct_inner(t, in_f, out_f, n, ocb)
    want = S.public_matmul(x.astype(np.float64), w_inner, u, v)
    assert S.rel_fro(y, want) < 1e-3, S.rel_fro(y, want)
    assert (S.row_rel(y, want) < 3e-3).all(), S.row_rel(y, want).max()
    if rows <= 300:
        yo = S.h2f(O.project(x.astype(np.float32), t, u, v, in_f, out_f, n, ocb))
        assert S.rel_fro(y, yo) < 1e-3


@pytest.mark.parametrize("n", [24, 40])
def test_frac_gemm_agrees_with_the_gemv_rows(n):
    rng = np.random.default_rng(7100 + n)
    in_f, out_f, rows = 1024, 512, 48
    t, u, v = S.linear(rng, in_f, out_f, n)
    lin = X.Linear(dev_u16(t), dev_f16(u), dev_f16(v))
    x = dev_f16(S.activations(rng, rows, in_f))
    y = lin(x).float()
    # the same rows 16 at a time: the GEMV
    yg = torch.cat([lin(x[i:i + 16]) for i in range(0, rows, 16)]).float()
    rel = float((y - yg).norm() / yg.norm())
    assert rel < 1e-3, rel


@pytest.mark.parametrize("n", [24, 40])
def test_frac_dense_swiglu_runs_the_gemm(n):
    rng = np.random.default_rng(7200 + n)
    hidden, inter, rows = 512, 256, 40
    parts = [S.linear(rng, hidden, inter, n), S.linear(rng, hidden, inter, n), S.linear(rng, inter, hidden, n)]
    lins = [X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)) for t, u, v in parts]
    assert X.swiglu_path(*[l.weight for l in lins], rows) == "dense-gemm"
    x = S.activations(rng, rows, hidden)
    y = X.swiglu(*[l.weight for l in lins], dev_f16(x)).float().cpu().numpy()
    one = [tuple(np.asarray(a)[None] for a in p) for p in parts]
    want = O.moe_swiglu(x, *one, np.zeros((rows, 1), np.int32), np.ones((rows, 1), np.float32),
                        hidden, inter, n)
    assert S.rel_fro(y, want) < 1e-3, S.rel_fro(y, want)
