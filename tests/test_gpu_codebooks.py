"""The table codebooks (spec1, std1: hash-mask; pair1: a pair of weights from
one codeword) through the C ABI against the CPU oracle: decoded tiles bit for
bit at every table's rates and at narrowed windows, and the GEMV, GEMM and
routed-MoE paths within the matmul bar (sushi_ds41/src/sushi/exl3/
expert_exl3.zig:288-357, codebook_tables.zig:99-206; paths relative to
/root/reference/plugins/).  The oracle's tables are pinned by the reference's
published digests (tests/test_oracle.py)."""
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


def host_u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# (codebook, table name, oracle codebook argument)
FORMS = {
    "spec1-w15": ("spec1", "spec1-w15", O.spec1(O.TAB_SPEC1_W15)),
    "spec1-w16": ("spec1", "spec1-w16", O.spec1(O.TAB_SPEC1_W16)),
    "std1": ("std1", "std1", O.CB_STD1),
    "pair1": ("pair1", "pair1-w16-v1", O.CB_PAIR1),
}
# every form at rates of its table: integer (compile-time windows) and
# fractional (run-time windows) ones
CASES = ([("spec1-w15", n) for n in (16, 18, 24, 32, 40, 48, 50, 64, 80, 96, 112, 126, 128)] +
         [("spec1-w16", n) for n in (24, 32, 40, 48, 64)] +
         [("std1", n) for n in (24, 32, 44, 48, 64)] +
         [("pair1", n) for n in (24, 26, 32, 40, 48, 58, 64)])


def make(rng, form, in_f, out_f, n, window=16):
    cb, table, _ = FORMS[form]
    trellis, suh, svh = S.linear(rng, in_f, out_f, n)
    lin = X.Linear(dev_u16(trellis), dev_f16(suh), dev_f16(svh), cb, window, table)
    return lin, trellis, suh, svh


@pytest.mark.parametrize("form,n", CASES)
def test_table_codebook_decode_bit_exact(form, n):
    rng = np.random.default_rng(2000 + n)
    lin, trellis, _, _ = make(rng, form, 256, 384, n)
    got = host_u16(X.decode_matrix(lin.weight))
    np.testing.assert_array_equal(got, O.reconstruct_inner(trellis, 256, 384, n, FORMS[form][2]))


@pytest.mark.parametrize("window", [8, 12, 15])
@pytest.mark.parametrize("form,n", [("spec1-w15", 32), ("spec1-w15", 40), ("std1", 48), ("spec1-w16", 64)])
def test_table_codebook_decode_narrowed_windows(form, n, window):
    # spec1 and std1 tables decode at any window (codebook_tables.zig:354-357)
    rng = np.random.default_rng(3000 + window + n)
    lin, trellis, _, _ = make(rng, form, 128, 256, n, window)
    got = host_u16(X.decode_matrix(lin.weight))
    np.testing.assert_array_equal(got, O.reconstruct_inner(trellis, 128, 256, n, FORMS[form][2], window))


@pytest.mark.parametrize("rows", [1, 4, 16, 40, 300])
@pytest.mark.parametrize("form,n", [("spec1-w15", 16), ("spec1-w15", 40), ("spec1-w15", 128), ("std1", 48),
                                    ("pair1", 32), ("pair1", 40), ("pair1", 64), ("spec1-w16", 24)])
def test_table_codebook_matmul_against_oracle(form, n, rows):
    # GEMV at <= 16 rows, the GEMM above (integer rates and the half-integer
    # rates n = 24 and 40 alike)
    rng = np.random.default_rng(4000 + n + rows)
    in_f, out_f = 512, 384
    lin, trellis, suh, svh = make(rng, form, in_f, out_f, n)
    x = S.activations(rng, rows, in_f)
    y = lin(dev_f16(x)).float().cpu().numpy()
    want = S.h2f(O.project(x.astype(np.float32), trellis, suh, svh, in_f, out_f, n, FORMS[form][2]))
    assert S.rel_fro(y, want) < 1e-3, S.rel_fro(y, want)
    assert np.isfinite(y).all()


@pytest.mark.parametrize("rows", [1, 5])
@pytest.mark.parametrize("form,n", [("spec1-w15", 48), ("pair1", 32)])
def test_table_codebook_routed_moe_against_oracle(form, n, rows):
    rng = np.random.default_rng(5000 + n + rows)
    cb, table, ocb = FORMS[form]
    E, hidden, inter, k = 8, 512, 256, 2
    parts = [S.linear(rng, hidden, inter, n, experts=E), S.linear(rng, hidden, inter, n, experts=E),
             S.linear(rng, inter, hidden, n, experts=E)]
    keep = [tuple(f(a) for f, a in zip((dev_u16, dev_f16, dev_f16), p)) for p in parts]
    banks = [X.wrap(*t, codebook=cb, table=table) for t in keep]
    x = S.activations(rng, rows, hidden)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    inds, scores = O.route_topk(logits, k)
    y = X.swiglu(*banks, dev_f16(x), torch.from_numpy(inds).to(DEV), torch.from_numpy(scores).to(DEV))
    want = O.moe_swiglu(x, *parts, inds, scores, hidden, inter, n, ocb)
    got = y.float().cpu().numpy()
    assert S.rel_fro(got, want) < 1e-3, S.rel_fro(got, want)


def test_table_codebooks_do_not_share_a_launch_with_another_table():
    # linears of one shared launch decode with one row: a spec1 and an std1
    # weight of the same rate are refused together
    rng = np.random.default_rng(6001)
    a, *_ = make(rng, "spec1-w15", 256, 128, 32)
    b, *_ = make(rng, "std1", 256, 128, 32)
    x = dev_f16(S.activations(rng, 1, 256))
    with pytest.raises(X.Exl3Error, match="codebook"):
        X.matmul_shared([a.weight, b.weight], x)
