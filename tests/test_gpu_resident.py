"""The table's resident entries (quant.zig:96-107: resident, resident_pending,
unrotate, linear_joined) through the C ABI: the un-rotated public matrix bit
for bit against the oracle's reconstructPublic (sushi_ds41/src/sushi/exl3/
expert_exl3.zig:440-488, the same f32 operation order) and against the
float64 formula; prefill matmuls over held matrices (rates without the
prefill GEMM; at the GEMM's rates nothing is held and the GEMM stays, bit for
bit) and joined matrices within the 1e-3 relative Frobenius bar of the
oracle's projection (bf16: 2^-8); decode widths unchanged (the EXL3 GEMV, bit
for bit); the accounting and the refusals.
Paths relative to /root/reference/plugins/."""
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


def bits(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _lin(seed, in_f, out_f, n=64, codebook="mul1"):
    rng = np.random.default_rng(seed)
    t, u, v = S.linear(rng, in_f, out_f, n)
    return rng, X.Linear(dev_u16(t), dev_f16(u), dev_f16(v), codebook=codebook), (t, u, v)


@pytest.fixture(autouse=True)
def _drop_resident():
    X.resident([])
    yield
    X.resident([])
    torch.cuda.synchronize()


@pytest.mark.parametrize("n,codebook", [(64, "mul1"), (48, "mul1"), (40, "mcg")])
def test_unrotate_is_reconstruct_public_bit_for_bit(n, codebook):
    in_f, out_f = 256, 384
    rng, lin, (t, u, v) = _lin(11 + n, in_f, out_f, n, codebook)
    assert X.resident([lin.weight]) == in_f * out_f * 2
    assert X.resident_pending() == in_f * out_f * 2
    assert X.unrotate([lin.weight], [1], X.DT_F16) == [True]
    assert X.resident_pending() == 0
    # the identity's rows through the joined matrix are its rows, exactly
    eye = torch.eye(in_f, dtype=torch.float16, device=DEV)
    wp = bits(X.linear_joined([lin.weight], eye))
    cb = O.CB_MUL1 if codebook == "mul1" else O.CB_MCG
    want = O.reconstruct_public(t, u, v, in_f, out_f, n, cb)
    assert np.array_equal(wp, want), int((wp != want).sum())
    # ... and the formula in float64, within f16's rounding
    w64 = S.public_weight(O.reconstruct_inner(t, in_f, out_f, n, cb), u, v)
    assert np.allclose(S.h2f(wp), w64, rtol=2 ** -10, atol=2e-7)


@pytest.mark.parametrize("act", [X.DT_F16, X.DT_BF16, X.DT_F32])
def test_joined_group_against_the_oracle(act):
    # a q/k/v-shaped group: one input, three widths side by side
    rng = np.random.default_rng(21 + act)
    in_f, outs, n = 512, (512, 128, 128), 64
    parts = [S.linear(rng, in_f, o, n) for o in outs]
    lins = [X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)) for t, u, v in parts]
    ws = [li.weight for li in lins]
    assert X.resident(ws) == sum(in_f * o * 2 for o in outs)
    assert X.unrotate(ws, [3], act) == [True]
    tdt = {X.DT_F16: torch.float16, X.DT_BF16: torch.bfloat16, X.DT_F32: torch.float32}[act]
    x16 = S.activations(rng, 40, in_f)
    x = torch.from_numpy(x16).to(DEV).to(tdt)
    y = X.linear_joined(ws, x)
    assert y.shape == (40, sum(outs)) and y.dtype == tdt
    want = np.concatenate([S.public_matmul(x.float().cpu().numpy(),
                                           O.reconstruct_inner(t, in_f, o, n), u, v)
                           for (t, u, v), o in zip(parts, outs)], axis=1)
    # bf16 keeps 8 significant bits: its matrix and its output each round by
    # up to 2^-9, so its bar is 2^-8; f16 and f32 take the 1e-3 bar
    bar = 2.0 ** -8 if act == X.DT_BF16 else 1e-3
    assert S.rel_fro(y.float().cpu().numpy(), want) < bar
    # each member's own prefill matmul takes its columns of the joined matrix
    c = 0
    for li, o in zip(lins, outs):
        yi = li(x)
        assert S.rel_fro(yi.float().cpu().numpy(), want[:, c:c + o]) < bar
        c += o
    # the same group again takes again; a part of it does not join another
    assert X.unrotate(ws, [3], act) == [True]
    assert X.unrotate(ws[:2], [2], act) == [False]


@pytest.mark.parametrize("rows", [17, 64, 300])
def test_resident_holds_nothing_at_gemm_rates(rows):
    """At the prefill GEMM's rates the fused GEMM outruns the held-matrix
    path: resident admits the weight and reserves its bytes (pending, for
    unrotate) but holds nothing, and prefill matmuls stay the EXL3 GEMM, bit
    for bit."""
    in_f, out_f = 512, 384
    rng, lin, _ = _lin(61 + rows, in_f, out_f, n=64)
    x = dev_f16(S.activations(rng, rows, in_f))
    plain = lin(x)
    assert X.resident([lin.weight]) == in_f * out_f * 2
    assert X.resident_pending() == in_f * out_f * 2
    assert (bits(lin(x)) == bits(plain)).all()
    assert X.resident_pending() == in_f * out_f * 2


@pytest.mark.parametrize("rows", [17, 64, 300])
def test_resident_prefill_matmul(rows):
    """A rate without the prefill GEMM (n = 50: 16-row GEMV passes above 16
    rows): the held W_inner path, within the bar."""
    in_f, out_f, n = 512, 384, 50
    rng, lin, (t, u, v) = _lin(31 + rows, in_f, out_f, n=n)
    assert X.matmul_path(lin.weight, rows) == "gemv"
    x = dev_f16(S.activations(rng, rows, in_f))
    plain = lin(x)
    one = dev_f16(S.activations(rng, 1, in_f))
    plain1 = lin(one)
    assert X.resident([lin.weight], room=in_f * out_f * 2) == in_f * out_f * 2
    assert X.resident_pending() == in_f * out_f * 2
    # decode widths: the GEMV as before, nothing held yet
    assert (bits(lin(one)) == bits(plain1)).all()
    assert X.resident_pending() == in_f * out_f * 2
    y = lin(x)  # the first prefill call holds the decoded matrix
    assert X.resident_pending() == 0
    yo = S.h2f(O.project(x.float().cpu().numpy(), t, u, v, in_f, out_f, n))
    assert S.rel_fro(y.float().cpu().numpy(), yo) < 1e-3
    assert S.rel_fro(y.float().cpu().numpy(), plain.float().cpu().numpy()) < 1e-3
    # twice in a row: the same bytes
    assert (bits(lin(x)) == bits(y)).all()
    # dropped: the EXL3 GEMM again, bit for bit
    X.resident([])
    assert (bits(lin(x)) == bits(plain)).all()


def test_resident_refusals():
    in_f, out_f = 256, 256
    rng, lin, _ = _lin(41, in_f, out_f, n=50)
    with pytest.raises(X.Exl3Error) as e:
        X.resident([lin.weight], room=in_f * out_f * 2 - 1)
    assert e.value.code == X.TOO_LARGE
    assert X.resident_pending() == 0
    x8 = dev_f16(S.activations(rng, 8, in_f))
    # not un-rotated: linear_joined refuses
    with pytest.raises(X.Exl3Error):
        X.linear_joined([lin.weight], dev_f16(S.activations(rng, 32, in_f)))
    X.resident([lin.weight])
    assert X.unrotate([lin.weight], [1], X.DT_F16) == [True]
    # decode widths are the GEMV's
    with pytest.raises(X.Exl3Error) as e:
        X.linear_joined([lin.weight], x8)
    assert "decode widths" in e.value.why
    # another dtype than the group's
    with pytest.raises(X.Exl3Error):
        X.linear_joined([lin.weight], dev_f16(S.activations(rng, 32, in_f)).float())
    # a weight not admitted does not take
    _, other, _ = _lin(42, in_f, out_f)
    assert X.unrotate([other.weight], [1], X.DT_F16) == [False]


def test_release_of_a_resident_weight():
    in_f, out_f = 256, 256
    rng, lin, _ = _lin(51, in_f, out_f, n=50)
    _, keep, _ = _lin(52, in_f, out_f, n=50)
    X.resident([lin.weight, keep.weight])
    x = dev_f16(S.activations(rng, 32, in_f))
    lin(x)
    keep(x)
    assert X.resident_pending() == 0
    del lin  # releases the weight and its held matrix
    torch.cuda.synchronize()
    assert X.resident_pending() == 0
    y = keep(x)
    assert y.shape == (32, out_f)
