"""BASELINE.json's configurations 0-3 at their real shapes, through the C ABI.

Bars: matmul outputs within 1e-3 relative
Frobenius error of a float64 (or the f16-rounding oracle's) reference, and,
so that one mis-indexed tile cannot hide inside a large matrix, every row
within 2e-3 of it (a wrong tile or column group moves its rows by O(1)).
Config 4 (the 36-layer decode step) is in tests/test_decoder.py.

  config 0  one K=4 linear 4096 -> 4096 at batch 1;
  config 1  K in {2, 3, 4, 5, 6, 8} on the Qwen3-8B shapes (q/o, k/v,
            gate/up, down) at batch 1, 2, 4 and 8, launched as the bench issues
            them (q+k+v and gate+up share a launch);
  config 2  the prefill GEMM at K=4 on the four shapes at M in {128, 512,
            2048, 4096}, every row against x @ W_public in float64;
  config 3  the DeepSeek-V3-shaped routed MoE layer (hidden 7168, expert
            intermediate 2048, 256 experts, top-8, K=3) plus its shared
            expert, at batch 1, 16 and 64, a 1024-token prefill through the
            grouped GEMM and an 8200-token prefill (65,600 slots: windows of
            rows), every row against a float64 restatement of the routed
            SwiGLU with the reference's f16 rounding points, and sampled rows
            against the oracle's composition
            (sushi_ds41/src/sushi/exl3/expert_exl3_kernels.zig:3151-3206;
            paths relative to /root/reference/plugins/).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from plugins_amd import exl3 as X  # noqa: E402
from tests import _synth as S  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ROW_BAR = 2e-3


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV)


def dev_f16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16) if a.dtype == np.uint16
                            else np.ascontiguousarray(a, np.float16)).to(DEV)


def host_u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def check_rows(got, want, what):
    got = np.asarray(got, np.float64)
    assert S.rel_fro(got, want) < 1e-3, (what, S.rel_fro(got, want))
    rr = S.row_rel(got, want)
    assert rr.max() < ROW_BAR, (what, int(rr.argmax()), float(rr.max()))


QWEN = {"q/o": (4096, 4096), "k/v": (4096, 1024), "gate/up": (4096, 12288), "down": (12288, 4096)}


# ----------------------------------------------------------------- config 0

def test_config0_single_linear_batch1():
    rng = np.random.default_rng(0)
    in_f, out_f, n = 4096, 4096, 64
    t, suh, svh = S.linear(rng, in_f, out_f, n)
    lin = X.Linear(dev_u16(t), dev_f16(suh), dev_f16(svh))
    x = S.activations(rng, 1, in_f)
    assert X.matmul_path(lin.weight, 1) == "gemv"
    y = lin(dev_f16(x)).float().cpu().numpy()
    w = O.reconstruct_inner(t, in_f, out_f, n)
    assert np.array_equal(host_u16(X.decode_matrix(lin.weight)), w)  # decode bit-exact
    check_rows(y, S.public_matmul(x, w, suh, svh), "float64")
    check_rows(y, S.h2f(O.project(x.astype(np.float32), t, suh, svh, in_f, out_f, n)), "oracle")


# ----------------------------------------------------------------- config 1

@pytest.mark.parametrize("k", [2, 3, 4, 5, 6, 8])
def test_config1_qwen3_shapes_every_rate(k):
    """The seven linears of a Qwen3-8B layer at rate K, batch 8, 4, 2 and 1
    (the first rows of the same activations), against the oracle's
    projection."""
    rng = np.random.default_rng(10 + k)
    n = 16 * k
    names = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
             ("gate", 4096, 12288), ("up", 4096, 12288), ("down", 12288, 4096)]
    parts, lins = {}, {}
    for name, i, o in names:
        parts[name] = S.linear(rng, i, o, n)
        t, u, v = parts[name]
        lins[name] = X.Linear(dev_u16(t), dev_f16(u), dev_f16(v))
    xs = {4096: S.activations(rng, 8, 4096), 12288: S.activations(rng, 8, 12288)}
    want = {}
    for name, i, o in names:
        t, u, v = parts[name]
        want[name] = S.h2f(O.project(xs[i].astype(np.float32), t, u, v, i, o, n))
    for B in (8, 4, 2, 1):
        got = {}
        for group in (["q", "k", "v"], ["o"], ["gate", "up"], ["down"]):
            i = lins[group[0]].in_features
            x = dev_f16(xs[i][:B])
            if len(group) == 1:
                got[group[0]] = lins[group[0]](x)
            else:
                ys = X.matmul_shared([lins[g].weight for g in group], x)
                got.update(zip(group, ys))
        for name, _, _ in names:
            check_rows(got[name].float().cpu().numpy(), want[name][:B], f"K={k} B={B} {name}")


# ----------------------------------------------------------------- config 2

_gemm_cache = {}


def _gemm_linear(shape):
    if shape not in _gemm_cache:
        _gemm_cache.clear()
        in_f, out_f = QWEN[shape]
        rng = np.random.default_rng(20 + list(QWEN).index(shape))
        t, suh, svh = S.linear(rng, in_f, out_f, 64)
        lin = X.Linear(dev_u16(t), dev_f16(suh), dev_f16(svh))
        _gemm_cache[shape] = (lin, O.reconstruct_inner(t, in_f, out_f, 64), suh, svh)
    return _gemm_cache[shape]


@pytest.mark.parametrize("shape", list(QWEN))
@pytest.mark.parametrize("M", [128, 512, 2048, 4096])
def test_config2_prefill_gemm_every_row(shape, M):
    lin, w, suh, svh = _gemm_linear(shape)
    in_f, out_f = QWEN[shape]
    rng = np.random.default_rng(M + in_f + out_f)
    x = S.activations(rng, M, in_f)
    assert X.matmul_path(lin.weight, M) == "gemm"
    y = lin(dev_f16(x)).float().cpu().numpy()
    check_rows(y, S.public_matmul(x, w, suh, svh), f"{shape} M={M}")


# ----------------------------------------------------------------- config 3

E, HIDDEN, INTER, TOPK, K3 = 256, 7168, 2048, 8, 3


@pytest.fixture(scope="module")
def deepseek():
    """The layer's three banks (gate/up 7168 -> 2048, down 2048 -> 7168 for
    each of 256 experts, K=3) and its shared expert, on the host (for the
    oracle) and wrapped on the device."""
    rng = np.random.default_rng(3)
    n = 16 * K3
    banks = [S.linear(rng, HIDDEN, INTER, n, experts=E), S.linear(rng, HIDDEN, INTER, n, experts=E),
             S.linear(rng, INTER, HIDDEN, n, experts=E)]
    dev = [X.wrap(dev_u16(t), dev_f16(u), dev_f16(v)) for (t, u, v) in banks]
    shared = [S.linear(rng, HIDDEN, INTER, n), S.linear(rng, HIDDEN, INTER, n),
              S.linear(rng, INTER, HIDDEN, n)]
    sdev = [X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)) for (t, u, v) in shared]
    yield banks, dev, shared, sdev
    for w in dev:
        X.release(w)


_H128 = None


def _had(v):
    """The 128-point Hadamard (unscaled) over each 128-block of v's last axis."""
    global _H128
    if _H128 is None:
        _H128 = torch.from_numpy(S.hadamard(128)).to(DEV, torch.float64)
    return (v.reshape(-1, 128) @ _H128).reshape(v.shape)


def _f16(v):
    return v.to(torch.float16).to(torch.float64)


def _project64(x, w, suh, svh):
    """One linear in float64 with the reference's f16 rounding points
    (sushi_ds41/src/sushi/exl3/expert_exl3.zig:490-544): xp = f16(H(f16(x) *
    suh) / sqrt(128)), z = f16(xp @ W_inner), y = f16(H(z) / sqrt(128) * svh);
    the sums in float64 instead of f32."""
    xp = _f16(_had(_f16(x) * suh) * S.HAD_SCALE)
    z = _f16(xp @ w)
    return _f16(_had(z) * S.HAD_SCALE * svh)


def _moe64(dev, x, inds, scores, rows=None):
    """The routed SwiGLU (moeSwigluHost, sushi_ds41/src/sushi/exl3/
    expert_exl3_kernels.zig:3151-3206) in float64 on the device, expert by
    expert: each expert's W_inner from exl3_decode_matrix (bit-exact against
    the oracle's reconstructInner: test_config3_decode_anchors and the decode
    tests), its routed rows through gate and up (_project64), h =
    f16(silu(g) * u), down, and y = sum_k score_k * down_k.  rows: the rows
    to form (all by default)."""
    T = x.shape[0]
    rows = np.arange(T) if rows is None else np.asarray(rows)
    xd = torch.from_numpy(x[rows].astype(np.float64)).to(DEV)
    ind = inds[rows]
    sc = torch.from_numpy(scores[rows].astype(np.float64)).to(DEV)
    y = torch.zeros(len(rows), x.shape[1], dtype=torch.float64, device=DEV)
    sv = [(b._keep[1].view(torch.float16).double(), b._keep[2].view(torch.float16).double())
          for b in dev]
    for e in np.unique(ind):
        r, k = np.nonzero(ind == e)
        rr = torch.from_numpy(r).to(DEV)
        w = [X.decode_matrix(b, int(e)).view(torch.float16).double() for b in dev]
        g = _project64(xd[rr], w[0], sv[0][0][e], sv[0][1][e])
        u = _project64(xd[rr], w[1], sv[1][0][e], sv[1][1][e])
        h = _f16(g / (1.0 + torch.exp(-g)) * u)
        d = _project64(h, w[2], sv[2][0][e], sv[2][1][e])
        y.index_add_(0, rr, d * sc[rr, torch.from_numpy(k).to(DEV)][:, None])
    return y.cpu().numpy()


def _routed(deepseek, tokens, sample, seed):
    """The layer's output for `tokens` routed rows: all rows against the
    float64 restatement, the `sample` rows against the oracle's composition
    (the reference's f32 arithmetic)."""
    banks, dev, _, _ = deepseek
    rng = np.random.default_rng(seed)
    x = S.activations(rng, tokens, HIDDEN)
    inds, scores = O.route_topk(rng.standard_normal((tokens, E)).astype(np.float32), TOPK)
    y = X.swiglu(dev[0], dev[1], dev[2], dev_f16(x).reshape(tokens, 1, HIDDEN),
                 torch.from_numpy(inds).to(DEV).reshape(tokens, 1, TOPK),
                 torch.from_numpy(scores).to(DEV).reshape(tokens, 1, TOPK))
    got = y.float().cpu().numpy().reshape(tokens, HIDDEN)
    check_rows(got, _moe64(dev, x, inds, scores), f"routed batch {tokens}, every row, float64")
    want = O.moe_swiglu(x[sample].astype(np.float32), banks[0], banks[1], banks[2], inds[sample],
                        scores[sample], HIDDEN, INTER, 16 * K3)
    check_rows(got[sample], want, f"routed batch {tokens}, sampled rows, oracle")
    return inds


def test_config3_decode_anchors(deepseek):
    """exl3_decode_matrix (the float64 restatement's W_inner) equals the
    oracle's reconstructInner at the DeepSeek-V3 shapes, for experts spread
    over each bank."""
    banks, dev, _, _ = deepseek
    for b, (t, _, _), (i, o) in zip(dev, banks, [(HIDDEN, INTER), (HIDDEN, INTER), (INTER, HIDDEN)]):
        for e in (0, 97, 255):
            assert np.array_equal(host_u16(X.decode_matrix(b, e)), O.reconstruct_inner(t[e], i, o, 16 * K3)), e


@pytest.mark.parametrize("tokens", [1, 16])
def test_config3_routed_every_row(deepseek, tokens):
    _, dev, _, _ = deepseek
    assert X.swiglu_path(dev[0], dev[1], dev[2], tokens, TOPK) == "routed-gemv"
    _routed(deepseek, tokens, np.arange(tokens), 300 + tokens)


@pytest.mark.parametrize("tokens,path", [(64, "routed-gemv"), (1024, "routed-gemm")])
def test_config3_routed_prefill_every_row(deepseek, tokens, path):
    """Every row against the float64 restatement, eight rows spread over the
    batch against the oracle.  At 1024 tokens (32 slots per expert on
    average) the experts' slots go through the grouped GEMM in items of up
    to 256 slots."""
    _, dev, _, _ = deepseek
    assert X.swiglu_path(dev[0], dev[1], dev[2], tokens, TOPK) == path
    sample = np.unique(np.linspace(0, tokens - 1, 8).astype(int))
    _routed(deepseek, tokens, sample, 400 + tokens)


def test_config3_beyond_one_launch(deepseek):
    """8200 tokens x top-8 = 65,600 slots, more than one launch orders
    (MOE_SLOTS_MAX = 65,535): the call runs as windows of 8191 rows (the
    reference's moePrefill has no such bound, sushi_ds41/src/sushi/exl3/
    expert_exl3_kernels.zig:2955-3023).  Every row against the float64
    restatement, rows on both sides of the window edge against the oracle."""
    _, dev, _, _ = deepseek
    tokens = 8200
    assert tokens * TOPK > 65535
    assert X.swiglu_path(dev[0], dev[1], dev[2], tokens, TOPK) == "routed-gemm"
    _routed(deepseek, tokens, np.array([0, 8190, 8191, 8199]), 600)


def test_routed_beyond_one_launch_small_bank_every_row():
    """A small bank (hidden 128, intermediate 128, 16 experts, top-8) at
    8300 tokens (66,400 slots, two windows): every row against the oracle's
    composition (sushi_ds41/src/sushi/exl3/expert_exl3_kernels.zig:3151-3206),
    in the grouped GEMM; the same rows in one call as in two calls split at
    the window edge, bit for bit."""
    rng = np.random.default_rng(8300)
    Es, hid, inter, k, T, n = 16, 128, 128, 8, 8300, 48
    banks = [S.linear(rng, hid, inter, n, experts=Es), S.linear(rng, hid, inter, n, experts=Es),
             S.linear(rng, inter, hid, n, experts=Es)]
    dev = [X.wrap(dev_u16(t), dev_f16(u), dev_f16(v)) for (t, u, v) in banks]
    x = S.activations(rng, T, hid)
    inds, scores = O.route_topk(rng.standard_normal((T, Es)).astype(np.float32), k)
    xs, ids, scs = dev_f16(x), torch.from_numpy(inds).to(DEV), torch.from_numpy(scores).to(DEV)
    assert X.swiglu_path(dev[0], dev[1], dev[2], T, k) == "routed-gemm"
    y = X.swiglu(dev[0], dev[1], dev[2], xs.reshape(T, 1, hid), ids.reshape(T, 1, k),
                 scs.reshape(T, 1, k))
    got = y.float().cpu().numpy().reshape(T, hid)
    want = O.moe_swiglu(x.astype(np.float32), banks[0], banks[1], banks[2], inds, scores, hid,
                        inter, n)
    check_rows(got, want, "small bank, 8300 tokens")
    w = 65535 // k
    parts = [X.swiglu(dev[0], dev[1], dev[2], xs[a:b].reshape(b - a, 1, hid),
                      ids[a:b].reshape(b - a, 1, k), scs[a:b].reshape(b - a, 1, k))
             for a, b in ((0, w), (w, T))]
    assert torch.equal(torch.cat([p.reshape(-1, hid) for p in parts]), y.reshape(T, hid))


@pytest.mark.parametrize("tokens", [1, 16, 64])
def test_config3_shared_expert(deepseek, tokens):
    _, _, shared, sdev = deepseek
    rng = np.random.default_rng(500 + tokens)
    x = S.activations(rng, tokens, HIDDEN)
    y = X.swiglu(sdev[0].weight, sdev[1].weight, sdev[2].weight, dev_f16(x))
    ones = np.zeros((tokens, 1), np.int32), np.ones((tokens, 1), np.float32)
    sample = np.unique(np.linspace(0, tokens - 1, min(tokens, 16)).astype(int))
    want = O.moe_swiglu(x[sample].astype(np.float32), *[tuple(a[None] for a in p) for p in shared],
                        ones[0][sample], ones[1][sample], HIDDEN, INTER, 16 * K3)
    check_rows(y.float().cpu().numpy()[sample], want, f"shared expert batch {tokens}")
