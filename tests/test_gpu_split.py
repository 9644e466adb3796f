"""The table's split entries (quant.zig:51-68, LinearParts :111-128) and the
grouped linear (turboexl3_ds41/plugin.zig:105-125,243-261; sushi_ds41/src/
sushi/exl3/linear.zig:24-36) through the C ABI, against the library's own
matmul (bit for bit where the same kernels run) and the CPU oracle (paths
relative to /root/reference/plugins/)."""
import ctypes

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
    return t.cpu().contiguous().view(torch.int16).numpy()


def _lin(seed, in_f=512, out_f=384, n=64):
    rng = np.random.default_rng(seed)
    t, u, v = S.linear(rng, in_f, out_f, n)
    return rng, X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)), (t, u, v)


@pytest.mark.parametrize("rows", [1, 5, 16, 40, 300])
@pytest.mark.parametrize("use_side", [False, True])
def test_linear_split_is_matmul(rows, use_side):
    rng, lin, (t, u, v) = _lin(400 + rows)
    x = dev_f16(S.activations(rng, rows, 512))
    side = torch.cuda.Stream() if use_side else None
    want = lin(x)
    y = X.linear_split(lin.weight, x, side=side)
    assert y.shape == want.shape and y.dtype == want.dtype
    assert (bits(y) == bits(want)).all(), (rows, use_side)
    # the inner product, then the finish: the same values
    z = X.linear_split(lin.weight, x, inner=True, side=side)
    assert (bits(z) == bits(X.inner(lin.weight, X.prepare(lin.weight, x)))).all()
    y2 = X.linear_finish(lin.weight, [z], X.DT_F16)
    assert (bits(y2) == bits(want)).all()
    yo = S.h2f(O.project(x.float().cpu().numpy(), t, u, v, 512, 384, 64))
    assert S.rel_fro(y.float().cpu().numpy(), yo) < 1e-3


@pytest.mark.parametrize("rows", [1, 7, 40])
@pytest.mark.parametrize("dt", [X.DT_F16, X.DT_BF16, X.DT_F32])
def test_linear_prepared_and_finish_dtypes(rows, dt):
    rng, lin, (t, u, v) = _lin(500 + rows)
    x = dev_f16(S.activations(rng, rows, 512))
    xp = X.prepare(lin.weight, x)
    y = X.linear_prepared(lin.weight, xp, dt)
    tdt = {X.DT_F16: torch.float16, X.DT_BF16: torch.bfloat16, X.DT_F32: torch.float32}[dt]
    assert y.dtype == tdt and y.shape == (rows, 384)
    # same values as the f16 matmul, in the requested dtype
    want = lin(x).to(tdt)
    assert torch.equal(y, want)


def test_linear_finish_of_row_pieces():
    rng, lin, _ = _lin(601)
    x = dev_f16(S.activations(rng, 70, 512))
    zs = [X.linear_split(lin.weight, x[a:b], inner=True) for a, b in ((0, 40), (40, 41), (41, 70))]
    y = X.linear_finish(lin.weight, zs, X.DT_F16)
    want = torch.cat([X.finish(lin.weight, z) for z in zs])
    assert (bits(y) == bits(want)).all()


def test_linear_pieces_and_piece():
    rng, lin, (t, u, v) = _lin(602)
    x = dev_f16(S.activations(rng, 64, 512))
    v_, held = X.linear_pieces(lin.weight, [40, 24])
    assert v_.is_ok(), v_
    assert held.owned == 0 and held.data == lin.weight.w.data
    zs = [X.linear_piece(lin.weight, x[:40], held), X.linear_piece(lin.weight, x[40:], held)]
    # a piece with prepared rows gives the same inner product
    zp = X.linear_piece(lin.weight, X.prepare(lin.weight, x[40:]), held, prepared=True)
    assert (bits(zp) == bits(zs[1])).all()
    y = X.linear_finish(lin.weight, zs, X.DT_F16)
    # each piece is the matmul of its rows
    want = torch.cat([lin(x[:40]), lin(x[40:])])
    assert (bits(y) == bits(want)).all()
    yo = S.h2f(O.project(x.float().cpu().numpy(), t, u, v, 512, 384, 64))
    assert S.rel_fro(y.float().cpu().numpy(), yo) < 1e-3
    # pieces that would take another kernel path than the whole call: refused
    v2, _ = X.linear_pieces(lin.weight, [40, 8])
    assert v2.code == X.UNSUPPORTED and "kernel path" in v2.reason
    # a held array of another weight: refused
    _, other, _ = _lin(603)
    _, held2 = X.linear_pieces(other.weight, [20])
    with pytest.raises(X.Exl3Error):
        X.linear_piece(lin.weight, x[:20], held2)


@pytest.mark.parametrize("rows", [1, 3, 16, 40])
def test_grouped_linear(rows):
    rng = np.random.default_rng(700 + rows)
    G, in_f, out_f, n = 4, 512, 256, 48
    parts = [S.linear(rng, in_f, out_f, n) for _ in range(G)]
    src = {}
    for g, (t, u, v) in enumerate(parts):
        src[f"m.wo_a.slice.{g}.trellis"] = t.view(np.int16)
        src[f"m.wo_a.slice.{g}.suh"] = u.view(np.float16)
        src[f"m.wo_a.slice.{g}.svh"] = v.view(np.float16)
    L = X.Loader('{"format":"exl3","codebook":"mul1"}', X.DictSource(src))
    assert L.opened.is_ok()
    v, w = L.load_tensor("m.wo_a", in_f)
    assert v.is_ok(), v
    assert w.flags == 1 and w.w.dims() == (G, in_f // 16, out_f // 16, n)
    assert X.matmul_path(w, rows) == ("gemm-groups" if rows > 16 else "per-group")
    x = S.activations(rng, rows * G, in_f).reshape(rows, G, in_f)
    y = X.matmul(w, dev_f16(x.reshape(rows, G, in_f)), out=torch.empty(rows, G, out_f,
                                                                     dtype=torch.float16, device=DEV))
    y = y.float().cpu().numpy()
    for g, (t, u, vv) in enumerate(parts):
        yo = S.h2f(O.project(x[:, g, :].astype(np.float32), t, u, vv, in_f, out_f, n))
        assert S.rel_fro(y[:, g, :], yo) < 1e-3, g
        assert S.row_rel(y[:, g, :], yo).max() < 2e-3, g
        if rows <= 16:
            # group g alone through its own linear: the same kernels, values
            lin = X.Linear(dev_u16(t), dev_f16(u), dev_f16(vv))
            yg = lin(dev_f16(np.ascontiguousarray(x[:, g, :]))).float().cpu().numpy()
            assert np.array_equal(y[:, g, :], yg), g
    # a grouped linear is not an expert bank
    xs = dev_f16(S.activations(rng, 2, in_f))
    with pytest.raises(X.Exl3Error):
        X.swiglu(w, w, w, xs)
    X.release(w)
    L.close()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_grouped_linear_prompt_in_one_gemm(dtype):
    """Prompt rows of a grouped linear: one prepare over every group (x read
    in place) and one grouped GEMM over every group's row tiles, finish
    fused (turboexl3_ds41/src/woa_join.zig:1-5).  At a shape where each
    group's linear alone runs the GEMM without splitting k (160 tiles), the
    values equal the per-group matmul bit for bit (the same kernel
    arithmetic); every row within the bar of the oracle, in every dtype."""
    rng = np.random.default_rng(1280)
    G, in_f, out_f, n, rows = 2, 512, 4096, 64, 1280
    parts = [S.linear(rng, in_f, out_f, n) for _ in range(G)]
    src = {}
    for g, (t, u, v) in enumerate(parts):
        src[f"m.wo_a.slice.{g}.trellis"] = t.view(np.int16)
        src[f"m.wo_a.slice.{g}.suh"] = u.view(np.float16)
        src[f"m.wo_a.slice.{g}.svh"] = v.view(np.float16)
    L = X.Loader('{"format":"exl3","codebook":"mul1"}', X.DictSource(src))
    v, wg = L.load_tensor("m.wo_a", in_f)
    assert v.is_ok(), v
    assert X.matmul_path(wg, rows) == "gemm-groups"
    x = S.activations(rng, rows * G, in_f).reshape(rows, G, in_f)
    xd = torch.from_numpy(x.astype(np.float32)).to(DEV).to(dtype)
    y = X.matmul(wg, xd, out=torch.empty(rows, G, out_f, dtype=dtype, device=DEV))
    for g, (t, u, vv) in enumerate(parts):
        lin = X.Linear(dev_u16(t), dev_f16(u), dev_f16(vv))
        assert X.matmul_path(lin.weight, rows) == "gemm"
        yg = lin(xd[:, g, :].contiguous())
        assert torch.equal(y[:, g, :], yg), g
        if dtype == torch.float16:
            yo = S.h2f(O.project(x[:, g, :].astype(np.float32), t, u, vv, in_f, out_f, n))
            got = y[:, g, :].float().cpu().numpy()
            assert S.rel_fro(got, yo) < 1e-3 and S.row_rel(got, yo).max() < 2e-3, g
    X.release(wg)
    L.close()


# ------------------------------------------------------- swiglu_shared

def _banks(rng, E, hidden, inter, n):
    parts = [S.linear(rng, hidden, inter, n, experts=E), S.linear(rng, hidden, inter, n, experts=E),
             S.linear(rng, inter, hidden, n, experts=E)]
    keep = [tuple(f(a) for f, a in zip((dev_u16, dev_f16, dev_f16), p)) for p in parts]
    return parts, [X.wrap(*k) for k in keep], keep


def _shared_oracle(x, parts, sparts, inds, scores, lg, hidden, inter, n):
    routed = O.moe_swiglu(x, *parts, inds, scores, hidden, inter, n)
    one = [tuple(np.asarray(a)[None] for a in p) for p in sparts]
    shared = O.moe_swiglu(x, *one, np.zeros((x.shape[0], 1), np.int32),
                          np.ones((x.shape[0], 1), np.float32), hidden, inter, n)
    sig = (1.0 / (1.0 + np.exp(-lg.astype(np.float32)))).astype(np.float16).astype(np.float32)
    return routed + sig[:, None] * shared


@pytest.mark.parametrize("rows", [1, 3, 8])
@pytest.mark.parametrize("mode", ["routes+logit", "logits+gate_vec"])
def test_swiglu_shared_against_oracle(rows, mode):
    rng = np.random.default_rng(800 + rows + (100 if mode[0] == "l" else 0))
    E, hidden, inter, k, n = 8, 512, 256, 3, 64
    parts, banks, keep = _banks(rng, E, hidden, inter, n)
    sparts = [S.linear(rng, hidden, inter, n), S.linear(rng, hidden, inter, n),
              S.linear(rng, inter, hidden, n)]
    shared = [X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)) for t, u, v in sparts]
    x = S.activations(rng, rows, hidden)
    xd = dev_f16(x)
    if mode == "routes+logit":
        logits = rng.standard_normal((rows, E)).astype(np.float32)
        inds, scores = O.route_topk(logits, k)
        lg = rng.standard_normal(rows).astype(np.float16)
        y = X.swiglu_shared(*banks, xd, [s.weight for s in shared],
                            inds=torch.from_numpy(inds).to(DEV),
                            scores=torch.from_numpy(scores).to(DEV), logit=dev_f16(lg))
    else:
        logits = rng.standard_normal((rows, E)).astype(np.float16)
        inds, scores = O.route_topk(logits.astype(np.float32), k)
        gv = (rng.standard_normal(hidden) * 0.05).astype(np.float16)
        lg = (x.astype(np.float32) @ gv.astype(np.float32)).astype(np.float16)
        y = X.swiglu_shared(*banks, xd, [s.weight for s in shared], logits=dev_f16(logits), k=k,
                            gate_vec=dev_f16(gv))
    want = _shared_oracle(x, parts, sparts, inds, scores, lg, hidden, inter, n)
    got = y.float().cpu().numpy()
    assert S.rel_fro(got, want) < 1e-3, S.rel_fro(got, want)
    assert (S.row_rel(got, want) < 3e-3).all()


@pytest.mark.parametrize("gate", ["logit", "gate_vec"])
def test_swiglu_shared_one_row_equals_batched_row(gate):
    # one row with given routes runs without the route launch (the routed
    # launches read the k routes, the combine forms the shared gate); the
    # same row inside a 2-row call runs through the route launch: equal bit
    # for bit, gate from the logit or from x . gate_vec
    rng = np.random.default_rng(950 + len(gate))
    E, hidden, inter, k, n = 8, 512, 256, 3, 64
    parts, banks, keep = _banks(rng, E, hidden, inter, n)
    sparts = [S.linear(rng, hidden, inter, n), S.linear(rng, hidden, inter, n),
              S.linear(rng, inter, hidden, n)]
    shared = [X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)) for t, u, v in sparts]
    x = S.activations(rng, 2, hidden)
    logits = rng.standard_normal((2, E)).astype(np.float32)
    inds, scores = O.route_topk(logits, k)
    kw = ({"logit": dev_f16(rng.standard_normal(2).astype(np.float16))} if gate == "logit" else
          {"gate_vec": dev_f16((rng.standard_normal(hidden) * 0.05).astype(np.float16))})
    ti, ts = torch.from_numpy(inds).to(DEV), torch.from_numpy(scores).to(DEV)
    y2 = X.swiglu_shared(*banks, dev_f16(x), [s.weight for s in shared], inds=ti, scores=ts, **kw)
    kw1 = {key: v[:1] for key, v in kw.items()} if gate == "logit" else kw
    y1 = X.swiglu_shared(*banks, dev_f16(x[:1]), [s.weight for s in shared], inds=ti[:1].contiguous(),
                         scores=ts[:1].contiguous(), **kw1)
    torch.cuda.synchronize()
    assert torch.equal(y1[0], y2[0])


def test_swiglu_shared_refusals():
    rng = np.random.default_rng(901)
    E, hidden, inter, k, n = 8, 512, 256, 2, 64
    parts, banks, keep = _banks(rng, E, hidden, inter, n)
    sp = [S.linear(rng, hidden, inter, n), S.linear(rng, hidden, inter, n),
          S.linear(rng, inter, hidden, n)]
    shared = [X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)) for t, u, v in sp]
    # prefill-sized batches: the host's chain
    x = dev_f16(S.activations(rng, 100, hidden))
    logits = dev_f16(rng.standard_normal((100, E)).astype(np.float16))
    gv = dev_f16((rng.standard_normal(hidden) * 0.05).astype(np.float16))
    with pytest.raises(X.Exl3Error, match="chain"):
        X.swiglu_shared(*banks, x, [s.weight for s in shared], logits=logits, k=k, gate_vec=gv)
    # a shared expert of another width
    wide = [S.linear(rng, hidden, 384, n), S.linear(rng, hidden, 384, n), S.linear(rng, 384, hidden, n)]
    other = [X.Linear(dev_u16(t), dev_f16(u), dev_f16(v)) for t, u, v in wide]
    x1 = dev_f16(S.activations(rng, 2, hidden))
    with pytest.raises(X.Exl3Error, match="differs"):
        X.swiglu_shared(*banks, x1, [s.weight for s in other], logits=logits[:2], k=k, gate_vec=gv)
    # neither a logit nor gate_vec
    with pytest.raises(X.Exl3Error):
        X.swiglu_shared(*banks, x1, [s.weight for s in shared], logits=logits[:2], k=k)


# ------------------------------------------------- new arrays (out.data NULL)

def _hip():
    return ctypes.CDLL("libamdhip64.so")


def _device_values(ptr, rows, cols):
    """rows x cols f16 at a raw device address, copied to the host."""
    torch.cuda.synchronize()
    h = np.empty((rows, cols), np.float16)
    assert _hip().hipMemcpy(ctypes.c_void_p(h.ctypes.data), ctypes.c_void_p(ptr),
                            ctypes.c_size_t(h.nbytes), 2) == 0  # device to host
    return h


def test_new_arrays_come_from_a_per_stream_pool():
    """The reference's convention: out receives a new array the caller owns
    (quant.zig:41-50).  exl3_array_free returns its memory to the pool of the
    stream it was made for; the next call on that stream reuses it (same
    address, no hipMalloc), a call on another stream does not take it, the
    values are those of a caller-buffer call, and exl3_scratch_release
    empties the pool."""
    rng = np.random.default_rng(41)
    t, u, v = S.linear(rng, 512, 256, 64)
    lin = X.Linear(dev_u16(t), dev_f16(u), dev_f16(v))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def new(x, s):
        a = X.Array()
        X.check(X.lib().exl3_matmul(ctypes.byref(lin.weight), X.array(x), X.stream_handle(s),
                                    ctypes.byref(a)), "matmul")
        assert a.owned == 1 and a.ndim == 2 and (a.shape[0], a.shape[1]) == (x.shape[0], 256)
        return a

    for rows in (1, 40):
        x = dev_f16(S.activations(rng, rows, 512))
        want = lin(x).cpu().numpy()
        a1 = new(x, s1)
        p1 = a1.data
        assert np.array_equal(_device_values(p1, rows, 256), want)
        X.lib().exl3_array_free(ctypes.byref(a1))
        assert not a1.data and a1.owned == 0
        a2 = new(x, s1)  # same stream, same size: the pooled block
        assert a2.data == p1
        a3 = new(x, s2)  # another stream: not s1's block
        assert a3.data != p1
        assert np.array_equal(_device_values(a2.data, rows, 256), want)
        for a in (a2, a3):
            X.lib().exl3_array_free(ctypes.byref(a))
    for s in (s1, s2):
        X.scratch_release(0, s)
    a4 = new(dev_f16(S.activations(rng, 1, 512)), s1)
    X.lib().exl3_array_free(ctypes.byref(a4))
    X.scratch_release(0, s1)
