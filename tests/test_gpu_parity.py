"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Bars: decoded f16 tiles bit-exact; the prepare and
finish rotations bit-exact (same f32 operation order); matmul outputs within
1e-3 relative Frobenius error of an fp32-or-better CPU reference, plus the
reference's per-element bar on the inner product
(sushi_ds41/src/sushi/exl3/expert_exl3_kernels.zig:3402-3461: |err| <=
(2^-11 + depth 2^-24) sum|w x|, relative to the exact dot of the same decoded
weights; paths relative to /root/reference/plugins/).
"""
import hashlib
import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from plugins_amd import exl3 as X  # noqa: E402
from tests import _synth as S  # noqa: E402

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_golden.json")))
DEV = "cuda:0"


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV)


def dev_f16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16) if a.dtype == np.uint16
                            else np.ascontiguousarray(a, np.float16)).to(DEV)


def host_u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def make(rng, in_f, out_f, n, codebook="mul1", window=16):
    trellis, suh, svh = S.linear(rng, in_f, out_f, n)
    lin = X.Linear(dev_u16(trellis), dev_f16(suh), dev_f16(svh), codebook, window)
    return lin, trellis, suh, svh


CB = {"mul1": O.CB_MUL1, "mcg": O.CB_MCG}


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("codebook", ["mul1", "mcg"])
@pytest.mark.parametrize("n", [16, 32, 48, 64, 80, 96, 112, 128, 24, 40, 18, 50, 126])
def test_decode_matrix_bit_exact(n, codebook):
    rng = np.random.default_rng(1000 + n)
    lin, trellis, _, _ = make(rng, 256, 384, n, codebook)
    got = host_u16(X.decode_matrix(lin.weight))
    want = O.reconstruct_inner(trellis, 256, 384, n, CB[codebook])
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("window", [8, 11, 15])
@pytest.mark.parametrize("n", [32, 40, 64])
def test_decode_matrix_windows(n, window):
    rng = np.random.default_rng(77 + window)
    for cb in ("mul1", "mcg"):
        lin, trellis, _, _ = make(rng, 128, 128, n, cb, window)
        got = host_u16(X.decode_matrix(lin.weight))
        np.testing.assert_array_equal(got, O.reconstruct_inner(trellis, 128, 128, n, CB[cb], window))


@pytest.mark.parametrize("name", ["gate_up", "down", "gate_up_k2", "down_k2"])
def test_decode_matrix_reproduces_reference_golden_planes(name):
    # turboexl3_ds41/src/exl3/kernels/exl3/manifest.json golden.planes
    p = GOLD["planes"][name]
    n = 16 * p["K"]
    code = O.synth_plane(p["seed"], (p["in"] // 16) * (p["out"] // 16) * n)
    t = dev_u16(code.reshape(p["in"] // 16, p["out"] // 16, n))
    ones_in = torch.ones(p["in"], dtype=torch.float16, device=DEV)
    ones_out = torch.ones(p["out"], dtype=torch.float16, device=DEV)
    lin = X.Linear(t, ones_in, ones_out)
    w = host_u16(X.decode_matrix(lin.weight))
    assert hashlib.sha256(w.astype("<u2").tobytes()).hexdigest() == p["w_hat_sha256"]


@pytest.mark.parametrize("n", [24, 32, 40, 48])
def test_decode_matrix_reference_frac_tiles(n):
    # turboexl3_ds41/src/frac_tiles.json: real pack tiles, row-major f16
    tiles = [t for t in GOLD["frac_tiles"] if t["n"] == n][:8]
    assert len(tiles) == 8
    trellis = np.stack([np.array(t["words"], np.uint16) for t in tiles]).reshape(1, 8, n)
    ones = torch.ones(128, dtype=torch.float16, device=DEV)
    # a weight's input width is a multiple of 128: stack the tile row 8 times
    stacked = np.concatenate([trellis] * 8, axis=0)  # [8, 8, n]: in = 128, out = 128
    lin = X.Linear(dev_u16(stacked), ones, ones)
    w = host_u16(X.decode_matrix(lin.weight))
    for j, t in enumerate(tiles):
        got = w[0:16, 16 * j:16 * j + 16].reshape(-1)
        np.testing.assert_array_equal(got, np.array(t["expect"], np.uint16), err_msg=t["src"])


# ------------------------------------------------------- prepare / finish

@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("rows,shift", [(5, 0), (37, 0), (37, 1)])
def test_prepare_bit_exact(dtype, rows, shift):
    """37 rows of 4 blocks: the last group of 16 blocks is partly past the end;
    shift 1 starts x one element into its buffer (not 16-byte aligned), which
    takes the one-pair-per-lane kernel instead of the 16-byte one."""
    rng = np.random.default_rng(3)
    lin, _, suh, _ = make(rng, 512, 128, 64)
    x32 = (rng.standard_normal((rows, 512)) * 3).astype(np.float32)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    x = torch.from_numpy(x32).to(tdt)
    buf = torch.zeros(rows * 512 + shift, dtype=tdt, device=DEV)
    xd = buf[shift:].view(rows, 512)
    xd.copy_(x.to(DEV))
    assert (xd.data_ptr() % 16 == 0) == (shift == 0)
    xp = host_u16(X.prepare(lin.weight, xd))
    want = O.prepare(x.float().numpy(), suh)
    np.testing.assert_array_equal(xp, want)


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
def test_finish_bit_exact(dtype):
    rng = np.random.default_rng(4)
    lin, _, _, svh = make(rng, 128, 384, 64)
    z = rng.standard_normal((3, 384)).astype(np.float16).view(np.uint16)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    y = X.finish(lin.weight, dev_f16(z), dtype=tdt).cpu()
    want16 = torch.from_numpy(O.finish(z, svh).view(np.float16))
    assert torch.equal(y, want16.to(tdt)), (y - want16.to(tdt)).abs().max()


# ---------------------------------------------------------- inner product

def _inner_bar(xp_bits, w_bits, z_bits):
    """The reference's parity bar: per element against the exact f64 dot of
    the same decoded weights, |err| <= (2^-11 + depth 2^-24) sum|w x|."""
    xp = S.h2f(xp_bits).astype(np.float64)
    W = S.h2f(w_bits).astype(np.float64)
    exact = xp @ W
    mag = np.abs(xp) @ np.abs(W)
    depth = W.shape[0]
    err = np.abs(S.h2f(z_bits).astype(np.float64) - exact)
    return err <= (2.0 ** -11 + depth * 2.0 ** -24) * mag + 1e-30


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 8, 9, 31, 130])
@pytest.mark.parametrize("n", [32, 64, 96])
def test_inner_against_oracle(rows, n):
    rng = np.random.default_rng(rows * 131 + n)
    in_f, out_f = 512, 384
    lin, trellis, suh, _ = make(rng, in_f, out_f, n)
    x = S.activations(rng, rows, in_f)
    xp = O.prepare(x.astype(np.float32), suh)
    z = host_u16(X.inner(lin.weight, dev_f16(xp)))
    w = O.reconstruct_inner(trellis, in_f, out_f, n)
    assert _inner_bar(xp, w, z).all()
    zo = O.inner(trellis, xp, in_f, out_f, n)
    assert S.rel_fro(S.h2f(z), S.h2f(zo)) < 1e-3


@pytest.mark.parametrize("n", [16, 48, 80, 112, 128, 24, 40])
@pytest.mark.parametrize("rows", [1, 6, 20])
def test_inner_every_rate(n, rows):
    rng = np.random.default_rng(9 * n + rows)
    in_f, out_f = 384, 256
    lin, trellis, suh, _ = make(rng, in_f, out_f, n)
    xp = O.prepare(S.activations(rng, rows, in_f).astype(np.float32), suh)
    z = host_u16(X.inner(lin.weight, dev_f16(xp)))
    assert _inner_bar(xp, O.reconstruct_inner(trellis, in_f, out_f, n), z).all()


def test_inner_mcg_window():
    rng = np.random.default_rng(12)
    lin, trellis, suh, _ = make(rng, 256, 256, 48, "mcg", 12)
    for rows in (1, 4, 40):
        xp = O.prepare(S.activations(rng, rows, 256).astype(np.float32), suh)
        z = host_u16(X.inner(lin.weight, dev_f16(xp)))
        assert _inner_bar(xp, O.reconstruct_inner(trellis, 256, 256, 48, O.CB_MCG, 12), z).all()


# ----------------------------------------------------------------- matmul

@pytest.mark.parametrize("rows", [1, 2, 4, 8, 16, 200])
@pytest.mark.parametrize("k", [2, 3, 4, 5, 6, 8])
def test_matmul_against_fp64_reference(rows, k):
    rng = np.random.default_rng(100 * k + rows)
    in_f, out_f = 512, 256
    lin, trellis, suh, svh = make(rng, in_f, out_f, 16 * k)
    x = S.activations(rng, rows, in_f)
    y = lin(dev_f16(x)).float().cpu().numpy()
    Wt = S.public_weight(O.reconstruct_inner(trellis, in_f, out_f, 16 * k), suh, svh)
    want = x.astype(np.float64) @ Wt
    assert S.rel_fro(y, want) < 1e-3
    yo = S.h2f(O.project(x.astype(np.float32), trellis, suh, svh, in_f, out_f, 16 * k))
    assert S.rel_fro(y, yo) < 1e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_matmul_dtypes_and_leading_dims(dtype):
    rng = np.random.default_rng(5)
    lin, trellis, suh, svh = make(rng, 256, 256, 64)
    x = torch.from_numpy(rng.standard_normal((2, 3, 256)).astype(np.float32)).to(dtype)
    y = lin(x.to(DEV))
    assert y.shape == (2, 3, 256) and y.dtype == dtype
    yo = O.project(x.float().numpy().reshape(6, 256), trellis, suh, svh, 256, 256, 64)
    got = y.float().cpu().numpy().reshape(6, 256)
    if dtype == torch.bfloat16:
        # y16 then bf16: one bf16 rounding of a value within the f16 bar, so
        # each element is within one bf16 ulp (plus the f16 bar's absolute
        # share) of the oracle's y16 in bf16
        want = torch.from_numpy(S.h2f(yo)).to(dtype).float().numpy()
        ulp = np.spacing(np.abs(want)).astype(np.float64) * 2.0**16
        slack = 1e-3 * np.sqrt(np.mean(want.astype(np.float64) ** 2))
        err = np.abs(got - want) - ulp - slack
        i = np.unravel_index(np.argmax(err), err.shape)
        assert err[i] <= 0, (i, got[i], want[i], S.h2f(yo)[i])
        assert S.rel_fro(got, S.h2f(yo)) < 4e-3
    else:
        assert S.rel_fro(got, S.h2f(yo)) < 1e-3


def test_matmul_is_row_invariant():
    # a row's output bytes do not depend on how many rows share the call
    # within one kernel path (sushi_ds41/src/sushi/exl3/linear.zig:450-491)
    rng = np.random.default_rng(6)
    lin, *_ = make(rng, 512, 256, 64)
    x = dev_f16(S.activations(rng, 8, 512))
    full = lin(x)
    for r in (1, 3, 5, 8):
        assert torch.equal(lin(x[:r].contiguous()), full[:r])
    xg = dev_f16(S.activations(rng, 300, 512))
    big = lin(xg)
    assert torch.equal(lin(xg[:129].contiguous()), big[:129])


def test_matmul_qwen3_8b_shapes_k4():
    # BASELINE configs 0-1 at full size (K=4, q/o, k/v, gate/up, down), one
    # row per shape against the oracle's projection
    rng = np.random.default_rng(2048)
    for in_f, out_f in ((4096, 4096), (4096, 1024), (4096, 12288), (12288, 4096)):
        lin, trellis, suh, svh = make(rng, in_f, out_f, 64)
        x = S.activations(rng, 2, in_f)
        y = lin(dev_f16(x)).float().cpu().numpy()
        yo = S.h2f(O.project(x.astype(np.float32), trellis, suh, svh, in_f, out_f, 64))
        assert S.rel_fro(y, yo) < 1e-3, (in_f, out_f)


def test_gemm_full_size_sampled_rows():
    # prefill config: M=2048 rows through the GEMM; rows are independent, so
    # a sample of them is checked against the oracle
    rng = np.random.default_rng(4096)
    in_f, out_f = 4096, 4096
    lin, trellis, suh, svh = make(rng, in_f, out_f, 64)
    x = S.activations(rng, 2048, in_f)
    assert X.matmul_path(lin.weight, 2048) == "gemm"
    y = lin(dev_f16(x)).float().cpu().numpy()
    pick = np.array([0, 1, 127, 128, 1000, 2047])
    yo = S.h2f(O.project(x[pick].astype(np.float32), trellis, suh, svh, in_f, out_f, 64))
    assert S.rel_fro(y[pick], yo) < 1e-3


def test_gemm_beyond_32bit_activation_offsets():
    """Prefill activations past 4 GiB (270,000 rows x 8192 f16 = 4.4 GB): the
    GEMM kernel addresses a launch's activations with 32-bit offsets, so such
    calls run as windows of whole row tiles (261,888 rows of 16 KiB here; the
    last window of 8,112 rows splits k).  Rows on both sides of the window
    edge and of the 4 GiB offset against the oracle's projection, within the
    bar."""
    rng = np.random.default_rng(8192)
    in_f, out_f, n, rows = 8192, 256, 64, 270000
    assert rows * in_f * 2 > 1 << 32
    lin, trellis, suh, svh = make(rng, in_f, out_f, n)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(rows, in_f, generator=g, device=DEV, dtype=torch.float32).to(torch.float16)
    y = lin(x)
    torch.cuda.synchronize()
    sample = np.array([0, 1, 131071, 261887, 261888, 262143, 262144, 269999])
    xs = x[torch.from_numpy(sample).to(DEV)].cpu().numpy()
    got = y[torch.from_numpy(sample).to(DEV)].float().cpu().numpy()
    del x, y
    want = S.h2f(O.project(xs.astype(np.float32), trellis, suh, svh, in_f, out_f, n))
    assert S.rel_fro(got, want) < 1e-3
    assert S.row_rel(got, want).max() < 2e-3


@pytest.mark.parametrize("rows,in_f,out_f,n", [(17, 4096, 1024, 64), (128, 4096, 4096, 64),
                                               (300, 2048, 512, 48), (513, 1024, 256, 80)])
def test_gemm_split_k(rows, in_f, out_f, n):
    # grids of at most 128 tiles split k; a second launch adds the splits'
    # planes in split order, so the result is deterministic and within the bar
    rng = np.random.default_rng(rows + in_f)
    lin, trellis, suh, svh = make(rng, in_f, out_f, n)
    x = S.activations(rng, rows, in_f)
    assert X.matmul_path(lin.weight, rows) == "gemm"
    y1 = lin(dev_f16(x))
    y2 = lin(dev_f16(x))
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    pick = np.unique(np.array([0, 1, rows // 2, rows - 2, rows - 1]))
    yo = S.h2f(O.project(x[pick].astype(np.float32), trellis, suh, svh, in_f, out_f, n))
    assert S.rel_fro(y1.float().cpu().numpy()[pick], yo) < 1e-3


# --------------------------------------------------------------- loading

def test_load_tensor_from_a_source_and_refusals():
    rng = np.random.default_rng(8)
    trellis, suh, svh = S.linear(rng, 256, 128, 48)
    src = X.DictSource({"m.q.trellis": trellis.view(np.int16), "m.q.suh": suh.view(np.float16),
                        "m.q.svh": svh.view(np.float16),
                        "m.bad.trellis": trellis.view(np.int16), "m.bad.suh": suh.view(np.float16),
                        "m.bad.svh": svh[:64].view(np.float16)})
    L = X.Loader('{"format":"exl3","codebook":"mul1"}', src)
    assert L.opened.is_ok(), L.opened
    v, w = L.load_tensor("m.q", 256)
    assert v.is_ok(), v
    assert w.w.dims() == (16, 8, 48) and w.scales.dims() == (256,) and w.biases.dims() == (128,)
    x = S.activations(rng, 3, 256)
    y = X.matmul(w, dev_f16(x)).float().cpu().numpy()
    yo = S.h2f(O.project(x.astype(np.float32), trellis, suh, svh, 256, 128, 48))
    assert S.rel_fro(y, yo) < 1e-3
    v2, _ = L.load_tensor("m.q", 512)
    assert v2.code == X.UNSUPPORTED and "expected input width" in v2.reason
    v3, _ = L.load_tensor("m.bad")
    assert v3.code == X.UNSUPPORTED
    v4, _ = L.load_tensor("m.missing")
    assert v4.code == X.FAILED and v4.reason == "MissingWeight"
    X.release(w)
    assert w.priv is None and w.w.data is None
    L.close()


def test_load_from_safetensors_pack(tmp_path):
    # a pack on disk (written by the `safetensors` package): one linear and a
    # bank of three experts with its router, through exl3_safetensors_open
    st = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(81)
    trellis, suh, svh = S.linear(rng, 256, 128, 64)
    bank = [S.linear(rng, 256, 128, 64) for _ in range(3)]
    f1 = {"m.q.trellis": trellis.view(np.int16), "m.q.suh": suh.view(np.float16),
          "m.q.svh": svh.view(np.float16)}
    f2 = {"L.mlp.gate.weight": rng.standard_normal((3, 256)).astype(np.float16)}
    for e, (t, u, v) in enumerate(bank):
        f2[f"L.mlp.experts.{e}.gate_proj.trellis"] = t.view(np.int16)
        f2[f"L.mlp.experts.{e}.gate_proj.suh"] = u.view(np.float16)
        f2[f"L.mlp.experts.{e}.gate_proj.svh"] = v.view(np.float16)
    st.save_file(f1, str(tmp_path / "model-00001.safetensors"))
    st.save_file(f2, str(tmp_path / "model-00002.safetensors"))
    src = X.SafetensorsSource(sorted(tmp_path.glob("*.safetensors")))
    L = X.Loader('{"format":"exl3","codebook":"mul1"}', src)
    assert L.opened.is_ok(), L.opened
    v, w = L.load_tensor("m.q", 256)
    assert v.is_ok(), v
    x = S.activations(rng, 5, 256)
    y = X.matmul(w, dev_f16(x)).float().cpu().numpy()
    yo = S.h2f(O.project(x.astype(np.float32), trellis, suh, svh, 256, 128, 64))
    assert S.rel_fro(y, yo) < 1e-3
    vb, wb = L.load_bank("L.mlp.experts.gate_proj", 256)
    assert vb.is_ok(), vb
    assert wb.w.dims() == (3, 16, 8, 64)
    for e in range(3):
        got = host_u16(X.decode_matrix(wb, e))
        assert np.array_equal(got, O.reconstruct_inner(bank[e][0], 256, 128, 64)), e
    X.release(w)
    X.release(wb)
    L.close()
    src.close()


# -------------------------------------------------------------------- MoE

def _bank(rng, E, in_f, out_f, n):
    t, u, v = S.linear(rng, in_f, out_f, n, experts=E)
    w = X.wrap(dev_u16(t), dev_f16(u), dev_f16(v))
    return (t, u, v), w, w._keep  # the wrapped tensors themselves (the Weight holds them too)


@pytest.mark.parametrize("rows,limit", [(1, 0), (3, 0), (16, 0), (5, 10), (64, 0)])
def test_swiglu_routed_against_oracle(rows, limit):
    rng = np.random.default_rng(rows + 50 * limit)
    E, hidden, inter, topk, n = 8, 256, 128, 3, 48
    g_np, g, g_keep = _bank(rng, E, hidden, inter, n)
    u_np, u, u_keep = _bank(rng, E, hidden, inter, n)
    d_np, d, d_keep = _bank(rng, E, inter, hidden, n)
    x = (rng.standard_normal((rows, hidden)) * (20.0 if limit else 1.0)).astype(np.float16)
    inds, scores = O.route_topk(rng.standard_normal((rows, E)).astype(np.float32), topk)
    y = X.swiglu(g, u, d, dev_f16(x).reshape(rows, 1, hidden),
                 torch.from_numpy(inds).to(DEV).reshape(rows, 1, topk),
                 torch.from_numpy(scores).to(DEV).reshape(rows, 1, topk), limit=limit)
    want = O.moe_swiglu(x.astype(np.float32), g_np, u_np, d_np, inds, scores, hidden, inter, n,
                        limit=float(limit))
    assert S.rel_fro(y.float().cpu().numpy().reshape(rows, hidden), want) < 1e-3


@pytest.mark.parametrize("which", ["gate", "up"])
@pytest.mark.parametrize("rows", [1, 16, 200])
def test_swiglu_clamp_keeps_nan(rows, which):
    """The clamp passes a NaN through (turboexl3_ds41/src/exl3/kernels/exl3/
    q3_exl3_prep_gu_epi.metal:47-52): a NaN in expert 1's gate (or up) svh
    makes one column of its output NaN, and every row routed to expert 1
    must come out NaN (down's Hadamard spreads it), in the grouped GEMV
    (1, 16 rows) and the grouped GEMM (200 rows); the other rows within the
    bar of the oracle.  The dense MLP with the NaN weight: every row NaN."""
    rng = np.random.default_rng(4400 + rows)
    E, hidden, inter, topk, n, limit = 4, 256, 128, 2, 48, 10
    g_np = S.linear(rng, hidden, inter, n, experts=E)
    u_np = S.linear(rng, hidden, inter, n, experts=E)
    d_np = S.linear(rng, inter, hidden, n, experts=E)
    (g_np if which == "gate" else u_np)[2][1, 5] = 0x7E00
    banks = [X.wrap(dev_u16(t), dev_f16(su), dev_f16(sv)) for t, su, sv in (g_np, u_np, d_np)]
    x = S.activations(rng, rows, hidden)
    inds, scores = O.route_topk(rng.standard_normal((rows, E)).astype(np.float32), topk)
    inds[0, 0] = 1 if inds[0, 1] != 1 else inds[0, 0]  # row 0 routed to expert 1
    y = X.swiglu(*banks, dev_f16(x).reshape(rows, 1, hidden),
                 torch.from_numpy(inds).to(DEV).reshape(rows, 1, topk),
                 torch.from_numpy(scores).to(DEV).reshape(rows, 1, topk), limit=limit)
    got = y.float().cpu().numpy().reshape(rows, hidden)
    want = O.moe_swiglu(x.astype(np.float32), g_np, u_np, d_np, inds, scores, hidden, inter, n,
                        limit=float(limit))
    hit = (inds == 1).any(axis=1)
    assert hit[0] and np.isnan(want[hit]).all() and np.isfinite(want[~hit]).all()
    assert np.isnan(got[hit]).all()
    assert np.isfinite(got[~hit]).all()
    if (~hit).any():
        assert S.rel_fro(got[~hit], want[~hit]) < 1e-3
    # the dense MLP over expert 1's linears (GEMV prologue at <= 16 rows, the
    # GEMM and the elementwise SwiGLU above)
    lins = [X.Linear(dev_u16(t[1]), dev_f16(su[1]), dev_f16(sv[1])) for t, su, sv in (g_np, u_np, d_np)]
    yd = X.swiglu(*(l.weight for l in lins), dev_f16(x), limit=limit).float().cpu().numpy()
    assert np.isnan(yd).all()


@pytest.mark.parametrize("E,topk,rows,limit", [(4, 2, 128, 0), (2, 1, 600, 0), (3, 2, 200, 7)])
def test_swiglu_routed_prefill_sizes(E, topk, rows, limit):
    # prefill-sized expert batches (32+ slots per expert on average, an
    # expert past 256 slots): the grouped GEMM over routed items of <= 256
    # slots, against the oracle's composition
    rng = np.random.default_rng(E * 1000 + rows + limit)
    hidden, inter, n = 512, 256, 48
    g_np, g, g_keep = _bank(rng, E, hidden, inter, n)
    u_np, u, u_keep = _bank(rng, E, hidden, inter, n)
    d_np, d, d_keep = _bank(rng, E, inter, hidden, n)
    x = (rng.standard_normal((rows, hidden)) * (20.0 if limit else 1.0)).astype(np.float16)
    inds, scores = O.route_topk(rng.standard_normal((rows, E)).astype(np.float32), topk)
    y = X.swiglu(g, u, d, dev_f16(x).reshape(rows, 1, hidden),
                 torch.from_numpy(inds).to(DEV).reshape(rows, 1, topk),
                 torch.from_numpy(scores).to(DEV).reshape(rows, 1, topk), limit=limit)
    want = O.moe_swiglu(x.astype(np.float32), g_np, u_np, d_np, inds, scores, hidden, inter, n,
                        limit=float(limit))
    assert S.rel_fro(y.float().cpu().numpy().reshape(rows, hidden), want) < 1e-3


def test_swiglu_verify_rows_takes_the_decode_chain():
    """verify_rows (the reference sends verify rows down its decode chain at
    any batch, sushi_ds41/src/sushi/exl3/root.zig:149): at 64 slots per
    expert, where a call takes the grouped GEMM, it takes the grouped GEMV
    items instead -- the same values, bit for bit, as the rows split into
    calls small enough for the GEMV items -- within the bar of the oracle."""
    rng = np.random.default_rng(77)
    E, hidden, inter, topk, n, rows = 4, 256, 128, 2, 48, 128
    g_np, g, g_keep = _bank(rng, E, hidden, inter, n)
    u_np, u, u_keep = _bank(rng, E, hidden, inter, n)
    d_np, d, d_keep = _bank(rng, E, inter, hidden, n)
    x = S.activations(rng, rows, hidden)
    inds, scores = O.route_topk(rng.standard_normal((rows, E)).astype(np.float32), topk)
    assert X.swiglu_path(g, u, d, rows, topk) == "routed-gemm"
    assert X.swiglu_path(g, u, d, rows, topk, verify_rows=True) == "routed-gemv"
    xd, ids, scs = dev_f16(x), torch.from_numpy(inds).to(DEV), torch.from_numpy(scores).to(DEV)

    def call(a, b, verify):
        return X.swiglu(g, u, d, xd[a:b].reshape(b - a, 1, hidden), ids[a:b].reshape(b - a, 1, topk),
                        scs[a:b].reshape(b - a, 1, topk), verify_rows=verify).reshape(b - a, hidden)

    yv = call(0, rows, True)
    part = rows // 4  # 64 slots: below 32 per expert, the GEMV items without the flag
    assert X.swiglu_path(g, u, d, part, topk) == "routed-gemv"
    assert torch.equal(yv, torch.cat([call(a, a + part, False) for a in range(0, rows, part)]))
    want = O.moe_swiglu(x.astype(np.float32), g_np, u_np, d_np, inds, scores, hidden, inter, n)
    assert S.rel_fro(yv.float().cpu().numpy(), want) < 1e-3
    assert S.rel_fro(call(0, rows, False).float().cpu().numpy(), want) < 1e-3


def test_swiglu_routed_long_splits():
    # enough experts and columns that the planner gives the gate+up launch
    # 256-tile splits (the most a work item takes: 32 blocks of its rows),
    # items of up to 4 slots; against the oracle's composition
    rng = np.random.default_rng(77)
    E, hidden, inter, topk, n, rows = 40, 4096, 1024, 8, 48, 8
    g_np, g, g_keep = _bank(rng, E, hidden, inter, n)
    u_np, u, u_keep = _bank(rng, E, hidden, inter, n)
    d_np, d, d_keep = _bank(rng, E, inter, hidden, n)
    x = rng.standard_normal((rows, hidden)).astype(np.float16)
    inds, scores = O.route_topk(rng.standard_normal((rows, E)).astype(np.float32), topk)
    y = X.swiglu(g, u, d, dev_f16(x).reshape(rows, 1, hidden),
                 torch.from_numpy(inds).to(DEV).reshape(rows, 1, topk),
                 torch.from_numpy(scores).to(DEV).reshape(rows, 1, topk))
    want = O.moe_swiglu(x.astype(np.float32), g_np, u_np, d_np, inds, scores, hidden, inter, n)
    assert S.rel_fro(y.float().cpu().numpy().reshape(rows, hidden), want) < 1e-3


@pytest.mark.parametrize("rows,limit,n,dtype", [(1, 0, 64, "f16"), (3, 7, 48, "f16"),
                                                (16, 0, 64, "f16"), (2, 0, 64, "bf16"),
                                                (5, 3, 32, "f32"), (24, 0, 64, "f16"),
                                                (300, 5, 48, "f16"), (64, 0, 64, "bf16")])
def test_swiglu_dense_decode_sizes(rows, limit, n, dtype):
    # the dense MLP (inds empty): up to 16 rows take gate+up in one GEMV and
    # the down GEMV with the SwiGLU in its prepare; more rows take the GEMM
    # for the three linears and the SwiGLU between; both against the
    # oracle's composition (clamp included)
    rng = np.random.default_rng(700 + rows + limit)
    hidden, inter = 512, 1024
    tg, sg, vg = S.linear(rng, hidden, inter, n)
    tu, su, vu = S.linear(rng, hidden, inter, n)
    td, sd, vd = S.linear(rng, inter, hidden, n)
    G = X.Linear(dev_u16(tg), dev_f16(sg), dev_f16(vg))
    U = X.Linear(dev_u16(tu), dev_f16(su), dev_f16(vu))
    D = X.Linear(dev_u16(td), dev_f16(sd), dev_f16(vd))
    x = S.activations(rng, rows, hidden)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    xd = torch.from_numpy(x.astype(np.float32)).to(DEV).to(tdt)
    y = X.swiglu(G.weight, U.weight, D.weight, xd, limit=limit)
    assert y.dtype == tdt and y.shape == (rows, hidden)
    want = O.moe_swiglu(xd.float().cpu().numpy(), (tg[None], sg[None], vg[None]),
                        (tu[None], su[None], vu[None]), (td[None], sd[None], vd[None]),
                        np.zeros((rows, 1), np.int32), np.ones((rows, 1), np.float32), hidden,
                        inter, n, limit=float(limit))
    got = y.float().cpu().numpy()
    if dtype == "bf16":
        # f16 result then bf16: three chained linears' f16 roundings (in
        # another summation order) move elements by a few f16 ulps, which can
        # cross bf16 rounding boundaries, so each element is within two bf16
        # ulps plus 4e-3 of the rms of the oracle's value in bf16, and the
        # whole within 4e-3 (the bf16 output's own rounding is 2^-9 relative)
        wb = torch.from_numpy(want).to(tdt).float().numpy()
        ulp = np.spacing(np.abs(wb)).astype(np.float64) * 2.0**16
        slack = 4e-3 * np.sqrt(np.mean(wb.astype(np.float64) ** 2))
        assert (np.abs(got - wb) - 2 * ulp - slack).max() <= 0
        assert S.rel_fro(got, want) < 4e-3
    else:
        assert S.rel_fro(got, want) < 1e-3


def test_swiglu_dense_shared_expert():
    rng = np.random.default_rng(31)
    hidden, inter, n = 256, 256, 64
    tg, sg, vg = S.linear(rng, hidden, inter, n)
    tu, su, vu = S.linear(rng, hidden, inter, n)
    td, sd, vd = S.linear(rng, inter, hidden, n)
    G = X.Linear(dev_u16(tg), dev_f16(sg), dev_f16(vg))
    U = X.Linear(dev_u16(tu), dev_f16(su), dev_f16(vu))
    D = X.Linear(dev_u16(td), dev_f16(sd), dev_f16(vd))
    x = S.activations(rng, 4, hidden)
    y = X.swiglu(G.weight, U.weight, D.weight, dev_f16(x)).float().cpu().numpy()
    want = O.moe_swiglu(x.astype(np.float32), (tg[None], sg[None], vg[None]), (tu[None], su[None], vu[None]),
                        (td[None], sd[None], vd[None]), np.zeros((4, 1), np.int32),
                        np.ones((4, 1), np.float32), hidden, inter, n)
    assert S.rel_fro(y, want) < 1e-3


# ------------------------------------------------------- shared-input linears

@pytest.mark.parametrize("rows", [1, 3, 16, 40])
def test_matmul_shared_against_oracle(rows):
    # q/k/v-like linears reading the same rows in one launch
    # (sushi_ds41/src/sushi/exl3/linear.zig:34-60)
    rng = np.random.default_rng(600 + rows)
    in_f, n = 512, 48
    outs = (256, 128, 384)
    lins, parts = [], []
    for o in outs:
        lin, t, u, v = make(rng, in_f, o, n)
        lins.append(lin)
        parts.append((t, u, v, o))
    x = S.activations(rng, rows, in_f)
    ys = X.matmul_shared([l.weight for l in lins], dev_f16(x))
    for y, (t, u, v, o) in zip(ys, parts):
        yo = S.h2f(O.project(x.astype(np.float32), t, u, v, in_f, o, n))
        assert y.shape == (rows, o)
        assert S.rel_fro(y.float().cpu().numpy(), yo) < 1e-3


def test_matmul_shared_refuses_mixed_rates():
    rng = np.random.default_rng(601)
    a, *_ = make(rng, 256, 128, 48)
    b, *_ = make(rng, 256, 128, 64)
    with pytest.raises(X.Exl3Error, match="differ"):
        X.matmul_shared([a.weight, b.weight], dev_f16(S.activations(rng, 1, 256)))


# ------------------------------------------------------------ scratch lifetime

def test_scratch_growth_keeps_captured_graphs_valid():
    """A graph captured on a stream keeps working after a larger eager call
    on the same stream grows the library's scratch (the old buffers are kept,
    not freed); growing while capturing is refused by name; releasing the
    stream's scratch afterwards leaves later calls working."""
    rng = np.random.default_rng(900)
    small, *_ = make(rng, 512, 256, 64)
    big, *_ = make(rng, 4096, 4096, 64)
    xs = dev_f16(S.activations(rng, 1, 512))
    xb = dev_f16(S.activations(rng, 16, 4096))
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    ys = torch.empty(1, 256, dtype=torch.float16, device=DEV)
    with torch.cuda.stream(cap):
        small(xs, out=ys, stream=cap)
        want = ys.clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap, capture_error_mode="thread_local"):
        small(xs, out=ys, stream=cap)
    # a larger call on the capture stream: its scratch grows past the graph's
    with torch.cuda.stream(cap):
        yb = big(xb, stream=cap)
    torch.cuda.synchronize()
    for _ in range(3):
        ys.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys, want)
    # growing inside a capture is refused before anything is recorded
    s2 = torch.cuda.Stream()
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(X.Exl3Error, match="captured"):
        with torch.cuda.graph(g2, stream=s2, capture_error_mode="thread_local"):
            big(xb, stream=s2)
    del g
    X.scratch_release(0, cap)
    with torch.cuda.stream(cap):
        again = big(xb, stream=cap)
    torch.cuda.synchronize()
    assert torch.equal(again, yb)


def test_splitk_give_up_is_reported_and_recovered():
    """A split-K wait that gives up leaves NaN in its output and sets the
    stream's status; exl3_stream_status reports it and resets the slots,
    after which calls are exact again.  The give-up is forced from the host:
    the splits other than the last skip their partial-sum stores (the test
    hook exl3_set_splitk_test_drop) and the wait's bound is 8 polls, so the
    last split's wait gives up every time and every kernel exits normally."""
    rng = np.random.default_rng(901)
    lin, *_ = make(rng, 4096, 4096, 64)  # 8 splits at batch 1
    x = dev_f16(S.activations(rng, 1, 4096))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        want = lin(x, stream=s)
    torch.cuda.synchronize()
    assert X.stream_status(0, s).is_ok()
    try:
        X.lib().exl3_set_splitk_poll_bound(8)
        X.lib().exl3_set_splitk_test_drop(1)
        with torch.cuda.stream(s):
            y = lin(x, stream=s)
        v = X.stream_status(0, s)
    finally:
        X.lib().exl3_set_splitk_test_drop(0)
        X.lib().exl3_set_splitk_poll_bound(-1)
    assert v.code == X.FAILED and "did not arrive" in v.reason
    assert torch.isnan(y.float()).all()  # every column group's wait gave up
    assert X.stream_status(0, s).is_ok()  # reported once, then reset
    for _ in range(3):
        with torch.cuda.stream(s):
            again = lin(x, stream=s)
        assert X.stream_status(0, s).is_ok()
        assert torch.equal(again, want)
