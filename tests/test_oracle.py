"""Pins the CPU oracle (oracle/exl3_oracle.c) before anything is compared to it.

Each check reaches the answer by a route other than the oracle's own code:
the reference's golden digests and fixture tiles (copied as data into
tests/golden/reference_golden.json), its known-answer values, the bit-by-bit
definition of the stream, closed forms evaluated with numpy, and textbook
identities of the Hadamard transform.  Planted mistakes (on the CPU) show the
checks fail when the arithmetic is wrong.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import scipy.linalg

from oracle import oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_golden.json")))


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).astype("<u2").tobytes()).hexdigest()


# ---------------------------------------------------------------- codebooks

def test_mul1_table_matches_manifest_digest():
    # turboexl3_ds41/src/exl3/kernels/exl3/manifest.json golden.mul1_table
    assert sha(O.mul1_table()) == GOLD["mul1_table_sha256"]


def test_mul1_known_answers():
    # sushi_ds41/src/sushi/exl3/expert_exl3.zig:699-704
    for cw, want in GOLD["kat_mul1"].items():
        assert O.decode_mul1(int(cw)) == want


def test_mul1_closed_form_in_f64_agrees_on_every_state():
    # ds41/src/exl3/kernels.zig:966-975 states the value is exact in f64 and
    # rounds once; numpy's f64 -> f16 cast is one nearest-even rounding.
    cw = np.arange(65536, dtype=np.uint64)
    x = (cw * 0x83DCD12D) & 0xFFFFFFFF
    s = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + (x >> 24)
    inv = float(np.array([0x1EEE], np.uint16).view(np.float16)[0])
    bias = float(np.array([0xC931], np.uint16).view(np.float16)[0])
    want = ((1024.0 + s.astype(np.float64)) * inv + bias).astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(O.mul1_table(), want)


def test_mul1_table_digest_catches_a_wrong_multiplier():
    bad = np.arange(65536, dtype=np.uint64)
    x = (bad * 0x83DCD12F) & 0xFFFFFFFF  # planted: one bit of the multiplier
    s = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + (x >> 24)
    vals = ((1024.0 + s) * 0.0067672729 - 10.3828125).astype(np.float16).view(np.uint16)
    assert sha(vals) != GOLD["mul1_table_sha256"]


def test_mcg_closed_form_every_state():
    # sushi_ds41/src/sushi/exl3/expert_exl3.zig:267-273 (and its cw = 0 test :853-862)
    cw = np.arange(65536, dtype=np.uint64)
    p = (0x3B603B60 ^ ((cw * 0xCBAC1FED) & 0x8FFF8FFF)).astype(np.uint32)
    lo = (p & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (p >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    want = (lo + hi).astype(np.float16).view(np.uint16)
    got = O.mcg_table()
    np.testing.assert_array_equal(got, want)
    # survey-computed digest of the same table (not a reference-held value)
    assert sha(got) == "95383563929baa9d1ae5de0be22490284382673620bdd85929feea7bdbef04a9"


# ------------------------------------------------------- table codebooks

TABLES = GOLD["codebook_tables"]
TABLE_IDS = {name: t for t, name in O.TABLE_NAMES.items()}


def table_digest(fields, ns, rows) -> str:
    # sushi_ds41/src/sushi/exl3/codebook_tables.zig:230-247: sha256 over one
    # line per row, "<n>,<field as 8 lowercase hex digits>,...\n", first 8 hex
    text = "".join(f"{n}," + ",".join(f"{v:08x}" for v in r[:fields]) + "\n" for n, r in zip(ns, rows))
    return hashlib.sha256(text.encode()).hexdigest()[:8]


def table_rows(table):
    n_lo, count, fields = O.table_info(table)
    ns = [n_lo + 2 * i for i in range(count)]
    return fields, ns, [O.table_row(table, n) for n in ns]


def test_table_digest_function_against_the_fixed_vector():
    v = TABLES["digest_vector"]
    assert table_digest(v["fields"], v["ns"], v["rows"]) == v["digest"]


@pytest.mark.parametrize("name", ["pair1-w16-v1", "spec1-w15", "spec1-w16", "std1"])
def test_codebook_tables_match_their_pinned_digests(name):
    # every constant of every row is under the reference's pinned digest
    fields, ns, rows = table_rows(TABLE_IDS[name])
    assert table_digest(fields, ns, rows) == TABLES["digests"][name]
    for n, want in TABLES["rows"].get(name, {}).items():
        assert O.table_row(TABLE_IDS[name], int(n))[:len(want)] == tuple(want), (name, n)
    for n in TABLES["no_row"].get(name, []):
        assert O.table_row(TABLE_IDS[name], n) is None, (name, n)
    assert all(O.table_row(TABLE_IDS[name], n) is None for n in range(ns[0] + 1, ns[-1], 2))


def test_spec1_w15_extends_its_superseded_version():
    # codebook_tables.zig:444-448: rows n = 24..64 are the table of digest 2ac2594d
    fields, ns, rows = table_rows(O.TAB_SPEC1_W15)
    keep = [(n, r) for n, r in zip(ns, rows) if 24 <= n <= 64]
    assert table_digest(fields, [n for n, _ in keep], [r for _, r in keep]) == TABLES["superseded"]["spec1-w15"][0]


def test_table_digest_catches_a_changed_constant():
    fields, ns, rows = table_rows(O.TAB_PAIR1_W16_V1)
    rows = [list(r) for r in rows]
    rows[3][0] = (rows[3][0] + 1) & 0xFFFFFFFF  # codebook_tables.zig:310-318's mutation
    assert table_digest(fields, ns, rows) != TABLES["digests"]["pair1-w16-v1"]


def test_hash_mask_known_answers():
    k = GOLD["kat_hash_mask"]
    for cw, want in k["values"].items():
        assert O.decode_hash_mask(int(cw), k["mult"], k["mask"]) == want, cw


def test_hash_mask_closed_form_every_state():
    # halfSumScaled (expert_exl3.zig:288-295) evaluated in float64: the exact
    # half sum rounded once to f16 equals the f32 sum rounded (24 >= 2 * 11 + 2
    # bits), and * 4096 is exact
    for table, n in ((O.TAB_STD1, 40), (O.TAB_SPEC1_W15, 16), (O.TAB_SPEC1_W15, 128)):
        mult, mask = O.table_row(table, n)[:2]
        cw = np.arange(65536, dtype=np.uint64)
        p = ((cw * mult) & mask).astype(np.uint32)
        lo = (p & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
        hi = (p >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
        want = ((lo + hi).astype(np.float16).astype(np.float64) * 4096.0).astype(np.float16).view(np.uint16)
        got = np.array([O.decode_hash_mask(c, mult, mask) for c in range(0, 65536, 7)], np.uint16)
        np.testing.assert_array_equal(got, want[::7])


def test_pair1_known_answers():
    for n, cw, w0, w1 in GOLD["kat_pair1"]:
        assert O.decode_pair1(cw, O.table_row(O.TAB_PAIR1_W16_V1, n)) == (w0, w1), (n, cw)


def test_pair1_kats_catch_a_rotation_the_other_way():
    # planted on the CPU: rotr instead of rotl fails the reference's values
    bad = 0
    for n, cw, w0, w1 in GOLD["kat_pair1"]:
        row = list(O.table_row(O.TAB_PAIR1_W16_V1, n))
        row[1] = (32 - row[1]) % 32
        bad += O.decode_pair1(cw, row) != (w0, w1)
    assert bad > 10


def test_table_tiles_decode_codeword_by_codeword():
    # spec1 / std1 tiles: each codeword decoded on its own through the pinned
    # unpack and permutation; pair1: slots 2j and 2j+1 from codeword 2j+1
    # (expert_exl3.zig:338-357; the reference's own pair1 tile fixture,
    # fixtures/exl3_pair1_tiles.safetensors, is not in its tree)
    rng = np.random.default_rng(31)
    perm = O.tile_perm()
    for cb, table, n, window in ((O.spec1(O.TAB_SPEC1_W15), O.TAB_SPEC1_W15, 40, 15),
                                 (O.spec1(O.TAB_SPEC1_W16), O.TAB_SPEC1_W16, 64, 16),
                                 (O.CB_STD1, O.TAB_STD1, 24, 12),
                                 (O.CB_PAIR1, O.TAB_PAIR1_W16_V1, 48, 16)):
        words = rng.integers(0, 65536, n, dtype=np.uint16)
        got = O.decode_tile(words, n, cb, window)
        cws = O.unpack_tile(words, n, bitwise=True) & ((1 << window) - 1)
        row = O.table_row(table, n)
        want = np.empty(256, np.uint16)
        if cb == O.CB_PAIR1:
            for j in range(128):
                want[perm[2 * j]], want[perm[2 * j + 1]] = O.decode_pair1(int(cws[2 * j + 1]), row)
        else:
            for i in range(256):
                want[perm[i]] = O.decode_hash_mask(int(cws[i]), row[0], row[1])
        np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------------- rates

@pytest.mark.parametrize("n", ["40", "44", "48", "64"])
def test_bit_end_tables(n):
    # sushi_ds41/src/sushi/exl3/expert_exl3.zig:661-697
    kat = GOLD["kat_bit_end"][n]
    nn = int(n)
    assert [O.bit_end(nn, i) for i in range(8)] == kat["ends"]
    fresh = [O.bit_end(nn, i) - (O.bit_end(nn, i - 1) if i else 0) for i in range(16)]
    assert fresh == kat["fresh"]
    assert O.bit_end(nn, 255) == 16 * nn


@pytest.mark.parametrize("n", [24, 40])
def test_fractional_bit_ends_follow_the_ring_rule(n):
    # turboexl3_ds41/src/frac_test.zig:46-57: KA or KA+1 fresh bits by mask 0xAAAA
    s = 0
    for i in range(256):
        s += n // 16 + ((0xAAAA >> (i % 16)) & 1)
        assert O.bit_end(n, i) == s


# -------------------------------------------------------- bitstream / tiles

def test_unpack_matches_bitwise_definition_every_even_rate():
    # sushi_ds41/src/sushi/exl3/expert_exl3.zig:1051-1090
    rng = np.random.default_rng(0x51555348)
    for n in range(16, 129, 2):
        for _ in range(4):
            words = rng.integers(0, 65536, n, dtype=np.uint16)
            np.testing.assert_array_equal(O.unpack_tile(words, n), O.unpack_tile(words, n, bitwise=True))


def test_tile_perm_is_a_permutation_and_chunks_are_two_columns():
    perm = O.tile_perm().astype(int)
    assert sorted(perm) == list(range(256))
    for a in range(8):
        cols = {p % 16 for p in perm[32 * a:32 * a + 32]}
        rows = {p // 16 for p in perm[32 * a:32 * a + 32]}
        assert cols == {a, a + 8} and rows == set(range(16))


def test_frac_tiles_decode_as_the_reference_fixture():
    # turboexl3_ds41/src/frac_tiles.json through frac_test.zig:23-44 (n 24/32/40/48)
    seen = {}
    for t in GOLD["frac_tiles"]:
        got = O.decode_tile(np.array(t["words"], np.uint16), t["n"])
        np.testing.assert_array_equal(got, np.array(t["expect"], np.uint16), err_msg=t["src"])
        seen[t["n"]] = seen.get(t["n"], 0) + 1
    assert all(seen[n] >= 14 for n in (24, 32, 40, 48))


def test_frac_tile_fixture_catches_a_transposed_tile():
    t = GOLD["frac_tiles"][0]
    got = O.decode_tile(np.array(t["words"], np.uint16), t["n"]).reshape(16, 16).T.reshape(-1)
    assert not np.array_equal(got, np.array(t["expect"], np.uint16))


@pytest.mark.parametrize("name", ["gate_up", "down", "gate_up_k2", "down_k2"])
def test_golden_planes(name):
    # manifest golden.planes: seeded code (splitmix64) and W_hat digests
    p = GOLD["planes"][name]
    n = 16 * p["K"]
    code = O.synth_plane(p["seed"], (p["in"] // 16) * (p["out"] // 16) * n)
    assert sha(code) == p["code_sha256"]
    w = O.reconstruct_inner(code, p["in"], p["out"], n)
    assert sha(w) == p["w_hat_sha256"]


def test_golden_plane_digest_catches_a_swapped_tile_order():
    p = GOLD["planes"]["gate_up_k2"]
    n = 32
    code = O.synth_plane(p["seed"], (p["in"] // 16) * (p["out"] // 16) * n)
    # planted: tiles read [out/16][in/16] instead of [in/16][out/16]
    it, ot = p["in"] // 16, p["out"] // 16
    swapped = code.reshape(it, ot, n).transpose(1, 0, 2).reshape(-1)
    w = O.reconstruct_inner(swapped, p["in"], p["out"], n)
    assert sha(w) != p["w_hat_sha256"]


def test_window_masks_the_codeword_before_decode():
    # sushi_ds41/src/sushi/exl3/expert_exl3.zig:1015-1039
    rng = np.random.default_rng(3)
    perm = O.tile_perm()
    words = rng.integers(0, 65536, 40, dtype=np.uint16)
    cws = O.unpack_tile(words, 40)
    wide = O.decode_tile(words, 40, O.CB_MCG, 16)
    for w in (8, 10, 12, 15):
        got = O.decode_tile(words, 40, O.CB_MCG, w)
        want = np.empty(256, np.uint16)
        want[perm] = [O.decode_mcg(int(c) & ((1 << w) - 1)) for c in cws]
        np.testing.assert_array_equal(got, want)
        assert not np.array_equal(got, wide)


# ---------------------------------------------------------------- Hadamard

def test_hadamard_forms_match_sylvester_matrix():
    H = scipy.linalg.hadamard(128).astype(np.float64)
    rng = np.random.default_rng(1)
    v = rng.standard_normal(128).astype(np.float32)
    want = H @ v.astype(np.float64)
    np.testing.assert_allclose(O.hadamard128(v, dense=False), want, rtol=0, atol=1e-4)
    np.testing.assert_allclose(O.hadamard128(v, dense=True), want / np.sqrt(128), rtol=0, atol=1e-5)


def test_hadamard_is_an_involution_up_to_scale():
    rng = np.random.default_rng(2)
    v = rng.standard_normal(128).astype(np.float32)
    twice = O.hadamard128(O.hadamard128(v, dense=False), dense=False)
    np.testing.assert_allclose(twice, 128 * v, rtol=1e-5, atol=1e-4)


# ------------------------------------------------------- prepare / finish

def _rand_linear(rng, in_f, out_f, k):
    n = 16 * k
    trellis = rng.integers(0, 65536, (in_f // 16, out_f // 16, n), dtype=np.uint16)
    suh = np.where(rng.random(in_f) < 0.5, -1.0, 1.0).astype(np.float16).view(np.uint16)
    sv = np.where(rng.random(out_f) < 0.5, -1.0, 1.0) * rng.uniform(0.5, 1.5, out_f) * 0.02
    svh = sv.astype(np.float16).view(np.uint16)
    return trellis, suh, svh, n


def test_prepare_and_finish_against_float64_matrix_route():
    rng = np.random.default_rng(5)
    in_f, out_f = 256, 384
    _, suh, svh, _ = _rand_linear(rng, in_f, out_f, 4)
    x = rng.standard_normal((3, in_f)).astype(np.float32)
    H = scipy.linalg.hadamard(128) / np.sqrt(128)
    xs = x.astype(np.float16).astype(np.float64) * O.h2f(suh)
    want = np.concatenate([xs[:, b:b + 128] @ H for b in range(0, in_f, 128)], axis=1)
    for dense in (False, True):
        got = O.h2f(O.prepare(x, suh, dense=dense)).astype(np.float64)
        # one f16 rounding (half an ulp, 2^-11 relative) plus f32 butterfly error
        assert np.all(np.abs(got - want) <= 2 ** -11 * np.abs(want) + 1e-5)
    z = rng.standard_normal((3, out_f)).astype(np.float16).view(np.uint16)
    zf = O.h2f(z).astype(np.float64)
    want = np.concatenate([zf[:, b:b + 128] @ H for b in range(0, out_f, 128)], axis=1) * O.h2f(svh)
    for dense in (False, True):
        got = O.h2f(O.finish(z, svh, dense=dense)).astype(np.float64)
        assert np.all(np.abs(got - want) <= 2 ** -11 * np.abs(want) + 1e-7)


@pytest.mark.parametrize("k", [2, 3, 4, 5, 6, 8])
def test_project_equals_dense_public_weight(k):
    # sushi_ds41/src/sushi/exl3/expert_exl3.zig:864-915: project vs x @ W_public
    rng = np.random.default_rng(10 + k)
    in_f, out_f = 256, 256
    trellis, suh, svh, n = _rand_linear(rng, in_f, out_f, k)
    x = rng.standard_normal((2, in_f)).astype(np.float32)
    y = O.h2f(O.project(x, trellis, suh, svh, in_f, out_f, n)).astype(np.float64)
    # independent route: W_inner from the decode, rotations as float64 matrices
    W = O.h2f(O.reconstruct_inner(trellis, in_f, out_f, n)).astype(np.float64)
    H = scipy.linalg.hadamard(128) / np.sqrt(128)
    Hi = np.kron(np.eye(in_f // 128), H)
    Ho = np.kron(np.eye(out_f // 128), H)
    Wt = np.diag(O.h2f(suh).astype(np.float64)) @ Hi @ W @ Ho @ np.diag(O.h2f(svh).astype(np.float64))
    want = x.astype(np.float16).astype(np.float64) @ Wt
    rel = np.linalg.norm(y - want) / np.linalg.norm(want)
    assert rel < 1e-3
    # and the reference's own dense route (reconstructPublic) agrees with it
    Wp = O.h2f(O.reconstruct_public(trellis, suh, svh, in_f, out_f, n)).astype(np.float64)
    assert np.linalg.norm(Wp - Wt) / np.linalg.norm(Wt) < 1e-3


def test_project_parity_bar_fails_on_a_planted_sign_error():
    rng = np.random.default_rng(77)
    in_f, out_f = 128, 128
    trellis, suh, svh, n = _rand_linear(rng, in_f, out_f, 4)
    x = rng.standard_normal((1, in_f)).astype(np.float32)
    y = O.h2f(O.project(x, trellis, suh, svh, in_f, out_f, n)).astype(np.float64)
    bad_suh = suh.copy()
    bad_suh[17] ^= 0x8000  # planted: one flipped input sign
    yb = O.h2f(O.project(x, trellis, bad_suh, svh, in_f, out_f, n)).astype(np.float64)
    assert np.linalg.norm(y - yb) / np.linalg.norm(y) > 1e-3


# --------------------------------------------------------------------- MoE

def test_route_topk_against_numpy():
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((5, 64)).astype(np.float32)
    inds, scores = O.route_topk(logits, 8)
    for r in range(5):
        order = np.argsort(-logits[r], kind="stable")[:8]
        np.testing.assert_array_equal(inds[r], order)
        e = np.exp(logits[r, order].astype(np.float64) - logits[r].max())
        np.testing.assert_allclose(scores[r], e / e.sum(), rtol=1e-5)


@pytest.mark.parametrize("limit", [0.0, 10.0])
def test_moe_swiglu_against_composed_projections(limit):
    rng = np.random.default_rng(21)
    E, hidden, inter, k = 4, 256, 128, 2
    gate = [np.stack(z) for z in zip(*[_rand_linear(rng, hidden, inter, 3)[:3] for _ in range(E)])]
    up = [np.stack(z) for z in zip(*[_rand_linear(rng, hidden, inter, 3)[:3] for _ in range(E)])]
    down = [np.stack(z) for z in zip(*[_rand_linear(rng, inter, hidden, 3)[:3] for _ in range(E)])]
    x = (rng.standard_normal((2, hidden)) * (40.0 if limit else 1.0)).astype(np.float32)
    inds, scores = O.route_topk(rng.standard_normal((2, E)).astype(np.float32), k)
    y = O.moe_swiglu(x, gate, up, down, inds, scores, hidden, inter, 48, limit=limit)
    want = np.zeros((2, hidden))
    for r in range(2):
        for j in range(k):
            e = inds[r, j]
            g = O.h2f(O.project(x[r], gate[0][e], gate[1][e], gate[2][e], hidden, inter, 48))[0].astype(np.float64)
            u = O.h2f(O.project(x[r], up[0][e], up[1][e], up[2][e], hidden, inter, 48))[0].astype(np.float64)
            if limit:
                g = np.minimum(g, limit)
                u = np.clip(u, -limit, limit)
            h = g / (1 + np.exp(-g)) * u
            d = O.h2f(O.project(h.astype(np.float32), down[0][e], down[1][e], down[2][e], inter, hidden, 48))
            want[r] += scores[r, j] * d[0]
    np.testing.assert_allclose(y, want, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("which", ["gate", "up"])
def test_moe_clamp_keeps_nan(which):
    """The clamp of mtl/q3_exl3_prep_gu_epi.metal:47-52 passes a NaN through
    (isnan(g) ? g : min(g, limit), the same for up's two bounds): one NaN
    column of expert 1's gate (or up) output, forced by a NaN in its svh,
    makes every row routed to expert 1 NaN through down's Hadamard, under a
    clamp; a clamp that turned NaN into a bound would leave them finite.
    Rows not routed to expert 1 stay finite."""
    rng = np.random.default_rng(33)
    E, hidden, inter, k, rows = 4, 256, 128, 2, 6
    gate = [np.stack(z) for z in zip(*[_rand_linear(rng, hidden, inter, 3)[:3] for _ in range(E)])]
    up = [np.stack(z) for z in zip(*[_rand_linear(rng, hidden, inter, 3)[:3] for _ in range(E)])]
    down = [np.stack(z) for z in zip(*[_rand_linear(rng, inter, hidden, 3)[:3] for _ in range(E)])]
    bank = gate if which == "gate" else up
    bank[2][1, 5] = 0x7E00  # f16 NaN in expert 1's svh, column 5
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    inds = np.array([[1, 0], [2, 3], [3, 1], [0, 2], [1, 2], [3, 0]], np.int32)
    scores = np.full((rows, k), 0.5, np.float32)
    y = O.moe_swiglu(x, gate, up, down, inds, scores, hidden, inter, 48, limit=10.0)
    hit = (inds == 1).any(axis=1)
    assert np.isnan(y[hit]).all()
    assert np.isfinite(y[~hit]).all()
