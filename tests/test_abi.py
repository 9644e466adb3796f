"""The C-ABI library without a GPU: it loads, exports every symbol
include/exl3_mi355x.h declares, and its host-side entries (claims, validate,
bill, the table) behave as the reference's do on the reference's own
fixtures (turboexl3_ds41/config.zig:69-82, turboexl3_qwen38/config.zig:
135-190; paths relative to /root/reference/plugins/)."""
import ctypes
import json
import os
import re

import pytest

from plugins_amd import exl3 as X

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CONFIGS = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_configs.json")))


def test_header_symbols_are_exported_and_bound():
    text = open(os.path.join(ROOT, "include", "exl3_mi355x.h")).read()
    declared = set(re.findall(r"\b(exl3_[a-z_0-9]+)\s*\(", text))
    declared -= {"exl3_str", "exl3_verdict", "exl3_claim"}
    L = X.lib()
    for name in sorted(declared):
        assert hasattr(L, name), name
    assert declared == set(X.SIGNATURES), declared ^ set(X.SIGNATURES)


def test_quant_table_fields():
    t = X.quant_table()
    # the whole layout of quant.zig:24-107: size, version, name (16 bytes),
    # then 29 entries, each one pointer
    assert ctypes.sizeof(X.QuantTable) == 4 + 4 + 16 + 29 * 8
    assert t.size == ctypes.sizeof(X.QuantTable)
    assert t.version == 1
    assert ctypes.string_at(t.name.ptr, t.name.len) == b"turboexl3_mi355x"
    served = ("claims", "validate", "bill", "open", "close", "load_tensor", "load_bank", "release",
              "matmul", "moe", "register_kernels", "swiglu", "linear_split", "linear_finish",
              "linear_prepared", "linear_pieces", "linear_piece", "swiglu_shared", "resident",
              "resident_pending", "unrotate", "linear_joined")
    for f in X.TABLE_ENTRIES:
        assert bool(getattr(t, f)) == (f in served), f
    # the table's pointers are the flat symbols
    assert t.matmul == ctypes.cast(X.lib().exl3_matmul, ctypes.c_void_p).value
    assert t.linear_split == ctypes.cast(X.lib().exl3_linear_split, ctypes.c_void_p).value
    assert t.linear_piece == ctypes.cast(X.lib().exl3_linear_piece, ctypes.c_void_p).value
    assert t.linear_joined == ctypes.cast(X.lib().exl3_linear_joined, ctypes.c_void_p).value


def test_resident_entries_refuse_on_the_host():
    """The resident entries' argument checks run before any device call
    (quant.zig:96-107): an empty span drops nothing held and admits nothing,
    a dtype that is not an activation dtype is refused by name, a span that
    is not an un-rotated group is refused."""
    L = X.lib()
    n = ctypes.c_uint64(7)
    v = L.exl3_resident(X.WeightSpan(None, 0), 0, None, ctypes.byref(n))
    assert v.code == X.OK and n.value == 0
    assert L.exl3_resident(X.WeightSpan(None, 0), 0, None, None).code == X.FAILED
    assert L.exl3_resident_pending() == 0
    took = (ctypes.c_bool * 1)()
    v = L.exl3_unrotate(X.WeightSpan(None, 0), X.U8Span(None, 0), X.DT_I32, None, took)
    assert v.code == X.UNSUPPORTED and "BadExl3Dtype" in v.reason
    sizes = (ctypes.c_uint8 * 1)(2)
    v = L.exl3_unrotate(X.WeightSpan(None, 0), X.U8Span(sizes, 1), X.DT_F16, None, took)
    assert v.code == X.UNSUPPORTED and "BadExl3Shape" in v.reason
    w = (X.Weight * 1)()
    out = X.Array()
    v = L.exl3_linear_joined(X.WeightSpan(w, 1), X.Array(), None, ctypes.byref(out))
    assert v.code == X.UNSUPPORTED and "linear_joined" in v.reason


def test_table_entry_order_matches_the_reference_layout():
    """The entries' order is the reference's (quant.zig:24-107), read from the
    header's table declaration."""
    text = open(os.path.join(ROOT, "include", "exl3_mi355x.h")).read()
    body = text[text.index("typedef struct exl3_quant_table {"):text.index("} exl3_quant_table;")]
    names = re.findall(r"\(\*([a-z_]+)\)\(", body)
    assert tuple(names) == X.TABLE_ENTRIES


def test_linear_parts_layout():
    # size, dtype, side, inner, prepared, held (an Array), rows, parts
    assert X.LinearParts.held.offset == 24
    assert X.LinearParts.rows.offset == 24 + ctypes.sizeof(X.Array)
    assert ctypes.sizeof(X.LinearParts) == 24 + ctypes.sizeof(X.Array) + 32


def _ds41_block():
    return json.dumps(CONFIGS["ds41"]["quantization_config"])


def _ds41_config():
    c = CONFIGS["ds41"]
    return json.dumps({"model_type": c["model_type"], "quantization_config": c["quantization_config"],
                       "text_config": {"num_experts_per_tok": c["num_experts_per_tok"]}})


def _q38_config(k):
    c = CONFIGS[k]
    return json.dumps({"model_type": c["model_type"], "trunk_quant": c["trunk_quant"],
                       "expert_quant": c["expert_quant"],
                       "text_config": {"num_experts_per_tok": c["num_experts_per_tok"]}})


def test_claims_follow_ds41():
    # turboexl3_ds41/config.zig:43-47,68-74: exllamav3's block on a
    # DeepSeek-V4.1 pack only
    assert X.claims(_ds41_block(), _ds41_config()) == X.CLAIM_BY_MARKER
    assert X.claims(_ds41_block(), '{"model_type":"qwen4_exp"}') == X.CLAIM_NO
    assert X.claims(_ds41_block(), "{}") == X.CLAIM_NO
    assert X.claims('{"quant_method":"fp8"}', _ds41_config()) == X.CLAIM_NO
    assert X.claims("{", _ds41_config()) == X.CLAIM_NO
    for k in ("k2", "k3", "k4", "k5"):  # qwen38's packs are the other table's
        assert X.claims(json.dumps(CONFIGS[k]["trunk_quant"]), _q38_config(k)) == X.CLAIM_NO


def test_claims_qwen38_rule():
    # turboexl3_qwen38/config.zig:18-32: a qwen4_exp pack naming a trunk block
    for k in ("k2", "k3", "k4", "k5"):
        for part in ("trunk_quant", "expert_quant"):
            assert X.claims_qwen38(json.dumps(CONFIGS[k][part]), _q38_config(k)) == X.CLAIM_BY_MARKER
    c = json.loads(_q38_config("k3"))
    for mt, tq, want in (("qwen4_exp_text", c["trunk_quant"], X.CLAIM_BY_MARKER),
                         ("qwen4_exp", None, X.CLAIM_NO), ("deepseek_v41", c["trunk_quant"], X.CLAIM_NO)):
        cfg = json.dumps({"model_type": mt, "trunk_quant": tq})
        assert X.claims_qwen38("{}", cfg) == want, (mt, tq)
    assert X.claims_qwen38("{}", json.dumps({"model_type": "qwen4_exp"})) == X.CLAIM_NO
    assert X.claims_qwen38(_ds41_block(), _ds41_config()) == X.CLAIM_NO
    assert X.claims_qwen38("{}", "[") == X.CLAIM_NO


def test_two_tables_differ_only_in_their_claim():
    a, b = X.quant_table(), X.quant_table(qwen38=True)
    assert ctypes.string_at(b.name.ptr, b.name.len) == b"turboexl3_mi355x_qwen38"
    assert a.claims == ctypes.cast(X.lib().exl3_claims, ctypes.c_void_p).value
    assert b.claims == ctypes.cast(X.lib().exl3_claims_qwen38, ctypes.c_void_p).value
    assert (a.size, a.version) == (b.size, b.version)
    for f in X.TABLE_ENTRIES:
        if f != "claims":
            assert getattr(a, f) == getattr(b, f), f


def test_claims_nothing_else():
    # turboexl3_ds41/config.zig:72-74 and turboexl3_qwen38/config.zig:141-147
    for block in ('{"quant_method":"fp8"}', "{", "[]", "7", "", '{"format":"gptq"}', "null"):
        assert X.claims(block, _ds41_config()) == X.CLAIM_NO, block


def test_validate_admits_the_fixture_packs():
    assert X.validate(_ds41_block(), _ds41_config()).is_ok()
    for k in ("k2", "k3", "k4", "k5"):
        cfg = json.dumps({"text_config": {"num_experts_per_tok": CONFIGS[k]["num_experts_per_tok"]}})
        assert X.validate(json.dumps(CONFIGS[k]["trunk_quant"]), cfg).is_ok(), k
        assert X.validate(json.dumps(CONFIGS[k]["expert_quant"]), cfg).is_ok(), k


@pytest.mark.parametrize("edit,why", [
    ({"codebook": "3inst"}, "Exl3CodebookUnsupported"),   # turboexl3_qwen38/config.zig:171
    ({"codebook": 7}, "Exl3CodebookUnsupported"),
    ({"window": 20}, "Exl3WindowUnsupported"),            # :172
    ({"window": 7}, "Exl3WindowUnsupported"),
    ({"window": 12.5}, "Exl3WindowUnsupported"),
    ({"format": "gptq"}, "NotExl3"),                      # :173
    ({"k": 9.25}, "Exl3RateUnsupported"),                 # :174
    ({"k": 0.5}, "Exl3RateUnsupported"),
    ({"k": 1.0625}, "Exl3RateUnsupported"),               # 17 halfwords: odd
    ({"k": "4"}, "Exl3RateUnsupported"),
])
def test_validate_refuses_by_name(edit, why):
    block = dict(CONFIGS["k4"]["expert_quant"])
    block.update(edit)
    v = X.validate(json.dumps(block))
    assert v.code == X.UNSUPPORTED
    assert v.reason == "turboexl3_mi355x: " + why


def test_validate_keeps_turboexl3s_codebooks():
    # turboexl3_qwen38/config.zig:91-93: mul1 or mcg; the table codebooks
    # (spec1, std1, pair1) serve through exl3_weight_wrap only
    for cb in ("spec1", "std1", "pair1"):
        block = json.loads(X.quant_block(cb, table="spec1-w15" if cb == "spec1" else None))
        v = X.validate(json.dumps(block))
        assert v.reason == "turboexl3_mi355x: Exl3CodebookUnsupported", cb


def _wrap_verdict(block: str, n: int = 40, fake: bool = False):
    """exl3_weight_wrap's verdict for a block; fake: shaped arrays at a dummy
    address (never read: the refusals come before any use)."""
    arrays = [X.Array(), X.Array(), X.Array()]
    if fake:
        for a, (dt, dims) in zip(arrays, ((X.DT_U16, (8, 8, n)), (X.DT_F16, (128,)), (X.DT_F16, (128,)))):
            a.data, a.dtype, a.ndim = 0x1000, dt, len(dims)
            for i, d in enumerate(dims):
                a.shape[i] = d
    w = X.Weight()
    return X.lib().exl3_weight_wrap(*arrays, X.Str.of(block), 0, ctypes.byref(w))


@pytest.mark.parametrize("block,why", [
    # sushi_ds41/src/sushi/exl3/codebook_tables.zig:351-368, through the block
    ({"codebook": "pair1"}, "Exl3CodebookTableUnknown"),
    ({"codebook": "pair1", "codebook_table": "pair1-w16-v9", "codebook_digest": "c089b4eb"},
     "Exl3CodebookTableUnknown"),
    ({"codebook": "pair1", "codebook_table": 7, "codebook_digest": "c089b4eb"}, "Exl3CodebookTableUnknown"),
    ({"codebook": "pair1", "codebook_table": "pair1-w16-v1"}, "Exl3CodebookTableDigestMismatch"),
    ({"codebook": "pair1", "codebook_table": "pair1-w16-v1", "codebook_digest": "deadbeef"},
     "Exl3CodebookTableDigestMismatch"),
    ({"codebook": "spec1", "codebook_table": "pair1-w16-v1", "codebook_digest": "c089b4eb"},
     "Exl3CodebookTableCodebookMismatch"),
    ({"codebook": "pair1", "window": 15, "codebook_table": "pair1-w16-v1", "codebook_digest": "c089b4eb"},
     "Exl3CodebookTableWindowMismatch"),
    ({"codebook": "std1", "window": 15, "codebook_table": "std1", "codebook_digest": "2ac2594d"},
     "Exl3CodebookTableDigestMismatch"),
    ({"codebook": "spec1", "window": 15, "codebook_table": "std1", "codebook_digest": "c5dba171"},
     "Exl3CodebookTableCodebookMismatch"),
    ({"codebook": "spec1", "window": 15}, "Exl3CodebookTableUnknown"),
    ({"codebook": "spec1", "window": 15, "codebook_table": "spec1-w15", "codebook_digest": "2ac2594d"},
     "Exl3CodebookTableLegacyConfig"),
    ({"codebook": "3inst"}, "Exl3CodebookUnsupported"),
])
def test_weight_wrap_refuses_codebook_tables_by_name(block, why):
    b = {"format": "exl3", "window": 16, **block}
    v = _wrap_verdict(json.dumps(b))
    assert v.code == X.UNSUPPORTED and v.reason == "turboexl3_mi355x: " + why, v


def test_weight_wrap_admits_every_window_for_spec1_and_std1_tables():
    # a spec1 / std1 table decodes at any window (codebook_tables.zig:354-357,
    # 404-414): the block passes, and the null arrays are what is refused
    for w in range(8, 17):
        for cb, t in (("spec1", "spec1-w15"), ("spec1", "spec1-w16"), ("std1", "std1")):
            v = _wrap_verdict(X.quant_block(cb, w, t))
            assert v.reason == "turboexl3_mi355x: BadExl3Shape", (cb, t, w, v)
    assert _wrap_verdict(X.quant_block("pair1", 16)).reason == "turboexl3_mi355x: BadExl3Shape"


@pytest.mark.parametrize("cb,table,n,has_row", [
    ("std1", "std1", 16, False), ("std1", "std1", 70, False), ("std1", "std1", 24, True),
    ("pair1", None, 22, False), ("pair1", None, 66, False), ("pair1", None, 64, True),
    ("spec1", "spec1-w16", 16, False), ("spec1", "spec1-w15", 16, True), ("spec1", "spec1-w15", 128, True),
])
def test_weight_wrap_refuses_a_rate_its_table_has_no_row_for(cb, table, n, has_row):
    # codebook_tables.zig:48-52 and 420-429 (std1 stops at K4, spec1-w15
    # reaches K1 and K8); a rate with a row passes to the arrays' device check
    v = _wrap_verdict(X.quant_block(cb, 16, table), n=n, fake=True)
    if has_row:
        assert v.reason != "turboexl3_mi355x: Exl3CodebookTableRateMissing", v
    else:
        assert v.reason == "turboexl3_mi355x: Exl3CodebookTableRateMissing", v


def test_validate_rates_every_even_halfword_count():
    for n in range(16, 129):
        v = X.validate(json.dumps({"format": "exl3", "codebook": "mcg", "k": n / 16}))
        assert v.is_ok() == (n % 2 == 0), n


def test_validate_refuses_topk_beyond_the_reduce_bank():
    # turboexl3_qwen38/config.zig:81-83 (max_topk = 32)
    block = json.dumps(CONFIGS["k4"]["expert_quant"])
    assert X.validate(block, json.dumps({"text_config": {"num_experts_per_tok": 32}})).is_ok()
    v = X.validate(block, json.dumps({"text_config": {"num_experts_per_tok": 33}}))
    assert v.reason == "turboexl3_mi355x: Exl3TopKExceedsReduceBank"
    v = X.validate(block, json.dumps({"num_experts_per_tok": 40}))
    assert v.reason == "turboexl3_mi355x: Exl3TopKExceedsReduceBank"


def test_bill_is_the_stored_bytes():
    # turboexl3_ds41/config.zig:56-61: resident as the pack stores it
    for stored in (0, 1, 8 << 20, 3 << 40):
        assert X.bill(_ds41_block(), "/packs/x", stored) == stored


def test_moe_entry_refuses_like_the_reference():
    # turboexl3_ds41/plugin.zig:263-265
    v = X.lib().exl3_moe(None, X.Array(), X.Array(), X.Array(), False, None, None)
    assert v.code == X.UNSUPPORTED and b"swiglu" in v.why


def test_matmul_refuses_without_a_weight():
    v = X.lib().exl3_matmul(None, X.Array(), None, None)
    assert v.code == X.FAILED


def test_json_reader_edge_cases():
    # escapes, nesting and trailing garbage go through the C++ reader
    cfg = _ds41_config()
    assert X.claims('{"quant_method":"ex\\u006c3"}', cfg) == X.CLAIM_BY_MARKER
    assert X.claims('{"a":[1,2,{"b":null}],"quant_method":"exl3"}', cfg) == X.CLAIM_BY_MARKER
    assert X.claims('{"quant_method":"exl3"} x', cfg) == X.CLAIM_NO
    assert X.claims('{"quant_method":"exl3",}', cfg) == X.CLAIM_NO
    assert X.claims('[' * 300 + ']' * 300, cfg) == X.CLAIM_NO
    assert X.claims('{"quant_method":"exl3"}', '{"model_type":"deepseek_v41"} x') == X.CLAIM_NO
