"""Writes tests/golden/reference_golden.json from the reference's own test data.

Run in the build container (where /root/reference exists):
    python tests/golden/make_golden.py

What it copies, as data only (no reference code is imported or run):
  * the golden digests of turboexl3_ds41/src/exl3/kernels/exl3/manifest.json
    (key "golden": the mul1 table sha256 and four seeded planes' code and
    W_hat sha256), consumed by the reference at
    turboexl3_ds41/src/exl3/kernels.zig:938-962 and selfcheck.zig:861-930;
  * every tile of turboexl3_ds41/src/frac_tiles.json (stored words and the
    f16 row-major decode), read by turboexl3_ds41/src/frac_test.zig:23-44;
  * the known-answer values written in the reference's tests:
    decodeMul1 (sushi_ds41/src/sushi/exl3/expert_exl3.zig:699-704), the
    bitEnd tables (expert_exl3.zig:661-697), decodeHashMask
    (expert_exl3.zig:728-739), decodePair on PAIR1's rows
    (expert_exl3.zig:767-792), and the codebook tables' pinned digests and
    sampled rows (sushi_ds41/src/sushi/exl3/codebook_tables.zig:281-303,
    389-460);
  * into reference_configs.json, the quantization blocks of the reference's
    pack-config fixtures that its claims/validate tests read
    (turboexl3_ds41/tests/fixtures/config.json via config.zig:67-82;
    turboexl3_qwen38/tests/fixtures/k{2,3,4,5}.json via config.zig:108-190):
    model_type, the EXL3 blocks and the top-k, nothing else.
"""
from __future__ import annotations

import json
import os

REF = "/root/reference/plugins"
HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> None:
    manifest = json.load(open(os.path.join(REF, "turboexl3_ds41/src/exl3/kernels/exl3/manifest.json")))
    g = manifest["golden"]
    planes = {}
    for name, p in g["planes"].items():
        planes[name] = {
            "K": p["K"],
            "codebook": p["codebook"],
            "in": p["projection"][0],
            "out": p["projection"][1],
            "seed": p["seed"],
            "code_sha256": p["code_sha256"],
            "w_hat_sha256": p["w_hat_sha256"],
        }
    frac = json.load(open(os.path.join(REF, "turboexl3_ds41/src/frac_tiles.json")))
    tiles = [{"src": t["src"], "n": t["n"], "words": t["words"], "expect": t["expect"]} for t in frac["tiles"]]
    out = {
        "what": "data copied from the reference's test fixtures by tests/golden/make_golden.py",
        "mul1_table_sha256": g["mul1_table"]["sha256"],
        "mul1_table_layout": g["mul1_table"]["layout"],
        "planes": planes,
        "planes_source": "turboexl3_ds41/src/exl3/kernels/exl3/manifest.json golden.planes",
        "frac_tiles": tiles,
        "frac_tiles_source": "turboexl3_ds41/src/frac_tiles.json",
        "kat_mul1": {"0": 49896, "1": 14625, "7": 47511},
        "kat_mul1_source": "sushi_ds41/src/sushi/exl3/expert_exl3.zig:699-704",
        "kat_bit_end": {
            "40": {"ends": [2, 5, 7, 10, 12, 15, 17, 20], "fresh": [2, 3] * 8},
            "44": {"ends": [2, 5, 8, 11, 13, 16, 19, 22], "fresh": [2, 3, 3, 3] * 4},
            "48": {"ends": [3, 6, 9, 12, 15, 18, 21, 24], "fresh": [3] * 16},
            "64": {"ends": [4, 8, 12, 16, 20, 24, 28, 32], "fresh": [4] * 16},
        },
        "kat_bit_end_source": "sushi_ds41/src/sushi/exl3/expert_exl3.zig:661-697",
        "kat_hash_mask": {"mult": 0x840C1F37, "mask": 0x8FFE8FD0,
                          "values": {"0": 0x0000, "1": 0x3E0D, "7": 0xBF94, "21": 0xC060, "62": 0xC164,
                                     "4660": 0xBAD0, "65535": 0xBB8A}},
        "kat_hash_mask_source": "sushi_ds41/src/sushi/exl3/expert_exl3.zig:728-739",
        "kat_pair1": [[24, 0x1, 0x3C74, 0xBDAA], [24, 0x1234, 0x3A7C, 0xB8CB], [32, 0x0, 0x0000, 0x0000],
                      [32, 0x1, 0xB440, 0xB804], [32, 0x1234, 0x3822, 0xB086], [32, 0xFFFF, 0xB19E, 0x3DA0],
                      [38, 0x1, 0x3FA4, 0x3610], [38, 0x1234, 0x3A99, 0xB898], [40, 0x1, 0x3FA6, 0x3610],
                      [40, 0x1234, 0x3A6D, 0xB898], [48, 0x1, 0xB5B2, 0xB7AF], [48, 0x15, 0x37C6, 0xA9D0],
                      [48, 0x8000, 0xA6E0, 0xB3EE], [56, 0x1, 0xBF92, 0xB91E], [56, 0x1234, 0xBCF0, 0xBAD6],
                      [58, 0x1, 0xBC90, 0x3608], [58, 0x1234, 0x3CB0, 0xB102], [64, 0x7, 0xAA00, 0xBA80],
                      [64, 0x15, 0xC010, 0x34F7], [64, 0xFFFF, 0x3B10, 0x3C0C]],
        "kat_pair1_source": "sushi_ds41/src/sushi/exl3/expert_exl3.zig:767-792 (n, codeword, w0, w1)",
        "codebook_tables": {
            "digest_vector": {"ns": [24, 64], "rows": [[1, 2, 3, 4], [0xFFFFFFFF, 0, 0x80000000, 0x7FFFFFFF]],
                              "fields": 4, "digest": "72fc0906"},
            "digests": {"pair1-w16-v1": "c089b4eb", "spec1-w15": "37f72431", "spec1-w16": "753ffa03",
                        "std1": "c5dba171"},
            "superseded": {"spec1-w15": ["2ac2594d"]},
            "rows": {"spec1-w15": {"16": [0x84d1cf89, 0x8fe08947], "22": [0x84d1cfc9, 0x8ff08b67],
                                   "24": [0x84c1cf49, 0x8fe08b47], "48": [0x84181FB5, 0x8FE08F80],
                                   "64": [0x3fed4cef, 0x8ff08ff0], "66": [0x3fed4cef, 0x8fe28ff0],
                                   "80": [0x8000387b, 0x8fe08ff7], "96": [0xd0003751, 0x8ff98fff],
                                   "112": [0xc00031f1, 0x8ffe8ffa], "128": [0x80003811, 0x8ffc8ffc]},
                     "std1": {"24": [0x840C1F37, 0x8FFE8FD0], "40": [0x840C1F37, 0x8FFE8FD0],
                              "64": [0x840C1F37, 0x8FFE8FD0]},
                     "pair1-w16-v1": {"24": [0x58F41BF3, 3, 0x8ED78C13, 0x8EEE8C03],
                                      "32": [0x3B22BE15, 3, 0x8ED78C13, 0x8ECE8C03],
                                      "48": [0xF75D60FF, 19, 0x8E6E8F9A, 0x8E258FFE],
                                      "56": [0x82439F67, 19, 0x8E6E8F9A, 0x8E258FAE],
                                      "64": [0xE2C7FC0D, 19, 0x8F408FA0, 0x8F118FC9]}},
            "no_row": {"spec1-w15": [14, 25, 130], "std1": [16, 18, 70, 120, 128],
                       "pair1-w16-v1": [16, 22, 66, 72]},
            "source": "sushi_ds41/src/sushi/exl3/codebook_tables.zig:281-303,389-460; "
                      "expert_exl3.zig:749-765",
        },
    }
    with open(os.path.join(HERE, "reference_golden.json"), "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", os.path.join(HERE, "reference_golden.json"), len(tiles), "frac tiles")

    ds = json.load(open(os.path.join(REF, "turboexl3_ds41/tests/fixtures/config.json")))
    configs = {
        "what": "quantization blocks of the reference's pack-config fixtures (tests/golden/make_golden.py)",
        "ds41": {
            "source": "turboexl3_ds41/tests/fixtures/config.json",
            "model_type": ds["model_type"],
            "quantization_config": ds["quantization_config"],
            "num_experts_per_tok": ds.get("text_config", {}).get("num_experts_per_tok"),
        },
    }
    for k in ("k2", "k3", "k4", "k5"):
        d = json.load(open(os.path.join(REF, f"turboexl3_qwen38/tests/fixtures/{k}.json")))
        configs[k] = {
            "source": f"turboexl3_qwen38/tests/fixtures/{k}.json",
            "model_type": d["model_type"],
            "trunk_quant": d["trunk_quant"],
            "expert_quant": d["expert_quant"],
            "num_experts_per_tok": d.get("text_config", {}).get("num_experts_per_tok"),
        }
    with open(os.path.join(HERE, "reference_configs.json"), "w") as f:
        json.dump(configs, f, indent=1)
    print("wrote", os.path.join(HERE, "reference_configs.json"))


if __name__ == "__main__":
    main()
