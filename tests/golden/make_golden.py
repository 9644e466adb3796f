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
    decodeMul1 (sushi_ds41/src/sushi/exl3/expert_exl3.zig:699-704) and the
    bitEnd tables (expert_exl3.zig:661-697);
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
