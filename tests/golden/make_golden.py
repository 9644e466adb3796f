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
    bitEnd tables (expert_exl3.zig:661-697).
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


if __name__ == "__main__":
    main()
