"""The load-time self-check exl3_open runs (turboexl3_ds41/src/exl3/
quant.zig:469-503 `accept` -> selfcheck.zig:861-930; paths relative to
/root/reference/plugins/).

Without a GPU: the host part (SHA-256 against its standard's example and
the manifest's golden-plane code digests) passes; the refusal path, forced
through the test hook, refuses exl3_self_check and exl3_open by name before
any device is needed; and the oracle shows the golden planes the device part
decodes hold every one of the 65,536 states (so one-hot rows through the
GEMV over a plane cover the whole codebook, as the reference's check asserts).
On the GPU: the device part passes, and each of its checks, forced to fail,
refuses by its name."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from plugins_amd import exl3 as X

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_golden.json")))
BLOCK = '{"quant_method":"exl3","codebook":"mul1"}'


def fault(check):
    X.lib().exl3_set_self_check_fault(check.encode() if check else None)


def test_host_part_passes():
    v = X.lib().exl3_self_check(-1)
    assert v.is_ok(), v


@pytest.mark.parametrize("check,name", [("sha256", "sha256 known answer"),
                                        ("code", "golden plane code digest")])
def test_host_refusals_are_named_and_refuse_open(check, name):
    fault(check)
    try:
        v = X.lib().exl3_self_check(-1)
        assert v.code == X.FAILED and v.reason == f"turboexl3_mi355x: Exl3SelfCheckFailed ({name})"
        L = X.Loader(BLOCK, X.DictSource({}))
        assert L.opened.code == X.FAILED and "Exl3SelfCheckFailed" in L.opened.reason
    finally:
        fault(None)
    assert X.lib().exl3_self_check(-1).is_ok()


@pytest.mark.parametrize("name", ["gate_up_k2", "gate_up"])
def test_golden_plane_covers_every_state(name):
    p = GOLD["planes"][name]
    n = 16 * p["K"]
    code = O.synth_plane(p["seed"], (p["in"] // 16) * (p["out"] // 16) * n)
    tiles = code.reshape(-1, n)
    seen = np.zeros(65536, bool)
    for t in tiles[:: max(1, len(tiles) // 20000)]:
        seen[O.unpack_tile(t, n)] = True
    if not seen.all():
        for t in tiles:
            seen[O.unpack_tile(t, n)] = True
    assert seen.all()


@pytest.mark.gpu
def test_device_part_passes():
    v = X.lib().exl3_self_check(0)
    assert v.is_ok(), v


@pytest.mark.gpu
@pytest.mark.parametrize("check,name", [
    ("states", "codebook state table digest"),
    ("decode", "golden plane W_hat digest, decode kernel"),
    ("gemm", "one-hot rows through the GEMM differ from W_hat"),
    ("gemv", "one-hot rows through the GEMV differ from W_hat")])
def test_device_refusals_are_named(check, name):
    fault(check)
    try:
        v = X.lib().exl3_self_check(0)
        assert v.code == X.FAILED and v.reason == f"turboexl3_mi355x: Exl3SelfCheckFailed ({name})"
        L = X.Loader(BLOCK, X.DictSource({}))
        assert L.opened.code == X.FAILED and v.reason == L.opened.reason
    finally:
        fault(None)
    assert X.lib().exl3_self_check(0).is_ok()
    L = X.Loader(BLOCK, X.DictSource({}))
    assert L.opened.is_ok(), L.opened
    L.close()
