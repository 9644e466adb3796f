"""The pack loader without a GPU: exl3_safetensors_open maps a pack's
safetensors files and hands out the tensors a linear is stored as
(<base>.trellis i16 [in/16, out/16, n], <base>.suh f16 [in], <base>.svh f16
[out]; turboexl3_ds41/plugin.zig:86-103, paths relative to
/root/reference/plugins/), and refuses malformed files by name.  Valid files
are written by the `safetensors` package (an independent writer of the
format); malformed ones by hand."""
import ctypes
import json
import struct

import numpy as np
import pytest

from plugins_amd import exl3 as X

st = pytest.importorskip("safetensors.numpy")


def _linear(rng, in_f=256, out_f=128, n=48):
    trellis = rng.integers(-32768, 32768, size=(in_f // 16, out_f // 16, n), dtype=np.int64)
    return (trellis.astype(np.int16), rng.standard_normal(in_f).astype(np.float16),
            rng.standard_normal(out_f).astype(np.float16))


def _raw(path, header: dict, data: bytes, length=None):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if length is None else length))
        f.write(h)
        f.write(data)


def _bytes_at(view, nbytes):
    return ctypes.string_at(view[2], nbytes)


def test_tensors_come_back_as_stored(tmp_path):
    rng = np.random.default_rng(1)
    t, u, v = _linear(rng)
    extra = rng.standard_normal((3, 5)).astype(np.float32)
    idx = np.arange(7, dtype=np.int32)
    p1, p2 = tmp_path / "a.safetensors", tmp_path / "b.safetensors"
    st.save_file({"m.q.trellis": t, "m.q.suh": u}, str(p1))
    st.save_file({"m.q.svh": v, "x.f32": extra, "x.idx": idx}, str(p2),
                 metadata={"format": "pt"})
    src = X.SafetensorsSource([p1, p2])
    for name, a, code in (("m.q.trellis", t, X.DT_I16), ("m.q.suh", u, X.DT_F16),
                          ("m.q.svh", v, X.DT_F16), ("x.f32", extra, X.DT_F32),
                          ("x.idx", idx, X.DT_I32)):
        view = src.tensor(name)
        assert view is not None, name
        assert view[0] == code and view[1] == a.shape, (name, view[:2])
        assert _bytes_at(view, a.nbytes) == a.tobytes(), name
    assert src.tensor("m.q.missing") is None
    assert src.tensor("__metadata__") is None
    src.close()


def test_refusals(tmp_path):
    rng = np.random.default_rng(2)
    t, u, _ = _linear(rng)
    good = tmp_path / "good.safetensors"
    st.save_file({"m.q.trellis": t}, str(good))
    dup = tmp_path / "dup.safetensors"
    st.save_file({"m.q.trellis": t, "m.q.suh": u}, str(dup))

    def refused(paths, code, text):
        with pytest.raises(OSError) as e:
            X.SafetensorsSource(paths)
        assert f"code={code}" in str(e.value) and text in str(e.value), str(e.value)

    refused([tmp_path / "absent.safetensors"], X.FAILED, "cannot be opened")
    refused([good, dup], X.FAILED, "two safetensors files")
    short = tmp_path / "short.safetensors"
    short.write_bytes(b"\x01\x02\x03")
    refused([short], X.FAILED, "shorter than its header")
    past = tmp_path / "past.safetensors"
    _raw(past, {}, b"", length=1 << 20)
    refused([past], X.FAILED, "runs past its file")
    notjson = tmp_path / "notjson.safetensors"
    with open(notjson, "wb") as f:
        f.write(struct.pack("<Q", 5) + b"[1,2]")
    refused([notjson], X.FAILED, "not a JSON object")
    data = np.arange(8, dtype=np.float16).tobytes()
    for name, header, text, code in (
            ("offs", {"a": {"dtype": "F16", "shape": [8], "data_offsets": [0, 14]}},
             "offsets disagree", X.FAILED),
            ("over", {"a": {"dtype": "F16", "shape": [16], "data_offsets": [0, 32]}},
             "offsets disagree", X.FAILED),
            ("dtype", {"a": {"dtype": "F8_E4M3", "shape": [16], "data_offsets": [0, 16]}},
             "unknown dtype", X.UNSUPPORTED),
            ("shape", {"a": {"dtype": "F16", "shape": [2.5], "data_offsets": [0, 16]}},
             "list of sizes", X.FAILED),
            ("entry", {"a": {"dtype": "F16", "shape": [8]}}, "malformed", X.FAILED)):
        p = tmp_path / f"{name}.safetensors"
        _raw(p, header, data)
        refused([p], code, text)
    # a well-formed hand-written file loads
    ok = tmp_path / "ok.safetensors"
    _raw(ok, {"a": {"dtype": "F16", "shape": [2, 4], "data_offsets": [0, 16]},
              "__metadata__": {"k": "v"}}, data)
    src = X.SafetensorsSource(ok)
    view = src.tensor("a")
    assert view[0] == X.DT_F16 and view[1] == (2, 4) and _bytes_at(view, 16) == data
    src.close()


def test_pack_directory(tmp_path):
    (tmp_path / "experts.bin").write_bytes(b"x" * 123)
    (tmp_path / "sub").mkdir()
    d = X.PackDirectory(tmp_path)
    assert d.file_bytes("experts.bin") == 123
    assert d.file_bytes("absent.bin") == 0
    assert d.file_bytes("sub") == 0
    assert d.file_bytes("../experts.bin") == 0 and d.file_bytes("/etc/hostname") == 0
    d.close()
    with pytest.raises(OSError):
        X.PackDirectory(tmp_path / "experts.bin")
