"""The C++ safetensors reader (ai_amd/host/safetensors.cpp) against files
written by the `safetensors` library, on the CPU.

Pins, per the reference (safetensors/safetensors.go, convert.go): BF16 -> fp32
is exact, F16 -> fp32 keeps subnormals, infinities and NaN, F64 rounds to
fp32, F32 is copied; metadata is read; shards of a directory are merged and
the index is checked; malformed headers are refused with the reference's
messages.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from ai_amd import build as B

DUMP = os.path.join(B.CPP_TEST_BIN, "st_dump")


def dump(path):
    if not os.path.exists(DUMP):
        pytest.fail(f"{DUMP} is missing: run __graft_entry__.build() first")
    r = subprocess.run([DUMP, str(path)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    rows = [json.loads(l) for l in r.stdout.splitlines()]
    errs = [x["error"] for x in rows if "error" in x]
    if errs:
        return {"error": errs[0]}
    return {"tensors": {x["name"]: x for x in rows if "name" in x},
            "meta": {x["meta"]: x["value"] for x in rows if "meta" in x}}


def values(entry):
    return np.array(entry["bits"], dtype=np.uint32).view(np.float32)


def test_dtypes_convert_like_the_reference(tmp_path):
    g = torch.Generator().manual_seed(5)
    f16 = torch.tensor([0.0, -0.0, 1.0, 65504.0, 6.1e-5, 5.96e-8, -3.0e-7, float("inf"), float("-inf")],
                       dtype=torch.float16)
    t = {
        "bf16": torch.randn(4, 33, generator=g).to(torch.bfloat16),
        "f16": f16,
        "f32": torch.randn(3, 5, 7, generator=g),
        "f64": torch.randn(17, generator=g, dtype=torch.float64) * 1e3,
        "i32": torch.arange(6, dtype=torch.int32).reshape(2, 3),
        "scalar": torch.tensor(2.5),
        "empty": torch.zeros(0, 3),
    }
    p = tmp_path / "m.safetensors"
    save_file(t, str(p), metadata={"format": "pt", "note": "x"})
    d = dump(p)
    assert "error" not in d, d
    ts = d["tensors"]
    assert d["meta"] == {"format": "pt", "note": "x"}
    for name in ("bf16", "f16", "f32", "f64", "scalar", "empty"):
        want = t[name].to(torch.float32).numpy().ravel()
        got = values(ts[name])
        assert list(ts[name]["shape"]) == list(t[name].shape), name
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)  # bit-exact
    assert ts["bf16"]["dtype"] == "BF16" and ts["i32"]["dtype"] == "I32" and "bits" not in ts["i32"]


def test_f16_subnormals_and_nan(tmp_path):
    bits = np.array([0x0001, 0x03FF, 0x8001, 0x7C01, 0x7E00, 0xFC00, 0x3555], dtype=np.uint16)
    t = torch.from_numpy(bits.view(np.float16).copy())
    save_file({"h": t}, str(tmp_path / "h.safetensors"))
    got = values(dump(tmp_path / "h.safetensors")["tensors"]["h"])
    want = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    np.testing.assert_array_equal(got[fin], want[fin])


def test_directory_shards_and_index(tmp_path):
    d = tmp_path / "shards"
    d.mkdir()
    save_file({"a": torch.ones(2, 2)}, str(d / "model-00001-of-00002.safetensors"))
    save_file({"b": torch.full((3,), 2.0)}, str(d / "model-00002-of-00002.safetensors"))
    idx = {"metadata": {}, "weight_map": {"a": "model-00001-of-00002.safetensors",
                                          "b": "model-00002-of-00002.safetensors"}}
    (d / "model.safetensors.index.json").write_text(json.dumps(idx))
    r = dump(d)
    assert set(r["tensors"]) == {"a", "b"}
    idx["weight_map"]["b"] = "model-00001-of-00002.safetensors"
    (d / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert "found in model-00002" in dump(d)["error"]
    idx["weight_map"]["b"] = "model-00002-of-00002.safetensors"
    idx["weight_map"]["c"] = "model-00001-of-00002.safetensors"
    (d / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert "no shard holds it" in dump(d)["error"]
    e = tmp_path / "empty"
    e.mkdir()
    assert "no *.safetensors" in dump(e)["error"]


def raw_file(path, header, data=b""):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("header,data,want", [
    ({"x": {"dtype": "Q8", "shape": [1], "data_offsets": [0, 1]}}, b"\0", "unknown dtype"),
    ({"x": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 0]}}, b"", "negative dimension"),
    ({"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 16]}}, b"\0" * 8, "outside the data section"),
    ({"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8, "want 12"),
])
def test_bad_headers(tmp_path, header, data, want):
    p = tmp_path / "bad.safetensors"
    raw_file(p, header, data)
    assert want in dump(p)["error"]


def test_truncated_files(tmp_path):
    p = tmp_path / "short.safetensors"
    p.write_bytes(b"\1\2\3")
    assert "too short" in dump(p)["error"]
    p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    assert "exceeds file size" in dump(p)["error"]
