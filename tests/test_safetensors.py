"""Checkpoint reader (host code, no GPU): the library's mmap'd safetensors
reader against files written by the `safetensors` package, the reference
loader's contract (src/loader/safetensors.h:44-75): every tensor's dtype, shape
and bytes, several files as one namespace, directory opening, and clean errors
for malformed files."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file


@pytest.fixture(scope="module")
def hip():
    import w4a16_hip

    w4a16_hip.lib()   # loads without a GPU; these tests only use host entry points
    return w4a16_hip


def _tensors(seed):
    g = torch.Generator().manual_seed(seed)
    return {
        "model.layers.0.self_attn.q_proj.weight_packed":
            torch.randint(-2**31, 2**31 - 1, (64, 16), dtype=torch.int32, generator=g),
        "model.layers.0.self_attn.q_proj.weight_scale":
            torch.randn(64, 1, generator=g).to(torch.bfloat16),
        "model.layers.0.self_attn.q_proj.weight_zero_point":
            torch.randint(-2**31, 2**31 - 1, (8, 1), dtype=torch.int32, generator=g),
        "norm.weight": torch.randn(7, generator=g, dtype=torch.float32),
        "f16": torch.randn(3, 5, generator=g).to(torch.float16),
        "f64": torch.randn(2, 2, generator=g, dtype=torch.float64),
        "i8": torch.randint(-128, 127, (9,), dtype=torch.int8, generator=g),
        "u8": torch.randint(0, 255, (4, 4), dtype=torch.uint8, generator=g),
        "i16": torch.randint(-30000, 30000, (6,), dtype=torch.int16, generator=g),
        "i64": torch.randint(-2**40, 2**40, (3,), dtype=torch.int64, generator=g),
        "bool": torch.tensor([True, False, True]),
        "scalar": torch.tensor(2.5, dtype=torch.float32),
        "empty": torch.zeros(0, 4, dtype=torch.float32),
        "name with ünïcode/and \"quotes\"": torch.arange(5, dtype=torch.int32),
    }


def _bytes(t):
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.contiguous().numpy().tobytes()


def test_roundtrip_every_dtype(hip, tmp_path):
    ts = _tensors(0)
    path = str(tmp_path / "a.safetensors")
    save_file(ts, path, metadata={"format": "pt"})
    st = hip.SafeTensors(paths=[path])
    assert len(st) == len(ts)
    names = {torch.bfloat16: "BF16", torch.float16: "F16", torch.float32: "F32",
             torch.float64: "F64", torch.int8: "I8", torch.uint8: "U8", torch.int16: "I16",
             torch.int32: "I32", torch.int64: "I64", torch.bool: "BOOL"}
    for name, t in ts.items():
        info = st.info(name)
        assert hip.ST_DTYPES[info.dtype] == names[t.dtype], name
        assert tuple(info.shape[k] for k in range(info.ndim)) == tuple(t.shape), name
        assert info.nbytes == t.numel() * t.element_size()
        got = st.get(name)
        assert got.tobytes() == _bytes(t), name
    assert not st.has("missing")
    with pytest.raises(hip.W4A16Error) as e:
        st.info("missing")
    assert e.value.status == hip.QW4_ERR_NOTFOUND
    st.close()


def test_several_files_and_directory(hip, tmp_path):
    a = {"x.a": torch.arange(10, dtype=torch.int32)}
    b = {"x.b": torch.ones(3, 3, dtype=torch.float32)}
    save_file(a, str(tmp_path / "model-00002-of-00002.safetensors"))
    save_file(b, str(tmp_path / "model-00001-of-00002.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"x.a": "model-00002-of-00002.safetensors",
                                   "x.b": "model-00001-of-00002.safetensors"}}))
    st = hip.SafeTensors(dir=str(tmp_path))
    assert len(st) == 2
    assert st.get("x.a").tolist() == list(range(10))
    assert st.get("x.b").sum() == 9.0
    st.close()
    # the same names in two files are rejected
    save_file(a, str(tmp_path / "dup.safetensors"))
    with pytest.raises(hip.W4A16Error) as e:
        hip.SafeTensors(dir=str(tmp_path))
    assert e.value.status == hip.QW4_ERR_IO and "twice" in str(e.value)


def _raw(tmp_path, header: bytes, data: bytes = b"", hlen=None, name="bad.safetensors"):
    p = tmp_path / name
    p.write_bytes(struct.pack("<Q", len(header) if hlen is None else hlen) + header + data)
    return str(p)


@pytest.mark.parametrize("case", ["short", "hlen", "json", "trailing", "offsets", "size",
                                  "dtype", "shape", "not_object"])
def test_malformed_files_fail_cleanly(hip, tmp_path, case):
    ok = {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    data = b"\0" * 8
    if case == "short":
        p = tmp_path / "bad.safetensors"
        p.write_bytes(b"\1\2\3")
        path = str(p)
    elif case == "hlen":
        path = _raw(tmp_path, json.dumps(ok).encode(), data, hlen=1 << 40)
    elif case == "json":
        path = _raw(tmp_path, b'{"t": {"dtype": "F32", "shape": [2], ', data)
    elif case == "trailing":
        path = _raw(tmp_path, json.dumps(ok).encode() + b" x", data)
    elif case == "offsets":
        bad = {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 16]}}
        path = _raw(tmp_path, json.dumps(bad).encode(), data)
    elif case == "size":
        bad = {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}
        path = _raw(tmp_path, json.dumps(bad).encode(), data)
    elif case == "dtype":
        bad = {"t": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 8]}}
        path = _raw(tmp_path, json.dumps(bad).encode(), data)
    elif case == "shape":
        bad = {"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}
        path = _raw(tmp_path, json.dumps(bad).encode(), data)
    else:
        path = _raw(tmp_path, b"[1, 2]", data)
    with pytest.raises(hip.W4A16Error) as e:
        hip.SafeTensors(paths=[path])
    assert e.value.status == hip.QW4_ERR_IO


def test_header_json_escapes_and_metadata(hip, tmp_path):
    """A hand-written header with escapes, whitespace and metadata (the forms a
    JSON writer may emit), checked against Python's json module."""
    name = "a\\u00e9\\ud83d\\ude00\\n\\t\\\"/\\\\"
    header = ('{ "__metadata__" : {"k": "v", "n": "1"} ,\n "' + name +
              '" : { "dtype" : "I16", "shape" : [ 2 , 1 ], "data_offsets" : [0, 4] } }')
    path = _raw(tmp_path, header.encode(), b"\x01\x00\xff\xff")
    st = hip.SafeTensors(paths=[path])
    py_name = json.loads('"' + name + '"')
    assert st.get(py_name).reshape(-1).tolist() == [1, -1]
    st.close()


def test_load_ct_fused_rejects_bad_checkpoints(hip, tmp_path):
    """Errors of qw4_load_ct_fused that are decided on the host, before any GPU
    work: missing parts and wrong dtypes/shapes (model.cu:103-128 contract)."""
    path = str(tmp_path / "m.safetensors")
    save_file({"p.weight_packed": torch.zeros(64, 16, dtype=torch.int32),
               "p.weight_scale": torch.zeros(64, 1, dtype=torch.float32),   # must be BF16
               "p.weight_zero_point": torch.zeros(8, 1, dtype=torch.int32)}, path)
    st = hip.SafeTensors(paths=[path])
    with pytest.raises(hip.W4A16Error) as e:
        st.load_ct_fused(["q"], in_f=128, stream=0)
    assert e.value.status == hip.QW4_ERR_NOTFOUND
    with pytest.raises(hip.W4A16Error) as e:
        st.load_ct_fused(["p"], in_f=128, stream=0)
    assert e.value.status == hip.QW4_ERR_SHAPE and "BF16" in str(e.value)
    with pytest.raises(hip.W4A16Error) as e:
        st.load_ct_fused(["p"], in_f=256, stream=0)
    assert e.value.status == hip.QW4_ERR_SHAPE
    st.close()
