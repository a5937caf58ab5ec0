"""The checkpoint reader (iro_hip_st_*) on the host: tensors, dtypes, shapes
and metadata as the safetensors format defines them (safetensors.c:1-7), and
the malformed headers safetensors.c:330-497 rejects.  No device is needed.
Files are written by the `safetensors` package or, for the malformed cases and
BF16, by hand from the format."""
import json
import os
import struct

import numpy as np
import pytest

import iro_hip


def _write(path, header: dict, data: bytes, hlen_override=None):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if hlen_override is None else hlen_override))
        f.write(h)
        f.write(data)


def test_reads_tensors_written_by_the_safetensors_package(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(3)
    tensors = {
        "blocks.0.attention.wq.weight": rng.standard_normal((8, 16)).astype(np.float32),
        "half": rng.standard_normal((3, 5)).astype(np.float16),
        "ids": np.arange(7, dtype=np.int64),
        "codes": rng.integers(-128, 127, (4, 4), dtype=np.int8),
        "scalar": np.array(2.5, np.float32),
        "empty": np.zeros((0, 3), np.float32),
    }
    p = str(tmp_path / "m.safetensors")
    save_file(tensors, p, metadata={"config_json": '{"dim": 1024}', "format": "pt"})
    st = iro_hip.Safetensors(p)
    try:
        assert sorted(st.names()) == sorted(tensors)
        for name, a in tensors.items():
            dt, shape, _, nb = st.info(name)
            assert shape == a.shape and nb == a.nbytes, name
            assert st.bytes(name) == a.tobytes(), name
            assert np.array_equal(st.array(name), a), name
        assert st.info("half")[0] == "F16" and st.info("ids")[0] == "I64"
        # values are the raw JSON text between the quotes (safetensors.c:66-104
        # checks escapes and keeps them)
        assert st.meta("config_json") == '{\\"dim\\": 1024}' and st.meta("format") == "pt"
        assert st.meta("absent") is None
        with pytest.raises(KeyError):
            st.info("absent")
    finally:
        st.close()


def test_bf16_tensor_and_widening(tmp_path):
    bits = np.array([0x3F80, 0xC000, 0x0001, 0x7F80, 0x8000], np.uint16)  # 1, -2, tiny, inf, -0
    p = str(tmp_path / "b.safetensors")
    _write(p, {"w": {"dtype": "BF16", "shape": [5], "data_offsets": [0, 10]}}, bits.tobytes())
    st = iro_hip.Safetensors(p)
    try:
        got = st.array("w")
        want = (bits.astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        st.close()


BAD = {
    "unknown dtype": ({"w": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}, 8),
    "size mismatch": ({"w": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, 12),
    "past the data": ({"w": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, 8),
    "reversed offsets": ({"w": {"dtype": "F32", "shape": [0], "data_offsets": [8, 4]}}, 8),
    "negative dim": ({"w": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 0]}}, 0),
    "nine dims": ({"w": {"dtype": "U8", "shape": [1] * 9, "data_offsets": [0, 1]}}, 1),
    "no offsets": ({"w": {"dtype": "F32", "shape": [1]}}, 4),
    "tensor not an object": ({"w": [1, 2]}, 0),
    "metadata not strings": ({"__metadata__": {"a": 1}}, 0),
}


def test_string_escapes(tmp_path):
    p = str(tmp_path / "e.safetensors")
    h = b'{"__metadata__": {"k": "a\\u00e9\\n"}, "w\\/x": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}'
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"\x07")
    st = iro_hip.Safetensors(p)
    try:
        assert st.meta("k") == "a\\u00e9\\n" and st.names() == ["w\\/x"]
    finally:
        st.close()
    for bad in (b'{"__metadata__": {"k": "\\q"}}', b'{"__metadata__": {"k": "\\u12g4"}}'):
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", len(bad)) + bad + b"  ")
        with pytest.raises(iro_hip.StError, match="malformed header"):
            iro_hip.Safetensors(p)


@pytest.mark.parametrize("case", sorted(BAD))
def test_malformed_headers_are_rejected(tmp_path, case):
    header, nbytes = BAD[case]
    p = str(tmp_path / "bad.safetensors")
    _write(p, header, bytes(nbytes))
    with pytest.raises(iro_hip.StError, match="malformed header"):
        iro_hip.Safetensors(p)


def test_bad_lengths_and_files(tmp_path):
    p = str(tmp_path / "x.safetensors")
    _write(p, {}, b"", hlen_override=1 << 40)  # header longer than the file
    with pytest.raises(iro_hip.StError, match="header length"):
        iro_hip.Safetensors(p)
    with open(p, "wb") as f:
        f.write(b"\x02\x00\x00\x00")  # shorter than any valid file
    with pytest.raises(iro_hip.StError, match="too small"):
        iro_hip.Safetensors(p)
    with pytest.raises(iro_hip.StError, match="cannot open"):
        iro_hip.Safetensors(str(tmp_path / "missing.safetensors"))
    h = b'{"w": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]'  # unterminated
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + bytes(4))
    with pytest.raises(iro_hip.StError, match="malformed header"):
        iro_hip.Safetensors(p)


def test_matches_the_safetensors_package_reader(tmp_path):
    from safetensors import safe_open
    from safetensors.numpy import save_file
    rng = np.random.default_rng(5)
    tensors = {f"t{i}": rng.standard_normal((i + 1, 7)).astype(np.float32) for i in range(6)}
    p = str(tmp_path / "m.safetensors")
    save_file(tensors, p)
    st = iro_hip.Safetensors(p)
    try:
        with safe_open(p, framework="numpy") as f:
            for name in f.keys():
                assert np.array_equal(f.get_tensor(name), st.array(name))
    finally:
        st.close()
