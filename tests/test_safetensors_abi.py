"""Model-file errors of ppocr_rh_create_from_safetensors, checked on the CPU: every
malformed file or tensor is reported as PPOCR_ERR_MODEL (OcrError::SafeTensorsError /
ModelError, src/engine/loader.rs:34-92) before any device is touched.  Files are written
with the safetensors package (the format the reference's loader reads) or by hand for the
malformed cases."""
import ctypes
import json
import os
import struct

import numpy as np
import pytest


def _create(rh, path, w="linear_8.w_0", b="linear_8.b_0", quantize=1):
    h = ctypes.c_void_p(123)
    enc = (lambda x: None if x is None else os.fsencode(x))
    rc = rh._lib.lib().ppocr_rh_create_from_safetensors(enc(path), enc(w), enc(b), quantize, 0, ctypes.byref(h))
    assert h.value is None  # never a handle on failure
    return rc, rh._lib.last_error()


def _raw_file(path, header, payload=b""):
    hb = header if isinstance(header, bytes) else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + payload)


@pytest.fixture
def model(tmp_path):
    """A small model file: the head weight [k][n] and bias [n], plus a graph in the
    metadata (a JSON string with escapes, as the reference's bundles carry) and an I64
    constant."""
    from safetensors.numpy import save_file
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((120, 70)) * 0.05).astype(np.float32)
    b = (rng.standard_normal(70) * 0.01).astype(np.float32)
    path = str(tmp_path / "rec.safetensors")
    graph = json.dumps({"nodes": [{"op": "MatMul", "name": "MatMul.12", "attr": "a \"quoted\" \\ é"}]})
    save_file({"linear_8.w_0": w, "linear_8.b_0": b, "shape_const": np.array([1, 2, 3], np.int64)}, path,
              metadata={"graph": graph})
    return path


def test_valid_file_reaches_the_device_step(rh, model):
    """A well-formed file passes every model check; without a GPU the call then fails on
    the device (never with a model error)."""
    rc, msg = _create(rh, model)
    if rc == rh.PPOCR_OK:
        pytest.skip("a GPU is present: the GPU tests cover the created head")
    assert rc in (rh.PPOCR_ERR_DEVICE, rh.PPOCR_ERR_INVALID_ARG), (rc, msg)
    assert not msg.startswith(("SafeTensors", "Model"))


def test_missing_file_and_null_names(rh, tmp_path):
    rc, msg = _create(rh, str(tmp_path / "absent.safetensors"))
    assert rc == rh.PPOCR_ERR_MODEL and msg.startswith("Model: failed to read model file")
    rc, msg = _create(rh, str(tmp_path / "absent.safetensors"), w=None)
    assert rc == rh.PPOCR_ERR_INVALID_ARG and "null weight name" in msg


def test_missing_and_mistyped_tensors(rh, model, tmp_path):
    rc, msg = _create(rh, model, w="linear_9.w_0")
    assert rc == rh.PPOCR_ERR_MODEL and msg == "Model: tensor 'linear_9.w_0' not found in the model file"
    rc, msg = _create(rh, model, w="shape_const")
    assert rc == rh.PPOCR_ERR_MODEL and "must be a 2-D F32 matrix" in msg
    rc, msg = _create(rh, model, w="linear_8.b_0")
    assert rc == rh.PPOCR_ERR_MODEL and "must be a 2-D F32 matrix" in msg
    rc, msg = _create(rh, model, b="shape_const")
    assert rc == rh.PPOCR_ERR_MODEL and "must be F32 with 70 values" in msg
    rc, msg = _create(rh, model, b="nope")
    assert rc == rh.PPOCR_ERR_MODEL and "'nope' not found" in msg


@pytest.mark.parametrize("case", ["short", "hlen", "json", "dtype", "offsets", "reversed", "size", "trailing",
                                  "escape", "fields"])
def test_malformed_headers(rh, tmp_path, case):
    path = str(tmp_path / f"{case}.safetensors")
    payload = np.zeros(6, np.float32).tobytes()
    good = {"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]}}
    if case == "short":
        open(path, "wb").write(b"\x01\x02")
    elif case == "hlen":
        open(path, "wb").write(struct.pack("<Q", 10 ** 6) + b"{}")
    elif case == "json":
        _raw_file(path, b'{"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]}', payload)
    elif case == "dtype":
        _raw_file(path, {"w": {"dtype": "F31", "shape": [2, 3], "data_offsets": [0, 24]}}, payload)
    elif case == "offsets":
        _raw_file(path, {"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 28]}}, payload)
    elif case == "reversed":
        _raw_file(path, {"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [24, 0]}}, payload)
    elif case == "size":
        _raw_file(path, {"w": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 24]}}, payload)
    elif case == "trailing":
        _raw_file(path, json.dumps(good).encode() + b" x", payload)
    elif case == "escape":
        _raw_file(path, b'{"w\\q": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]}}', payload)
    elif case == "fields":
        _raw_file(path, {"w": {"dtype": "F32", "shape": [2, 3]}}, payload)
    rc, msg = _create(rh, path, w="w", b=None)
    assert rc == rh.PPOCR_ERR_MODEL, (case, rc, msg)
    assert msg.startswith("SafeTensors: "), msg


def test_header_padding_and_metadata_are_accepted(rh, tmp_path):
    """Spaces after the JSON (the format pads the header to 8 bytes) and unknown fields
    are accepted; an escaped tensor name is matched after unescaping."""
    path = str(tmp_path / "pad.safetensors")
    hdr = {"__metadata__": {"graph": "{\"a\": [1, 2]}"},
           "wé": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24], "extra": [1, {"x": None}]}}
    _raw_file(path, json.dumps(hdr).encode() + b"     ", np.zeros(6, np.float32).tobytes())
    rc, msg = _create(rh, path, w="wé", b=None)
    assert not msg.startswith(("SafeTensors", "Model")), msg
