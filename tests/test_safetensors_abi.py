"""Model-file errors of ppocr_rh_create_from_safetensors, checked on the CPU: every
malformed file or tensor is reported as PPOCR_ERR_MODEL (OcrError::SafeTensorsError /
ModelError, src/engine/loader.rs:34-92) before any device is touched.  Files are written
with the safetensors package (the format the reference's loader reads) or by hand for the
malformed cases."""
import ctypes
import json
import os
import re
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


# ---------------------------------------------------------------- the head in the graph
def _graph_file(tmp_path, nodes, outputs=("probs",), inputs=("x",), name="g.safetensors", graph=None, n=70, k=120,
                with_bias=True):
    from safetensors.numpy import save_file
    t = {"linear_8.w_0": np.zeros((k, n), np.float32), "other.w": np.zeros((4, 4), np.float32),
         "other.b": np.zeros(4, np.float32)}
    if with_bias:
        t["linear_8.b_0"] = np.zeros(n, np.float32)
    g = graph if graph is not None else json.dumps({"inputs": list(inputs), "outputs": list(outputs), "nodes": nodes})
    path = str(tmp_path / name)
    save_file(t, path, metadata={"graph": g})
    return path


def _node(name, op, inputs, outputs, attrs=None):
    d = {"name": name, "op": op, "inputs": inputs, "outputs": outputs}
    if attrs is not None:
        d["attrs"] = attrs
    return d


NECK = [_node("MatMul.11", "MatMul", ["h", "other.w"], ["x2"])]
HEAD = [_node("MatMul.12", "MatMul", ["x2", "linear_8.w_0"], ["mm"]),
        _node("Add.9", "Add", ["mm", "linear_8.b_0"], ["logits"]),
        _node("Softmax.2", "Softmax", ["logits"], ["probs"], {"axis": -1})]


def test_find_head_in_the_graph(rh, tmp_path):
    """The MatMul.12 -> Add -> Softmax.2 -> output tail of the recognition model."""
    r = rh.find_rec_head(_graph_file(tmp_path, NECK + HEAD))
    assert r == {"weight": "linear_8.w_0", "bias": "linear_8.b_0", "n": 70, "k": 120}


@pytest.mark.parametrize("variant", ["bias_first", "no_bias", "identities", "no_axis", "tiny", "transpose_axis2",
                                     "two_matmuls_axis2"])
def test_find_head_variants(rh, tmp_path, variant):
    nodes = [dict(n) for n in NECK + HEAD]
    n, k, with_bias = 70, 120, True
    outputs = ("probs",)
    if variant == "bias_first":
        nodes[2]["inputs"] = ["linear_8.b_0", "mm"]
    elif variant == "no_bias":
        nodes = NECK + [_node("MatMul.12", "MatMul", ["x2", "linear_8.w_0"], ["logits"]),
                        _node("Softmax.2", "Softmax", ["logits"], ["probs"])]
        with_bias = False
    elif variant == "identities":
        nodes = NECK + [HEAD[0], HEAD[1], _node("Identity.1", "Identity", ["logits"], ["logits2"]),
                        _node("Softmax.2", "Softmax", ["logits2"], ["p"], {"axis": -1}),
                        _node("Identity.2", "Identity", ["p"], ["probs"])]
    elif variant == "no_axis":
        del nodes[3]["attrs"]
    elif variant == "tiny":
        n, k = 6906, 80
    elif variant == "transpose_axis2":  # the small PP-OCRv6 model's tail: a rank-3 softmax on axis 2
        nodes = [_node("Transpose.8", "Transpose", ["h"], ["x2"], {"perm": [0, 2, 1]})] + [dict(x) for x in HEAD]
        nodes[-1]["attrs"] = {"axis": 2}
    elif variant == "two_matmuls_axis2":  # the tiny model's tail: the rank traced through a MatMul and an Add
        nodes = [_node("Transpose.2", "Transpose", ["h"], ["t"], {"perm": [0, 2, 1]}),
                 _node("MatMul.0", "MatMul", ["t", "other.w"], ["m0"]),
                 _node("Add.104", "Add", ["m0", "other.b"], ["a0"]),
                 _node("Identity.89", "Identity", ["a0"], ["x2"])] + [dict(x) for x in HEAD]
        nodes[-1]["attrs"] = {"axis": 2}
    r = rh.find_rec_head(_graph_file(tmp_path, nodes, outputs, n=n, k=k, with_bias=with_bias))
    assert r == {"weight": "linear_8.w_0", "bias": None if variant == "no_bias" else "linear_8.b_0", "n": n, "k": k}


@pytest.mark.parametrize("variant,msg", [
    ("axis_1", "no MatMul"), ("not_output", "no MatMul"), ("logits_used_twice", "no MatMul"),
    ("weight_missing", "no MatMul"), ("no_graph", "missing 'graph'"), ("bad_json", "failed to parse graph JSON"),
    ("empty_outputs", "both must be non-empty"), ("no_outputs", "declares no outputs"),
    ("transpose_axis1", "no MatMul"), ("axis2_rank_unknown", "no MatMul")])
def test_find_head_rejects(rh, tmp_path, variant, msg):
    nodes = [dict(n) for n in NECK + HEAD]
    outputs, graph = ("probs",), None
    if variant == "axis_1":
        nodes[3]["attrs"] = {"axis": 1}
    elif variant == "not_output":
        nodes.append(_node("Mul.1", "Mul", ["probs", "probs"], ["y"]))
        outputs = ("y",)
    elif variant == "logits_used_twice":
        outputs = ("probs", "mm")
    elif variant == "weight_missing":
        nodes[1]["inputs"] = ["x2", "linear_9.w_0"]
    elif variant == "bad_json":
        graph = '{"inputs": ["x"], "outputs": ["probs"], "nodes": [}'
    elif variant == "empty_outputs":
        nodes[0]["outputs"] = []
    elif variant == "no_outputs":
        outputs = ()
    elif variant == "transpose_axis1":  # a softmax over the steps, not the classes
        nodes = [_node("Transpose.8", "Transpose", ["h"], ["x2"], {"perm": [0, 2, 1]})] + [dict(x) for x in HEAD]
        nodes[-1]["attrs"] = {"axis": 1}
    elif variant == "axis2_rank_unknown":  # no Transpose to give the rank: axis 2 may not be the last
        nodes[3]["attrs"] = {"axis": 2}
    if variant == "no_graph":
        from safetensors.numpy import save_file
        path = str(tmp_path / "nograph.safetensors")
        save_file({"linear_8.w_0": np.zeros((120, 70), np.float32)}, path)
    else:
        path = _graph_file(tmp_path, nodes, outputs, graph=graph)
    with pytest.raises(rh.OcrError) as ei:
        rh.find_rec_head(path)
    assert ei.value.code == rh.PPOCR_ERR_MODEL and msg in str(ei.value), str(ei.value)


def test_find_head_name_buffer_too_small(rh, tmp_path):
    path = _graph_file(tmp_path, NECK + HEAD)
    w, b = ctypes.create_string_buffer(5), ctypes.create_string_buffer(64)
    rc = rh._lib.lib().ppocr_model_find_rec_head(os.fsencode(path), w, 5, b, 64, None, None)
    assert rc == rh.PPOCR_ERR_INVALID_ARG and "does not fit" in rh._lib.last_error()


def _mutated_files(tmp_path, count=300, seed=77):
    """Seeded truncations and byte mutations of a valid model file with a graph (header
    length field, header JSON, graph JSON, data), written under tmp_path; the valid file
    first."""
    src = _graph_file(tmp_path, NECK + HEAD)
    blob = open(src, "rb").read()
    hlen = struct.unpack("<Q", blob[:8])[0]
    rng = np.random.default_rng(seed)
    cases = [src]
    for x in range(count):
        b = bytearray(blob)
        kind = x % 4
        if kind == 0:  # truncation anywhere
            b = b[:int(rng.integers(0, len(blob)))]
        elif kind == 1:  # bytes of the header JSON replaced
            for _ in range(int(rng.integers(1, 6))):
                b[8 + int(rng.integers(0, hlen))] = int(rng.choice(list(b'{}[]",:0-9e\\ ')))
        elif kind == 2:  # the header length field
            vals = [0, 1, hlen - 1, hlen + 1, len(blob), 2**63 - 1, 2**64 - 1]
            b[:8] = struct.pack("<Q", vals[int(rng.integers(0, len(vals)))])
        else:  # a digit of an offset or shape changed
            digits = [i for i in range(8, 8 + hlen) if chr(b[i]).isdigit()]
            b[digits[int(rng.integers(0, len(digits)))]] = ord(str(int(rng.integers(0, 10))))
        p = tmp_path / f"m{x}.safetensors"
        p.write_bytes(bytes(b))
        cases.append(str(p))
    return cases


def test_mutated_files_never_crash(rh, tmp_path):
    """The parser returns PPOCR_OK or PPOCR_ERR_MODEL for each seeded mutation of a valid
    model file, never crashes.  Runs in a child process so that a crash fails this test
    alone."""
    import subprocess
    import sys
    cases = _mutated_files(tmp_path)
    code = r"""
import ctypes, os, sys
import ppocr_rechead as rh
L = rh._lib.lib()
seen = set()
for path in sys.argv[1:]:
    w, b = ctypes.create_string_buffer(256), ctypes.create_string_buffer(256)
    n, k = ctypes.c_int64(), ctypes.c_int64()
    rc = L.ppocr_model_find_rec_head(os.fsencode(path), w, 256, b, 256, ctypes.byref(n), ctypes.byref(k))
    seen.add(rc)
print(sorted(seen))
"""
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([os.path.join(os.path.dirname(os.path.dirname(
        os.path.abspath(__file__))), "rust-ppocrv6_amd")]))
    out = subprocess.run([sys.executable, "-c", code] + cases, env=env, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, (out.returncode, out.stderr[-2000:])
    seen = set(json.loads(out.stdout.strip().splitlines()[-1]))
    assert seen <= {rh.PPOCR_OK, rh.PPOCR_ERR_MODEL}, seen
    assert rh.PPOCR_ERR_MODEL in seen


def test_mutated_files_under_address_sanitizer(tmp_path):
    """The host-only sanitizer build of the parser and the graph search (`make asan` in
    rust-ppocrv6_amd/csrc: AddressSanitizer and UndefinedBehaviorSanitizer, any finding
    fatal) over the same seeded mutations, more of them, and the reference's model files
    where they are mounted: no finding, no crash."""
    import glob
    import shutil
    import subprocess
    if not shutil.which("g++"):
        pytest.skip("no host C++ compiler")
    csrc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "rust-ppocrv6_amd", "csrc")
    build = subprocess.run(["make", "-C", csrc, "asan"], capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-2000:]
    exe = os.path.join(csrc, "..", "lib", "_asan", "parser_check")
    cases = _mutated_files(tmp_path, count=1200, seed=78)
    cases += sorted(glob.glob("/root/reference/models/*.safetensors"))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    out = subprocess.run([exe] + cases, capture_output=True, text=True, timeout=600, env=env)
    assert out.returncode == 0, (out.returncode, out.stderr[-3000:])
    assert "Sanitizer" not in out.stderr and "runtime error" not in out.stderr, out.stderr[-3000:]
    acc, ref = map(int, re.search(r"accepted (\d+) refused (\d+)", out.stdout).groups())
    print(f"parser under ASan/UBSan: {acc} accepted, {ref} refused")
    assert acc >= 1 and ref >= 1 and acc + ref == len(cases)


@pytest.mark.skipif(not os.path.isdir("/root/reference/models"), reason="reference model files not mounted")
def test_find_head_in_the_reference_models(rh):
    """The reference's own model files: the small and tiny recognition models' heads are
    found (Softmax on axis 2 of a rank-3 tensor, the rank traced to Transpose.8); the
    classifier and the detectors have none."""
    d = "/root/reference/models"
    assert rh.find_rec_head(os.path.join(d, "PP-OCRv6_small_rec.safetensors")) == {
        "weight": "linear_8.w_0", "bias": "linear_8.b_0", "n": 18710, "k": 120}
    assert rh.find_rec_head(os.path.join(d, "PP-OCRv6_tiny_rec.safetensors")) == {
        "weight": "linear_1.w_0", "bias": "linear_1.b_0", "n": 6906, "k": 80}
    for name in ("PP-OCRv6_cls", "PP-OCRv6_small_det", "PP-OCRv6_tiny_det"):
        with pytest.raises(rh.OcrError) as ei:
            rh.find_rec_head(os.path.join(d, name + ".safetensors"))
        assert ei.value.code == rh.PPOCR_ERR_MODEL
