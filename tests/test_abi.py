"""CPU-side checks of the C ABI: the library loads, exports every function the header
declares, and reports argument errors (the OcrError::OperatorError convention) without
touching a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ppocr_rechead.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ppocr_\w+)\s*\(", text)))


def test_header_and_binding_agree(rh):
    names = declared_functions()
    assert len(names) >= 20
    assert set(names) == set(rh._lib.SIGNATURES), set(names) ^ set(rh._lib.SIGNATURES)


def test_library_exports_every_declared_symbol(rh):
    L = rh._lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), name


def test_library_is_built_for_gfx950_only():
    """The embedded offload bundle of this repository's own build names gfx950 and no
    other GPU target."""
    lib = os.path.join(ROOT, "rust-ppocrv6_amd", "lib", "libppocr_rechead.so")
    blob = open(lib, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa-+(gfx[0-9a-f]+)", blob))
    assert targets == {b"gfx950"}, targets


def test_argument_errors_do_not_need_a_device(rh):
    L = rh._lib.lib()
    rc = L.ppocr_rh_pack_int8(None, -1, 120, None, None)
    assert rc == rh.PPOCR_ERR_INVALID_ARG
    assert rh._lib.last_error() == "QuantizedWeight: negative shape"
    assert L.ppocr_rh_pack_int8(None, 0, 120, None, None) == rh.PPOCR_OK
    h = ctypes.c_void_p(123)
    assert L.ppocr_rh_create(None, None, None, 10, 8, 0, ctypes.byref(h)) == rh.PPOCR_ERR_INVALID_ARG
    assert h.value is None
    assert "MatMulQuantizedB" in rh._lib.last_error()
    assert L.ppocr_ctc_greedy(None, None, None, -1, 0, None, None, None) == rh.PPOCR_ERR_INVALID_ARG
    assert L.ppocr_ctc_greedy(None, None, None, 0, 0, None, None, None) == rh.PPOCR_OK
    off = np.array([0, 3, 2], np.int64)
    rc = L.ppocr_ctc_greedy(None, None, off.ctypes.data_as(ctypes.c_void_p), 2, 0, None,
                            np.zeros(2, np.int64).ctypes.data_as(ctypes.c_void_p),
                            np.zeros(2, np.float32).ctypes.data_as(ctypes.c_void_p))
    assert rc == rh.PPOCR_ERR_INVALID_ARG and "non-decreasing" in rh._lib.last_error()
    assert L.ppocr_softmax_rows(None, 0, 5) == rh.PPOCR_OK  # empty input is not an error
    assert L.ppocr_softmax_rows(None, -1, 5) == rh.PPOCR_ERR_INVALID_ARG
    assert L.ppocr_rh_footprint_bytes(None) == 0
    assert L.ppocr_rh_auto_mode(None) == -1
    assert L.ppocr_rh_guard_limits(None, 2, None, None, None) == rh.PPOCR_ERR_INVALID_ARG
    assert L.ppocr_rn_gemm_halves(None) == rh.PPOCR_ERR_INVALID_ARG
    assert rh._lib.last_error() == "RecNeckHip: null neck handle"
    assert L.ppocr_rh_logits(None, None, 1, 2, None) == rh.PPOCR_ERR_INVALID_ARG
    assert rh._lib.last_error() == "MatMulQuantizedB: null head handle"


def test_python_mirror_errors_match_the_reference_messages(rh):
    with pytest.raises(rh.OcrError) as e:
        rh.softmax(np.zeros((2, 3), np.float32), 2)
    assert str(e.value) == "Softmax: Axis 2 out of bounds for ndim 2"
    with pytest.raises(rh.OcrError):
        rh.softmax(np.zeros((2, 3), np.float32), -3)
    dec = rh.CtcDecoder.from_vocab(["blank", "a", " "])
    with pytest.raises(rh.OcrError) as e:
        dec.decode(np.zeros((1, 2, 4), np.float32))
    assert "mismatch" in str(e.value)
    with pytest.raises(rh.OcrError):
        dec.decode(np.zeros((2, 2), np.float32))
    # an empty batch decodes to ("", 0.0) (decode_handles_empty_batch_gracefully)
    assert dec.decode(np.zeros((0, 5, 3), np.float32)) == ("", 0.0)
    qw = rh.QuantizedWeight(np.zeros((16, 8), np.int8), np.ones(16, np.float32))
    for n_bias in (0, 1, 15, 17):
        with pytest.raises(rh.OcrError):
            rh.matmul_quantized_b(np.zeros((1, 8), np.float32), qw, np.zeros(n_bias, np.float32))
    with pytest.raises(rh.OcrError) as e:
        rh.matmul_quantized_b(np.zeros((2, 3), np.float32), qw)
    assert "Inner dimensions must match: 3 != 8" in str(e.value)


def test_dictionary_loading(rh, tmp_path):
    p = tmp_path / "keys.txt"
    p.write_text("a\nb\r\nc\n", encoding="utf-8")
    dec = rh.CtcDecoder.from_file(str(p))
    assert dec.vocab == ["blank", "a", "b", "c", " "]
    ref_keys = "/root/reference/models/ppocrv6_keys.txt"
    if os.path.exists(ref_keys):
        assert rh.CtcDecoder.from_file(ref_keys).vocab_size() == 18710
        # the tiny model's dictionary matches its head's 6906 classes
        assert rh.CtcDecoder.from_file("/root/reference/models/ppocrv6_tiny_keys.txt").vocab_size() == 6906


def test_dictionary_lines_split_on_newline_only(rh, tmp_path):
    """BufRead::lines splits on '\n' alone and trim_end_matches drops trailing '\r' / '\n'
    (src/postprocess/ctc.rs:20-23): a lone '\r' inside an entry stays in it, so later class
    indices do not shift; invalid UTF-8 is a ModelError; a missing final newline or an
    empty file changes nothing else."""
    p = tmp_path / "keys.txt"
    p.write_bytes("x\ry\nb\r\r\nc".encode("utf-8"))
    assert rh.CtcDecoder.from_file(str(p)).vocab == ["blank", "x\ry", "b", "c", " "]
    p.write_bytes(b"")
    assert rh.CtcDecoder.from_file(str(p)).vocab == ["blank", " "]
    p.write_bytes(b"\n\n")
    assert rh.CtcDecoder.from_file(str(p)).vocab == ["blank", "", "", " "]
    p.write_bytes(b"a\n\xff\xfe\n")
    with pytest.raises(rh.OcrError) as e:
        rh.CtcDecoder.from_file(str(p))
    assert e.value.op == "ModelError" and "Dict read error" in str(e.value)
    with pytest.raises(rh.OcrError) as e:
        rh.CtcDecoder.from_file(str(tmp_path / "missing.txt"))
    assert e.value.op == "ModelError" and "Failed to open dict file" in str(e.value)


def test_engine_config_backend_selector(rh):
    """OcrEngineConfig keeps the reference's quantize_rec_head default (False) and adds the
    backend selector; an unknown backend is a ModelError, and the CPU backend builds no
    head (nothing touches a GPU)."""
    cfg = rh.OcrEngineConfig()
    assert cfg.quantize_rec_head is False and cfg.rec_head_backend == "cpu"
    assert rh.RecHead.for_config(cfg, "/nonexistent/model.safetensors") is None
    cfg.enable_rec_quantization()
    assert cfg.quantize_rec_head is True
    with pytest.raises(rh.OcrError) as e:
        rh.OcrEngineConfig(rec_head_backend="cuda")
    assert e.value.op == "ModelError"


def test_workloads_are_deterministic():
    from ppocr_rechead import workloads as wl
    w1, b1 = wl.weights()
    w2, b2 = wl.weights()
    assert w1.shape == (18710, 120) and np.array_equal(w1, w2) and np.array_equal(b1, b2)
    lines = wl.lines_for("a4_page")
    assert len(lines) == 29 and all(20 <= t <= 120 for t in lines)
    assert sum(wl.lines_for("dense_256")) == 30720
    assert sum(wl.lines_for("stress_1024")) == 245760
    ws, _ = wl.weights(stress=True)
    zero_rows = np.nonzero(~ws.any(axis=1))[0]
    assert zero_rows.size == 18710 // 200
    assert (np.abs(ws) == 5.0).sum() == 18710 // 200


def test_decode_dev_argument_errors_do_not_need_a_device(rh):
    """ppocr_rh_decode_dev rejects a null head, negative counts and missing outputs before
    any HIP call; zero lines is a no-op."""
    L = rh._lib.lib()
    args = (None, 0, None, 1, 2, None, None, None, None, None, None, 0, None)
    assert L.ppocr_rh_decode_dev(None, *args) == rh.PPOCR_ERR_INVALID_ARG
    assert rh._lib.last_error() == "RecHeadHip: null head handle"
    assert L.ppocr_rh_decode(None, None, None, 1, 2, None, None, None, None, None) == rh.PPOCR_ERR_INVALID_ARG
    assert L.ppocr_rh_decode_nct(None, None, 1, 120, 2, None, None, None, None, None) == rh.PPOCR_ERR_INVALID_ARG
    assert L.ppocr_rh_decode_nct_dev(None, None, 1, 120, 2, None, None, None, None, None, None, 0,
                                     None) == rh.PPOCR_ERR_INVALID_ARG
    assert rh._lib.last_error() == "RecHeadHip: null head handle"


def test_missing_library_fails_loudly(tmp_path):
    """With the HIP library absent, every compute entry of the mirror raises; nothing falls
    back to a CPU path."""
    import subprocess
    import sys
    code = r"""
import numpy as np
import ppocr_rechead as rh
calls = {
    "softmax_inplace": lambda: rh.softmax_inplace(np.zeros((1, 4), np.float32)),
    "pack": lambda: rh.QuantizedWeight.from_f32_transposed(np.ones((3, 4), np.float32)),
    "matmul_quantized_b": lambda: rh.matmul_quantized_b(
        np.ones((1, 4), np.float32), rh.QuantizedWeight(np.ones((3, 4), np.int8), np.ones(3, np.float32))),
    "collapse": lambda: rh.CtcDecoder.collapse(np.zeros(2, np.int32), np.zeros(2, np.float32),
                                               np.array([0, 2], np.int64)),
}
for name, f in calls.items():
    try:
        f()
        print(name, "RETURNED")
    except RuntimeError as e:
        print(name, "RAISED", "not found" in str(e))
"""
    env = dict(os.environ, PPOCR_RECHEAD_LIB=str(tmp_path / "absent" / "libppocr_rechead.so"),
               PYTHONPATH=os.pathsep.join([os.path.join(ROOT, "rust-ppocrv6_amd"), ROOT]))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    lines = dict(l.split(" ", 1) for l in out.stdout.strip().splitlines())
    assert lines == {k: "RAISED True" for k in ("softmax_inplace", "pack", "matmul_quantized_b", "collapse")}, out.stdout
