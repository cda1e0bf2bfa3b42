"""A head created from a model file (ppocr_rh_create_from_safetensors: transpose, INT8
packing, guard limits and tile records on the device) equals the head created from the
host-transposed weight (ppocr_rh_create / ppocr_rh_create_f32), bit for bit in every
output, for the PP-OCRv6 small head (120 x 18710), the tiny head's k = 80 and shapes
without an MFMA path."""
import numpy as np
import pytest

from gpu_common import assert_close_rel, check_argmax, f64_logits_q, top2_gap

pytestmark = pytest.mark.gpu


def _save(tmp_path, w_kn, bias, name="rec.safetensors"):
    from safetensors.numpy import save_file
    path = str(tmp_path / name)
    t = {"linear_8.w_0": np.ascontiguousarray(w_kn, np.float32)}
    if bias is not None:
        t["linear_8.b_0"] = np.ascontiguousarray(bias, np.float32)
    save_file(t, path, metadata={"graph": "{}"})
    return path


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("k,n,with_bias", [(120, 18710, True), (80, 6906, True), (120, 70, False), (50, 33, True)])
def test_int8_head_from_file_equals_host_packed(orc, rh, tmp_path, k, n, with_bias):
    rng = np.random.default_rng(k * 7 + n)
    w_t = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    w_t[3] = 0.0                       # an all-zero class: scale 1.0
    w_t[5, 7] = 5.0                    # an outlier class
    bias = (rng.standard_normal(n) * 0.01).astype(np.float32) if with_bias else None
    path = _save(tmp_path, w_t.T, bias)
    print(f"model file head k={k} n={n} bias={with_bias}", flush=True)
    hf = rh.RecHead.from_safetensors(path, "linear_8.w_0", "linear_8.b_0" if with_bias else None)
    q, s = orc.pack_int8(w_t)
    hh = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    assert (hf.n, hf.k, hf.quantized) == (n, k, True)
    assert hf.weight_footprint_bytes() == hh.weight_footprint_bytes() == n * k + 4 * n
    assert hf.device_bytes() == hh.device_bytes()
    a = rng.standard_normal((300, k)).astype(np.float32)
    a[::37] *= np.float32(40.0)        # rows over the precision guard
    modes = (0, 2, 3, 4) if k in (120, 80) else (0,)
    for mode in modes:
        _same(hf.logits(a, mode), hh.logits(a, mode))
        i1, p1 = hf.argmax(a, mode)
        i2, p2 = hh.argmax(a, mode)
        _same(i1, i2)
        _same(p1, p2)
    if k in (120, 80):
        _same(hf.probs(a[:40], 2), hh.probs(a[:40], 2))
        idx, _ = hf.argmax(a, 2)
        ref = orc.rechead_lines(a, np.array([0, 300], np.int64), q, s, bias)
        check_argmax(idx, ref["idx"], top2_gap(f64_logits_q(a, q, s, bias)), label=f"file head k={k}")
    hf.close()
    hh.close()


@pytest.mark.parametrize("k,n", [(120, 18710), (80, 6906), (50, 33)])
def test_fp32_head_from_file_equals_host_transposed(rh, tmp_path, k, n):
    rng = np.random.default_rng(k + n)
    w_t = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
    path = _save(tmp_path, w_t.T, bias)
    print(f"model file fp32 head k={k} n={n}", flush=True)
    hf = rh.RecHead.from_safetensors(path, "linear_8.w_0", "linear_8.b_0", quantize=False)
    hh = rh.RecHead(w_t=w_t, bias=bias)
    assert (hf.n, hf.k, hf.quantized) == (n, k, False)
    assert hf.weight_footprint_bytes() == hh.weight_footprint_bytes() == 4 * n * k
    assert hf.device_bytes() == hh.device_bytes()
    a = rng.standard_normal((200, k)).astype(np.float32)
    for mode in ((0, 1, 3, 4) if k in (120, 80) else (0,)):
        _same(hf.logits(a, mode), hh.logits(a, mode))
        i1, p1 = hf.argmax(a, mode)
        i2, p2 = hh.argmax(a, mode)
        _same(i1, i2)
        _same(p1, p2)
    hf.close()
    hh.close()


def test_head_found_in_the_model_graph(orc, rh, tmp_path):
    """RecHead.from_model finds MatMul.12 -> Add -> Softmax.2 in the file's graph and builds
    the same head as naming its tensors; the whole-head decode agrees with the oracle."""
    import json
    from safetensors.numpy import save_file
    from gpu_common import assert_close_rel, check_argmax, f64_logits_q, top2_gap
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    graph = {"inputs": ["x"], "outputs": ["probs"], "nodes": [
        {"name": "MatMul.12", "op": "MatMul", "inputs": ["x", "linear_8.w_0"], "outputs": ["mm"]},
        {"name": "Add.9", "op": "Add", "inputs": ["mm", "linear_8.b_0"], "outputs": ["logits"]},
        {"name": "Softmax.2", "op": "Softmax", "inputs": ["logits"], "outputs": ["probs"], "attrs": {"axis": -1}}]}
    path = str(tmp_path / "rec.safetensors")
    save_file({"linear_8.w_0": np.ascontiguousarray(w_t.T), "linear_8.b_0": bias}, path,
              metadata={"graph": json.dumps(graph)})
    print("head from the model graph", flush=True)
    hm = rh.RecHead.from_model(path)
    hs = rh.RecHead.from_safetensors(path, "linear_8.w_0", "linear_8.b_0")
    a = wl.activations("a4_page")
    off = wl.line_offsets(wl.lines_for("a4_page"))
    gm, gs = hm.decode(a, off), hs.decode(a, off)
    _same(gm["idx"], gs["idx"])
    _same(gm["maxprob"], gs["maxprob"])
    _same(gm["score"], gs["score"])
    q, s = orc.pack_int8(w_t)
    ref = orc.rechead_lines(a, off, q, s, bias)
    check_argmax(gm["idx"], ref["idx"], top2_gap(f64_logits_q(a, q, s, bias)), label="model graph head")
    assert_close_rel(gm["maxprob"], ref["maxprob"], "model-file head maxprob")
    hm.close()
    hs.close()


def test_head_found_in_a_pp_ocr_v6_style_graph(orc, rh, tmp_path):
    """The tail as the reference's small recognition model carries it (Squeeze ->
    Transpose.8 perm [0,2,1] -> MatMul.12 -> Add.204 -> Identity.210 -> Softmax.2 axis 2 ->
    fetch_name_0): RecHead.from_model finds the head, and fed the Transpose.8 input
    (channels first, decode_nct) it gives the results of the head built from the tensor
    names on the transposed rows, bit for bit, within the bars against the oracle."""
    import json
    from safetensors.numpy import save_file
    from gpu_common import assert_close_rel, check_argmax, f64_logits_q, top2_gap
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    graph = {"inputs": ["x"], "outputs": ["fetch_name_0"], "nodes": [
        {"name": "Squeeze.7", "op": "Squeeze", "inputs": ["p2o.pd_op.add.78.0"], "outputs": ["p2o.pd_op.squeeze.0.0"],
         "attrs": {"axes": [2]}},
        {"name": "Transpose.8", "op": "Transpose", "inputs": ["p2o.pd_op.squeeze.0.0"],
         "outputs": ["p2o.pd_op.transpose.8.0"], "attrs": {"perm": [0, 2, 1]}},
        {"name": "MatMul.12", "op": "MatMul", "inputs": ["p2o.pd_op.transpose.8.0", "linear_8.w_0"],
         "outputs": ["p2o.pd_op.matmul.12.0"], "attrs": {}},
        {"name": "Add.204", "op": "Add", "inputs": ["p2o.pd_op.matmul.12.0", "linear_8.b_0"], "outputs": ["Add.205"],
         "attrs": {}},
        {"name": "Identity.210", "op": "Identity", "inputs": ["Add.205"], "outputs": ["p2o.pd_op.add.79.0"],
         "attrs": {}},
        {"name": "Softmax.2", "op": "Softmax", "inputs": ["p2o.pd_op.add.79.0"], "outputs": ["fetch_name_0"],
         "attrs": {"axis": 2}}]}
    path = str(tmp_path / "rec_v6.safetensors")
    save_file({"linear_8.w_0": np.ascontiguousarray(w_t.T), "linear_8.b_0": bias}, path,
              metadata={"graph": json.dumps(graph)})
    print("head from a PP-OCRv6-style graph", flush=True)
    hm = rh.RecHead.from_model(path)
    hs = rh.RecHead.from_safetensors(path, "linear_8.w_0", "linear_8.b_0")
    rng = np.random.default_rng(23)
    lines, T = 12, 120
    x = rng.standard_normal((lines, 120, T)).astype(np.float32)  # the Transpose.8 input
    a = np.ascontiguousarray(x.transpose(0, 2, 1).reshape(-1, 120))
    off = np.arange(lines + 1, dtype=np.int64) * T
    gm, gs = hm.decode_nct(x), hs.decode(a, off)
    _same(gm["idx"], gs["idx"])
    _same(gm["maxprob"], gs["maxprob"])
    _same(gm["score"], gs["score"])
    q, s = orc.pack_int8(w_t)
    ref = orc.rechead_lines(a, off, q, s, bias)
    check_argmax(gm["idx"], ref["idx"], top2_gap(f64_logits_q(a, q, s, bias)), label="v6-style graph head")
    assert_close_rel(gm["maxprob"], ref["maxprob"], "model-file head maxprob")
    hm.close()
    hs.close()


def test_backend_switch_builds_the_configured_head(orc, rh, tmp_path):
    """OcrEngineConfig's INT8 switch is unchanged and the backend selector picks the head:
    "hip" with quantize_rec_head builds the INT8 head (the packing of
    Model::quantize_matmul_weights, bit for bit), "hip" without it the FP32 head, and
    enable_rec_quantization turns a later build INT8 (src/pipeline.rs:38-40, 195-199, 267-270);
    "cpu" builds nothing on the GPU."""
    import json
    from safetensors.numpy import save_file
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights(n=700)
    graph = {"inputs": ["x"], "outputs": ["probs"], "nodes": [
        {"name": "MatMul.12", "op": "MatMul", "inputs": ["x", "linear_8.w_0"], "outputs": ["mm"]},
        {"name": "Add.9", "op": "Add", "inputs": ["mm", "linear_8.b_0"], "outputs": ["logits"]},
        {"name": "Softmax.2", "op": "Softmax", "inputs": ["logits"], "outputs": ["probs"]}]}
    path = str(tmp_path / "rec.safetensors")
    save_file({"linear_8.w_0": np.ascontiguousarray(w_t.T), "linear_8.b_0": bias}, path,
              metadata={"graph": json.dumps(graph)})
    print("backend switch", flush=True)
    assert rh.RecHead.for_config(rh.OcrEngineConfig(quantize_rec_head=True), path) is None
    cfg = rh.OcrEngineConfig(rec_head_backend="hip")
    h32 = rh.RecHead.for_config(cfg, path)
    assert (h32.quantized, h32.n, h32.k) == (False, 700, 120)
    assert h32.weight_footprint_bytes() == 4 * 700 * 120
    cfg.enable_rec_quantization()
    h8 = rh.RecHead.for_config(cfg, path)
    assert (h8.quantized, h8.n, h8.k) == (True, 700, 120)
    assert h8.weight_footprint_bytes() == 700 * 120 + 4 * 700
    q, s = orc.pack_int8(w_t)
    a = np.random.default_rng(3).standard_normal((50, 120)).astype(np.float32)
    assert np.abs(h8.logits(a) - orc.matmul_quantized_b(a, q, s, bias)).max() < 1e-4
    assert np.abs(h32.logits(a) - orc.matmul_transposed_b(a, w_t, bias)).max() < 1e-4
    h8.close()
    h32.close()
