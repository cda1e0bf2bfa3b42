"""Device-failure error paths, forced from the host: with PPOCR_RECHEAD_FAULT=alloc in the
environment every device allocation of the library fails as an exhausted HBM would, so
each entry point that allocates must return PPOCR_ERR_NO_MEMORY with an
"<op>: <msg>" message (the OcrError::OperatorError mapping, src/error.rs:4-27), launch
nothing, and leave the library usable once the condition is gone."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture
def fault():
    """Sets the allocation fault for the duration of a `with` block."""
    class _Fault:
        def __enter__(self):
            os.environ["PPOCR_RECHEAD_FAULT"] = "alloc"

        def __exit__(self, *exc):
            os.environ.pop("PPOCR_RECHEAD_FAULT", None)

    yield _Fault()
    os.environ.pop("PPOCR_RECHEAD_FAULT", None)


def test_allocation_failures_map_to_no_memory(orc, rh, fault, tmp_path):
    from safetensors.numpy import save_file
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray
    w_t, bias = wl.weights(n=1000)
    q, s = orc.pack_int8(w_t)

    print("fault: head creation", flush=True)
    with fault:
        with pytest.raises(rh.OcrError) as e:
            rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    assert e.value.code == rh.PPOCR_ERR_NO_MEMORY
    assert e.value.op == "RecHeadHip" and "device allocation failed" in e.value.msg

    path = str(tmp_path / "rec.safetensors")
    save_file({"linear_8.w_0": np.ascontiguousarray(w_t.T), "linear_8.b_0": bias}, path)
    print("fault: head from a model file", flush=True)
    with fault:
        with pytest.raises(rh.OcrError) as e:
            rh.RecHead.from_safetensors(path, "linear_8.w_0", "linear_8.b_0")
    assert e.value.code == rh.PPOCR_ERR_NO_MEMORY

    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    # host-pointer call: 80000 rows of logits need an arena above the 256 MiB kept between
    # calls, so the call allocates whatever earlier calls left in the pool
    a_big = np.zeros((80000, 120), np.float32)
    print("fault: host call arena", flush=True)
    with fault:
        with pytest.raises(rh.OcrError) as e:
            head.logits(a_big)
    assert e.value.code == rh.PPOCR_ERR_NO_MEMORY and "device allocation of" in e.value.msg

    # device call with no workspace: the stream-ordered scratch allocation fails
    m = 256
    L = rh._lib.lib()
    da = DeviceArray((m, 120), np.float32)
    di, dp = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
    print("fault: device call without a workspace", flush=True)
    with fault:
        rc = L.ppocr_rh_argmax_dev(head.handle, da.p, m, 2, di.p, dp.p, None, 0, None)
    assert rc == rh.PPOCR_ERR_NO_MEMORY
    assert L.ppocr_last_error().startswith(b"RecHeadHip: workspace allocation failed")

    # the condition gone, the same head and entry points work and agree with the oracle
    print("fault cleared: the head works", flush=True)
    a = np.random.default_rng(6).standard_normal((64, 120)).astype(np.float32)
    assert np.abs(head.logits(a) - orc.matmul_quantized_b(a, q, s, bias)).max() < 1e-4
    rh._check(L.ppocr_rh_argmax_dev(head.handle, da.p, m, 2, di.p, dp.p, None, 0, None))
    for d in (da, di, dp):
        d.free()
    head.close()


def test_errors_are_operator_errors_with_the_op_name(rh):
    """Argument errors on a live head keep the reference's op names and messages."""
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights(n=64)
    head = rh.RecHead(qw=rh.QuantizedWeight.from_f32_transposed(w_t), bias=bias)
    with pytest.raises(rh.OcrError) as e:
        head.logits(np.zeros((3, 7), np.float32))
    assert e.value.op == "MatMulQuantizedB" and e.value.code == rh.PPOCR_ERR_INVALID_ARG
    with pytest.raises(rh.OcrError) as e:
        head.logits(np.zeros((3, 120), np.float32), 9)
    assert e.value.op == "RecHeadHip" and "unknown mode 9" in e.value.msg
    head.close()
