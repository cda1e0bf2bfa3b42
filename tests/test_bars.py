"""The parity bars can fail: planted mistakes in a CPU model of the fused head's softmax
sum (a vocabulary chunk's partial sum lost or counted twice, the bias left out) pass the
1e-4 absolute bar on the synthetic workload and are caught by the relative bar that the
GPU tests apply beside it (gpu_common.assert_close_rel)."""
import numpy as np
import pytest

from gpu_common import assert_close_rel, f64_logits_q


@pytest.fixture(scope="module")
def rows(orc):
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    q, s = orc.pack_int8(w_t)
    a = wl.activations("single_line")[:16]
    ref = orc.rechead_lines(a, np.array([0, 16], np.int64), q, s, bias)
    return {"lg": f64_logits_q(a, q, s, bias), "ref": ref, "q": q, "s": s, "a": a}


def _maxprob(lg, chunks=64, drop=None, twice=None):
    e = np.exp(lg - lg.max(axis=1, keepdims=True))
    parts = np.array_split(e, chunks, axis=1)
    sums = np.stack([p.sum(axis=1) for p in parts], axis=1)
    if drop is not None:
        sums[:, drop] = 0.0
    if twice is not None:
        sums[:, twice] *= 2.0
    return (1.0 / sums.sum(axis=1)).astype(np.float32)


def test_faithful_model_passes(rows):
    assert_close_rel(_maxprob(rows["lg"]), rows["ref"]["maxprob"], "faithful")


@pytest.mark.parametrize("plant", ["drop", "twice"])
def test_lost_or_doubled_chunk_sum_is_caught(rows, plant):
    bad = _maxprob(rows["lg"], drop=5 if plant == "drop" else None, twice=5 if plant == "twice" else None)
    ref = rows["ref"]["maxprob"]
    assert np.abs(bad - ref).max() < 1e-4  # the absolute bar alone would pass it
    with pytest.raises(AssertionError):
        assert_close_rel(bad, ref, f"planted {plant}")


def test_missing_bias_is_caught(orc, rows):
    lg = f64_logits_q(rows["a"], rows["q"], rows["s"], None)
    bad = _maxprob(lg)
    assert np.abs(bad - rows["ref"]["maxprob"]).max() < 1e-4
    with pytest.raises(AssertionError):
        assert_close_rel(bad, rows["ref"]["maxprob"], "planted no-bias")
