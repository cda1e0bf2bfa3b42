"""Pins the oracle's softmax (src/ops/softmax.rs), argmax and CTC collapse
(src/postprocess/ctc.rs) against f64 closed forms and the reference's own known-answer
tests, restated with their inputs and tolerances."""
import numpy as np
import pytest


def softmax_f64(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def test_softmax_last_axis_reference_test(orc):
    """softmax_matches_f64_reference_on_last_axis (src/ops/softmax.rs:481-506)."""
    data = np.array([[1, 2, 3, 4, 5], [-1, 0, 0, 0.5, 100], [0.25, -0.25, 0.75, -0.75, 0]], np.float32)
    for avx2 in (True, False):
        out = orc.softmax_rows(data, use_avx2=avx2)
        assert np.abs(out - softmax_f64(data)).max() <= 1e-6
        assert np.all(np.abs(out.sum(axis=1) - 1) < 1e-5)


def test_softmax_large_magnitudes_reference_test(orc):
    """softmax_is_stable_on_large_magnitudes (src/ops/softmax.rs:522-540)."""
    data = np.array([[1000, 1001, 999, 1000.5], [-1000, -999, -1001, -1000.5]], np.float32)
    out = orc.softmax_rows(data)
    assert np.all(np.isfinite(out))
    assert np.all(np.abs(out.sum(axis=1) - 1) < 1e-5)


def test_softmax_empty_and_single_row(orc):
    for shape in ((0,), (3, 0), (2, 5, 0)):
        out = orc.softmax_rows(np.zeros(shape, np.float32))
        assert out.shape == shape
    out = orc.softmax_rows(np.array([1, 2, 3], np.float32))
    assert abs(out.sum() - 1) < 1e-6 and out[2] > out[1]


def test_softmax_avx2_matches_scalar_reference_test(orc):
    """softmax_avx2_row_matches_scalar (src/ops/softmax.rs:578-598): rows of 40."""
    i = np.arange(1600)
    data = (np.sin(i.astype(np.float32) * np.float32(0.113)) * np.float32(6.0) + (i % 7).astype(np.float32) * np.float32(0.5))
    data = data.astype(np.float32).reshape(40, 40)
    a = orc.softmax_rows(data, use_avx2=True)
    b = orc.softmax_rows(data, use_avx2=False)
    assert np.all(np.abs(a - b) <= 1e-6 + 1e-5 * np.abs(b))


def test_softmax_vocab_rows_match_f64(orc):
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((16, 18710), dtype=np.float32) * np.float32(0.6)).astype(np.float32)
    x[3] *= 40  # peaked row
    for avx2 in (True, False):
        out = orc.softmax_rows(x, use_avx2=avx2)
        ref = softmax_f64(x)
        assert np.abs(out - ref).max() <= 1e-6
        assert np.all(np.abs(out.astype(np.float64).sum(axis=1) - 1) < 1e-5)


def test_exp_polynomial_accuracy(orc):
    """avx2_exp_ps (src/ops/softmax.rs:5-47) stays within a few ulp of exp over the whole
    clamped range, and exp(0) is exactly 1; a wrong constant would break this."""
    x = np.linspace(-87.0, 88.0, 800001, dtype=np.float32)
    x = x[: x.size - x.size % 8]
    got = orc.exp_ps(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    rel = np.abs(got - ref) / ref
    assert rel.max() < 4e-7
    assert orc.exp_ps(np.zeros(8, np.float32))[0] == 1.0


def test_find_argmax_reference_tests(orc):
    """test_find_argmax_avx2_matches_scalar (src/postprocess/ctc.rs:308-326)."""
    data = np.full(18710, 0.01, np.float32)
    data[42] = 0.95
    data[1000] = 0.88
    for avx2 in (True, False):
        assert orc.find_argmax(data, avx2) == (42, pytest.approx(0.95))
    data2 = np.full(35, -1.0, np.float32)
    data2[34] = 10.0
    assert orc.find_argmax(data2, True) == (34, 10.0)
    assert orc.find_argmax(data2, False) == (34, 10.0)


def test_find_argmax_first_occurrence_and_nan(orc):
    x = np.zeros(64, np.float32)
    x[[11, 3, 40]] = 2.0  # lanes 3 and 3 of different blocks, and lane 0
    for avx2 in (True, False):
        assert orc.find_argmax(x, avx2)[0] == 3
    x = np.full(40, np.nan, np.float32)
    i, v = orc.find_argmax(x, True)
    assert i == 0 and v == -np.inf
    x[17] = 1.0
    assert orc.find_argmax(x, True)[0] == 17
    assert orc.find_argmax(np.zeros(0, np.float32)) == (0, -np.inf)


def test_find_argmax_matches_numpy(orc):
    rng = np.random.default_rng(22)
    x = rng.integers(0, 50, (200, 777)).astype(np.float32)  # many ties
    idx, val = orc.argmax_rows(x)
    assert np.array_equal(idx, np.argmax(x, axis=1))
    assert np.array_equal(val, x.max(axis=1))


def _onehot(seq_len, vocab, picks):
    d = np.zeros((seq_len, vocab), np.float32)
    for t, c in picks:
        d[t, c] = 1.0
    return d


def _decode(orc, probs_btc):
    b, t, c = probs_btc.shape
    idx, val = orc.argmax_rows(probs_btc.reshape(b * t, c))
    off = np.arange(0, b * t + 1, t, dtype=np.int64)
    return orc.ctc_collapse(idx, val, off)


def test_ctc_collapse_reference_tests(orc):
    # decode_collapses_repeats_and_blank (src/postprocess/ctc.rs:272-286): a, a, blank, b -> "ab", 1.0
    seqs, score = _decode(orc, _onehot(4, 4, [(0, 1), (1, 1), (2, 0), (3, 2)])[None])
    assert seqs[0].tolist() == [1, 2] and abs(score[0] - 1.0) < 1e-6
    # decode_batch_decodes_multiple_lines (src/postprocess/ctc.rs:337-363)
    d = np.zeros((2, 2, 4), np.float32)
    d[0, 0, 1] = d[0, 1, 2] = d[1, 0, 2] = d[1, 1, 0] = 1.0
    seqs, _ = _decode(orc, d)
    assert [s.tolist() for s in seqs] == [[1, 2], [2]]


def test_ctc_collapse_closed_forms(orc):
    # last is updated on blanks: a, blank, a -> "aa"
    seqs, score = orc.ctc_collapse(np.array([1, 0, 1], np.int32), np.array([0.5, 0.9, 0.25], np.float32),
                                   np.array([0, 3], np.int64))
    assert seqs[0].tolist() == [1, 1] and score[0] == np.float32(0.375)
    # nothing emitted -> score 0; empty line -> empty
    seqs, score = orc.ctc_collapse(np.array([0, 0, 5, 5], np.int32), np.ones(4, np.float32),
                                   np.array([0, 2, 2, 4], np.int64))
    assert [s.tolist() for s in seqs] == [[], [], [5]] and score.tolist() == [0.0, 0.0, 1.0]


def test_rechead_lines_composes_the_parts(orc):
    rng = np.random.default_rng(23)
    n, k = 2048, 120
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    q, s = orc.pack_int8(w)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    off = np.array([0, 7, 7, 20, 51], np.int64)
    a = rng.standard_normal((51, k), dtype=np.float32)
    got = orc.rechead_lines(a, off, q, s, bias, want_probs=True)
    logits = orc.matmul_quantized_b(a, q, s, bias, partition_threads=1)
    probs = orc.softmax_rows(logits)
    assert np.array_equal(got["probs"].view(np.uint32), probs.view(np.uint32))
    idx, val = orc.argmax_rows(probs)
    assert np.array_equal(got["idx"], idx) and np.array_equal(got["maxprob"], val)
    seqs, score = orc.ctc_collapse(idx, val, off)
    assert all(np.array_equal(x, y) for x, y in zip(got["seqs"], seqs))
    assert np.array_equal(got["score"], score)
    # the max probability is 1/sum: the max element's exp is exactly 1
    l64 = logits.astype(np.float64)
    inv = 1.0 / np.exp(l64 - l64.max(axis=1, keepdims=True)).sum(axis=1)
    assert np.abs(got["maxprob"] - inv).max() < 1e-6
