"""Pins the oracle's projections: matmul_quantized_b (src/ops/matmul.rs:1204-1514) and
matmul_transposed_b (src/ops/matmul.rs:514-1163), against f64 brute force and the
reference's own tests (src/ops/matmul.rs:1516-1931) restated with their inputs and
tolerances."""
import numpy as np
import pytest


def f64_ref_q(a, q, s, bias=None):
    y = a.astype(np.float64) @ (q.astype(np.float64) * s.astype(np.float64)[:, None]).T
    return y + (0 if bias is None else bias.astype(np.float64))


def f64_ref_t(a, w_t, bias=None):
    y = a.astype(np.float64) @ w_t.astype(np.float64).T
    return y + (0 if bias is None else bias.astype(np.float64))


@pytest.mark.parametrize("threads", [1, 8])
@pytest.mark.parametrize("use_avx2", [True, False])
def test_int8_matches_f64(orc, threads, use_avx2):
    rng = np.random.default_rng(11)
    n, k, m = 1531, 120, 9
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    q, s = orc.pack_int8(w)
    a = rng.standard_normal((m, k), dtype=np.float32)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    got = orc.matmul_quantized_b(a, q, s, bias, partition_threads=threads, use_avx2=use_avx2)
    assert np.abs(got - f64_ref_q(a, q, s, bias)).max() < 1e-4


def test_int8_partition_changes_only_tail_columns(orc):
    """With column chunks, each chunk's last (len % 4) columns take avx2_dot_product_w8
    (src/ops/matmul.rs:1430-1441).  Every other column must be bit-identical to the
    serial path, and the set of columns that can differ is predicted exactly."""
    rng = np.random.default_rng(12)
    n, k, m = 18710, 120, 4
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    q, s = orc.pack_int8(w)
    a = rng.standard_normal((m, k), dtype=np.float32)
    serial = orc.matmul_quantized_b(a, q, s, None, partition_threads=1)
    par = orc.matmul_quantized_b(a, q, s, None, partition_threads=8)
    chunk = max(-(-n // 8), 64)
    tails = set()
    for c0 in range(0, n, chunk):
        ln = min(chunk, n - c0)
        tails.update(range(c0 + 4 * (ln // 4), c0 + ln))
    tails.update(range(4 * (n // 4), n))  # serial path's own tail
    differ = set(np.nonzero((serial.view(np.uint32) != par.view(np.uint32)).any(axis=0))[0].tolist())
    assert differ and differ <= tails
    assert np.abs(serial - par).max() < 1e-5


def test_int8_leading_batch_dims_reference_test(orc):
    """quantized_matmul_handles_leading_batch_dims (src/ops/matmul.rs:1673-1697)."""
    batch, k, n = 3, 8, 1024
    bt = np.sin(np.arange(n * k, dtype=np.float32) * np.float32(0.07)).astype(np.float32).reshape(n, k)
    q, s = orc.pack_int8(bt)
    a = np.cos(np.arange(batch * k, dtype=np.float32) * np.float32(0.11)).astype(np.float32).reshape(batch, k)
    got = orc.matmul_quantized_b(a, q, s, None, partition_threads=8)
    fp32 = orc.matmul_transposed_b(a, bt, None, partition_threads=8)
    assert np.all(np.abs(got - fp32) <= 0.05 + 0.05 * np.abs(fp32))


def test_int8_tracks_fp32_reference_test(orc):
    """matmul_quantized_b_tracks_fp32_within_quantization_error (src/ops/matmul.rs:1812-1840)."""
    k, n = 64, 48
    i = np.arange(k, dtype=np.float32)
    a = (np.sin(i * np.float32(0.19)) * np.float32(2.0)).astype(np.float32)[None, :]
    j = np.arange(n * k)
    w = (np.cos(j.astype(np.float32) * np.float32(0.07)) * np.float32(0.5) + (j % 11).astype(np.float32) * np.float32(0.01))
    w = w.astype(np.float32).reshape(n, k)
    q, s = orc.pack_int8(w)
    fp32 = orc.matmul_transposed_b(a, w, None)
    int8 = orc.matmul_quantized_b(a, q, s, None)
    max_abs = np.abs(fp32).max()
    assert np.all(np.abs(int8 - fp32) <= 1e-4 + 0.02 * np.abs(fp32) + 0.02 * max_abs)


def test_int8_avx2_matches_scalar_reference_test(orc):
    """matmul_quantized_b_avx2_matches_scalar (src/ops/matmul.rs:1879-1904): k = 123
    exercises the scalar k tail, n = 533 the tail columns."""
    m, k, n = 1, 123, 533
    a = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.083)).astype(np.float32).reshape(m, k)
    w = (np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.037)) * np.float32(1.3)).astype(np.float32).reshape(n, k)
    q, s = orc.pack_int8(w)
    scalar = orc.matmul_quantized_b(a, q, s, None, use_avx2=False)
    avx2 = orc.matmul_quantized_b(a, q, s, None, use_avx2=True)
    assert np.all(np.abs(avx2 - scalar) <= 1e-4 + 1e-4 * np.abs(scalar))
    assert np.abs(avx2 - f64_ref_q(a, q, s)).max() < 1e-3


def test_int8_catches_planted_mistakes(orc):
    """The f64 check fails for a dropped bias, a missing scale or a transposed weight."""
    rng = np.random.default_rng(13)
    n, k = 256, 120
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    q, s = orc.pack_int8(w)
    a = rng.standard_normal((5, k), dtype=np.float32)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    ref = f64_ref_q(a, q, s, bias)
    good = orc.matmul_quantized_b(a, q, s, bias)
    assert np.abs(good - ref).max() < 1e-4
    assert np.abs(orc.matmul_quantized_b(a, q, s, None) - ref).max() > 1e-3
    assert np.abs(orc.matmul_quantized_b(a, q, np.ones_like(s), bias) - ref).max() > 1e-3
    qt = np.ascontiguousarray(q[:, ::-1])
    assert np.abs(orc.matmul_quantized_b(a, qt, s, bias) - ref).max() > 1e-3


@pytest.mark.parametrize("threads", [1, 8])
def test_fp32_ragged_edges_reference_test(orc, threads):
    """blocked_kernel_matches_reference_on_ragged_edges (src/ops/matmul.rs:1634-1671)."""
    K = 8
    for n_tail in range(4):
        n = 24 + n_tail
        bt = np.cos(np.arange(n * K, dtype=np.float32) * np.float32(0.031)).astype(np.float32).reshape(n, K)
        for rows in range(1, 6):
            a = np.sin(np.arange(rows * K, dtype=np.float32) * np.float32(0.07)).astype(np.float32).reshape(rows, K)
            for bias in (None, np.full(n, 0.5, np.float32)):
                got = orc.matmul_transposed_b(a, bt, bias, partition_threads=threads)
                assert np.abs(got - f64_ref_t(a, bt, bias)).max() < 1e-4


def test_fp32_batched_and_both_paths_reference_test(orc):
    """batched_matmul_is_identical_on_both_paths (src/ops/matmul.rs:1597-1631)."""
    for shape in ([3, 1, 8], [2, 3, 8], [4, 1, 16]):
        batch, m, k = shape
        n = 1024
        bt = np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.03)).astype(np.float32).reshape(n, k)
        a = np.sin(np.arange(batch * m * k, dtype=np.float32) * np.float32(0.05)).astype(np.float32).reshape(-1, k)
        scalar = orc.matmul_transposed_b(a, bt, None, partition_threads=8, use_avx2=False)
        wide = orc.matmul_transposed_b(a, bt, None, partition_threads=8, use_avx2=True)
        assert np.all(np.abs(wide - scalar) <= 1e-4 + 1e-4 * np.abs(scalar))
        assert np.abs(scalar - f64_ref_t(a, bt)).max() < 1e-4


@pytest.mark.parametrize("k", [96, 97, 120, 123])
def test_fp32_avx2_matches_scalar(orc, k):
    """matmul_transposed_b_avx2_matches_scalar and _m1_large_n (src/ops/matmul.rs:1852-1930)."""
    m, n = 8, 533
    a = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.083)).astype(np.float32).reshape(m, k)
    w = (np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.037)) * np.float32(1.3)).astype(np.float32).reshape(n, k)
    for rows in (1, m):
        scalar = orc.matmul_transposed_b(a[:rows], w, None, partition_threads=8, use_avx2=False)
        avx2 = orc.matmul_transposed_b(a[:rows], w, None, partition_threads=8, use_avx2=True)
        assert np.all(np.abs(avx2 - scalar) <= 1e-4 + 1e-4 * np.abs(scalar))


def test_fp32_head_shape_matches_f64(orc):
    rng = np.random.default_rng(14)
    n, k, m = 18710, 120, 6
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    a = rng.standard_normal((m, k), dtype=np.float32)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    got = orc.matmul_transposed_b(a, w, bias, partition_threads=8)
    assert np.abs(got - f64_ref_t(a, w, bias)).max() < 1e-4
