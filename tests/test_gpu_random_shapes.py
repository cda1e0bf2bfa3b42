"""Seeded sweep of head shapes and ragged batches through the whole head
(ppocr_rh_decode) against the oracle: k in the two supported ranges (73..80, 113..120,
aligned and not), n from 1 class to the tiny head's 6906, lines of 1..130 steps, with
zero-weight classes and outlier weights.  Indices and sequences must agree except at
top-2 gaps below 1e-4 (lines holding such a row are excused from the sequence check);
max probabilities and scores within 1e-4.  Also: an activation pointer that is not
16-byte aligned gives bit-identical results to an aligned copy."""
import ctypes

import numpy as np
import pytest

from gpu_common import assert_close_rel, check_argmax, f64_logits_q, rel_scale, top2_gap

pytestmark = pytest.mark.gpu

TOL = 1e-4
CASES = [
    # (seed, k, n, line lengths, mode)
    (1, 120, 1, [5, 1, 33], 2),
    (2, 120, 31, [120], 2),
    (3, 113, 33, [7, 130, 64], 2),
    (4, 116, 500, [1, 2, 3, 4, 5, 6, 7, 8], 3),
    (5, 80, 6906, [40, 97, 12], 2),
    (6, 73, 2049, [130, 1, 129], 3),
    (7, 77, 32, [64, 64], 2),
    (8, 119, 2049, [25] * 12, 2),
    (9, 120, 18710, [3, 120, 77], 2),
    (10, 80, 64, [0, 10, 0, 5], 2),
    (11, 120, 18710, [120, 37, 1], 4),
    (12, 80, 6906, [40, 97, 12], 4),
    (13, 115, 500, [1, 2, 3, 4, 5, 6, 7, 8], 4),
]


def _head(orc, rng, n, k):
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    if n > 4:
        w[rng.choice(n, max(1, n // 50), replace=False)] = 0.0          # scale 1.0 rows
        w[rng.choice(n, max(1, n // 50), replace=False), rng.integers(0, k)] = 5.0  # outliers
    q, s = orc.pack_int8(w)
    bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
    return q, s, bias


@pytest.mark.parametrize("seed,k,n,lens,mode", CASES)
def test_decode_random_shapes(orc, rh, seed, k, n, lens, mode):
    rng = np.random.default_rng(seed)
    q, s, bias = _head(orc, rng, n, k)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    m = int(off[-1])
    a = rng.standard_normal((m, k)).astype(np.float32)
    if m > 3:
        a[rng.choice(m, max(1, m // 20), replace=False)] *= np.float32(30.0)  # guarded rows
    print(f"random shapes seed={seed} k={k} n={n} lines={len(lens)} m={m} mode={mode}", flush=True)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    got = head.decode(a, off, mode)
    head.close()
    ref = orc.rechead_lines(a, off, q, s, bias)
    if m == 0:
        return
    lg = f64_logits_q(a, q, s, bias)
    gap = top2_gap(lg) if n > 1 else np.full(m, np.inf)
    exempt = check_argmax(got["idx"], ref["idx"], gap, label=f"seed {seed}")
    assert_close_rel(got["maxprob"], ref["maxprob"], f"seed {seed} maxprob", row_scale=rel_scale(lg))
    for b in range(len(lens)):
        if np.any((exempt >= off[b]) & (exempt < off[b + 1])):
            continue  # a near-tie row may change this line's collapse
        assert np.array_equal(got["seqs"][b], ref["seqs"][b]), (seed, b)
        assert abs(float(got["score"][b]) - float(ref["score"][b])) < TOL, (seed, b)


def test_unaligned_activation_pointer(orc, rh):
    """Rows that start 4 bytes past a 16-byte boundary take the scalar-load path; the
    results equal those of the aligned copy bit for bit."""
    from ppocr_rechead.hip import DeviceArray, synchronize
    L = rh._lib.lib()
    rng = np.random.default_rng(11)
    q, s, bias = _head(orc, rng, 3000, 120)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    m = 300
    a = rng.standard_normal((m, 120)).astype(np.float32)
    buf = np.zeros(m * 120 + 1, np.float32)
    buf[1:] = a.reshape(-1)
    d_al, d_un = DeviceArray.from_numpy(a), DeviceArray.from_numpy(buf)
    un_ptr = ctypes.c_void_p(d_un.p.value + 4)
    outs = []
    for ptr in (d_al.p, un_ptr):
        di, dp = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
        dl = DeviceArray((m, 3000), np.float32)
        print("unaligned activations", flush=True)
        rh._check(L.ppocr_rh_argmax_dev(head.handle, ptr, m, 2, di.p, dp.p, None, 0, None))
        rh._check(L.ppocr_rh_logits_dev(head.handle, ptr, m, 2, dl.p, None, 0, None))
        synchronize()
        outs.append((di.numpy(), dp.numpy().view(np.uint32), dl.numpy().view(np.uint32)))
    for x, y in zip(*outs):
        assert np.array_equal(x, y)
    head.close()


@pytest.mark.parametrize("seed,k,n,lens,mode", [c for c in CASES if c[2] <= 6906])
def test_logits_and_probs_random_shapes(orc, rh, seed, k, n, lens, mode):
    """The same sweep through the unfused projection (logits) and the fused probabilities,
    against the oracle's matmul_quantized_b and softmax, max-abs 1e-4."""
    rng = np.random.default_rng(seed + 100)
    q, s, bias = _head(orc, rng, n, k)
    m = max(1, min(int(sum(lens)), 300))
    a = rng.standard_normal((m, k)).astype(np.float32)
    a[rng.choice(m, max(1, m // 20), replace=False)] *= np.float32(30.0)
    print(f"logits/probs seed={seed} k={k} n={n} m={m} mode={mode}", flush=True)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    logits = head.logits(a, mode)
    probs = head.probs(a, mode)
    head.close()
    ref = orc.matmul_quantized_b(a, q, s, bias)
    tol = 1e-4 + 1e-5 * np.abs(ref)  # f32 rounding of the x30 rows' large logits
    assert np.all(np.abs(logits - ref) <= tol)
    assert_close_rel(probs, orc.softmax_rows(ref), f"seed {seed} probs", row_scale=rel_scale(f64_logits_q(a, q, s, bias)))


@pytest.mark.parametrize("k,n,mode", [(120, 500, 0), (120, 500, 3), (80, 6906, 3), (77, 33, 0), (119, 2049, 3),
                                      (120, 500, 4), (80, 6906, 4), (117, 2049, 4)])
def test_fp32_head_random_shapes(orc, rh, k, n, mode):
    """FP32 heads (W^T in fp32, matmul_transposed_b): logits, probabilities and the whole
    head against the oracle, for the fp32 FMA and the three-term MFMA modes."""
    rng = np.random.default_rng(k * 31 + n)
    w_t = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
    lens = [37, 120, 5]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    a = rng.standard_normal((int(off[-1]), k)).astype(np.float32)
    print(f"fp32 head k={k} n={n} mode={mode}", flush=True)
    head = rh.RecHead(w_t=w_t, bias=bias)
    logits = head.logits(a, mode)
    probs = head.probs(a, mode)
    got = head.decode(a, off, mode)
    head.close()
    ref = orc.matmul_transposed_b(a, w_t, bias)
    assert np.abs(logits - ref).max() < TOL
    refp = orc.softmax_rows(ref)
    assert_close_rel(probs, refp, f"fp32 head k={k} n={n} probs")
    ref64 = a.astype(np.float64) @ w_t.astype(np.float64).T + bias
    gap = top2_gap(ref64)
    check_argmax(got["idx"], np.argmax(ref64, axis=1).astype(np.int32), gap, label=f"fp32 head k={k}")
    assert_close_rel(got["maxprob"], refp.max(axis=1), f"fp32 head k={k} n={n} maxprob")


@pytest.mark.parametrize("n,mode", [(120, 3), (240, 3), (360, 3), (360, 0)])
def test_neck_matmuls_with_k_120(orc, rh, n, mode):
    """The rec neck's MatMul nodes with K = 120 (weights [120, 120 | 240 | 360], bias
    folded) run as FP32 heads through the same entry points (ppocr_rh_create_f32 +
    ppocr_rh_logits): against the oracle's matmul_transposed_b, max-abs 1e-4, for a
    neck-like activation batch (3 lines x T=120, N(0,1)) and weights N(0, 0.1^2)."""
    rng = np.random.default_rng(n + mode)
    w_t = (rng.standard_normal((n, 120)) * 0.1).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.02).astype(np.float32)
    a = rng.standard_normal((360, 120)).astype(np.float32)
    print(f"neck matmul n={n} mode={mode}", flush=True)
    head = rh.RecHead(w_t=w_t, bias=bias)
    got = head.logits(a, mode)
    head.close()
    ref = orc.matmul_transposed_b(a, w_t, bias)
    assert got.shape == (360, n)
    assert np.abs(got - ref).max() < TOL
