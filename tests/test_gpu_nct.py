"""The whole head entered at the neck's Transpose.8 (ppocr_rh_decode_nct[_dev],
src/engine/model.rs:1325-1342): x [lines][k][T], channels first, the transpose folded into
the activation loads.  Its results must equal, bit for bit, those of ppocr_rh_decode on
the transposed activations (same rows, same arithmetic) for the INT8 head in every mode
(fp32 FMA; bf16x2 with its precision guard and rescue, one and two blocks per wave;
bf16x3), the tiny head (k=80) and an FP32 head; and agree with the oracle (argmax except
at top-2 gaps below 1e-4, max probabilities and scores within 1e-4)."""
import numpy as np
import pytest

from gpu_common import assert_close_rel, check_argmax, f64_logits_q, rel_scale, top2_gap
from test_gpu_random_shapes import _head

pytestmark = pytest.mark.gpu

TOL = 1e-4
CASES = [
    # (seed, k, n, lines, T, mode, fp32 head)
    (1, 120, 18710, 1, 120, 2, False),   # one line
    (2, 120, 18710, 80, 120, 2, False),  # 9600 rows: two 32-row blocks per wave
    (3, 120, 3000, 5, 240, 3, False),
    (4, 120, 3000, 7, 33, 0, False),     # fp32 FMA path
    (5, 80, 6906, 29, 40, 2, False),     # tiny head
    (6, 117, 500, 3, 1, 2, False),       # one step per line
    (7, 120, 2049, 4, 97, 3, True),      # FP32 head, bf16x3
    (8, 119, 2049, 4, 50, 0, True),      # FP32 head, fp32 FMA
    (9, 120, 18710, 80, 120, 4, False),  # fp16 terms, two blocks per wave
    (10, 80, 6906, 6, 33, 4, False),     # fp16 terms, tiny head
    (11, 120, 2049, 4, 97, 4, True),     # FP32 head, fp16 halves
]


def _inputs(orc, seed, k, n, lines, T, fp32):
    rng = np.random.default_rng(seed)
    if fp32:
        w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
        q = s = None
    else:
        q, s, bias = _head(orc, rng, n, k)
        w = None
    x = rng.standard_normal((lines, k, T)).astype(np.float32)
    m = lines * T
    for r in rng.choice(m, max(1, m // 20), replace=False):  # guarded rows
        x[r // T, :, r % T] *= np.float32(30.0)
    return q, s, w, bias, x


@pytest.mark.parametrize("seed,k,n,lines,T,mode,fp32", CASES)
def test_nct_equals_transposed_rows(orc, rh, seed, k, n, lines, T, mode, fp32):
    q, s, w, bias, x = _inputs(orc, seed, k, n, lines, T, fp32)
    print(f"nct seed={seed} k={k} n={n} lines={lines} T={T} mode={mode} fp32={fp32}", flush=True)
    head = rh.RecHead(w_t=w, bias=bias) if fp32 else rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    got = head.decode_nct(x, mode)
    a = np.ascontiguousarray(x.transpose(0, 2, 1).reshape(-1, k))
    off = np.arange(lines + 1, dtype=np.int64) * T
    rows = head.decode(a, off, mode)
    head.close()
    assert np.array_equal(got["idx"], rows["idx"])
    assert np.array_equal(got["maxprob"].view(np.uint32), rows["maxprob"].view(np.uint32))
    assert np.array_equal(got["score"].view(np.uint32), rows["score"].view(np.uint32))
    assert all(np.array_equal(u, v) for u, v in zip(got["seqs"], rows["seqs"]))
    if fp32:
        return
    ref = orc.rechead_lines(a, off, q, s, bias)
    lg = f64_logits_q(a, q, s, bias)
    exempt = check_argmax(got["idx"], ref["idx"], top2_gap(lg), label=f"nct seed {seed}")
    assert_close_rel(got["maxprob"], ref["maxprob"], f"nct seed {seed} maxprob", row_scale=rel_scale(lg))
    for b in range(lines):
        if np.any((exempt >= off[b]) & (exempt < off[b + 1])):
            continue
        assert np.array_equal(got["seqs"][b], ref["seqs"][b]), (seed, b)
        assert abs(float(got["score"][b]) - float(ref["score"][b])) < TOL, (seed, b)


def test_nct_dev_with_workspace_and_errors(orc, rh):
    """The device entry on a caller stream and workspace gives the host entry's results;
    shape and argument errors are reported, zero lines is a no-op."""
    import ctypes
    from ppocr_rechead.hip import DeviceArray, Stream, synchronize
    L = rh._lib.lib()
    lines, k, T, n = 6, 120, 64, 4000
    q, s, _, bias, x = _inputs(orc, 21, k, n, lines, T, False)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    host = head.decode_nct(x, 2)
    m = lines * T
    dx = DeviceArray.from_numpy(x)
    di, dp, dseq = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32), DeviceArray((m,), np.int32)
    dlen, dsc = DeviceArray((lines,), np.int64), DeviceArray((lines,), np.float32)
    ws = head.workspace_bytes(m, 2)
    dws = DeviceArray((ws,), np.uint8)
    st = Stream()
    print("nct dev", flush=True)
    rh._check(L.ppocr_rh_decode_nct_dev(head.handle, dx.p, lines, T, 2, di.p, dp.p, dseq.p, dlen.p, dsc.p, dws.p,
                                        ws, st.h))
    synchronize()
    assert np.array_equal(di.numpy(), host["idx"])
    assert np.array_equal(dp.numpy().view(np.uint32), host["maxprob"].view(np.uint32))
    seq, ln = dseq.numpy(), dlen.numpy()
    assert all(np.array_equal(seq[b * T:b * T + ln[b]], host["seqs"][b]) for b in range(lines))
    assert np.array_equal(dsc.numpy().view(np.uint32), host["score"].view(np.uint32))
    # errors: negative sizes, too small a workspace, a wrong shape in the mirror
    assert L.ppocr_rh_decode_nct_dev(head.handle, dx.p, -1, T, 2, None, None, dseq.p, dlen.p, dsc.p, None, 0,
                                     None) == rh.PPOCR_ERR_INVALID_ARG
    assert L.ppocr_rh_decode_nct(head.handle, None, 1, -3, 2, None, None, None, None, None) == rh.PPOCR_ERR_INVALID_ARG
    assert L.ppocr_rh_decode_nct_dev(head.handle, dx.p, lines, T, 2, None, None, dseq.p, dlen.p, dsc.p, dws.p,
                                     ctypes.c_size_t(16), None) == rh.PPOCR_ERR_INVALID_ARG
    with pytest.raises(rh.OcrError):
        head.decode_nct(x.transpose(0, 2, 1), 2)
    assert L.ppocr_rh_decode_nct(head.handle, None, 0, T, 2, None, None, None, None, None) == rh.PPOCR_OK
    empty = head.decode_nct(np.zeros((3, k, 0), np.float32), 2)  # lines without steps
    assert [len(x) for x in empty["seqs"]] == [0, 0, 0] and not np.any(empty["score"])
    head.close()
