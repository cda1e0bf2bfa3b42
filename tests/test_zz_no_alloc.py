"""The allocation-free entry point ppocr_rh_decode_dev_noalloc, through the C ABI, against
ppocr_rh_decode_dev (its own workspace) on the same inputs: two calls in a row, the
second with a smaller batch (the scratch array keeps the first call's contents), for the
MFMA and the fp32 FMA paths, bit for bit; a batch whose scratch would exceed the array is
refused before anything is launched."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(rh, L, head, a, off, mode, noalloc, stream=None):
    from ppocr_rechead.hip import DeviceArray, synchronize
    m, lines = a.shape[0], len(off) - 1
    da = DeviceArray.from_numpy(a)
    doff = DeviceArray.from_numpy(off)
    didx, dmp, dseq = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32), DeviceArray((m,), np.int32)
    dlen, dscore = DeviceArray((lines,), np.int64), DeviceArray((lines,), np.float32)
    if noalloc:
        rc = L.ppocr_rh_decode_dev_noalloc(head.handle, da.p, m, doff.p, lines, mode, didx.p, dmp.p, dseq.p, dlen.p,
                                           dscore.p, stream)
    else:
        rc = L.ppocr_rh_decode_dev(head.handle, da.p, m, doff.p, lines, mode, didx.p, dmp.p, dseq.p, dlen.p,
                                   dscore.p, None, 0, stream)
    rh._check(rc)
    synchronize()
    out = {"idx": didx.numpy(), "maxprob": dmp.numpy(), "seq": dseq.numpy(), "seq_len": dlen.numpy(),
           "score": dscore.numpy()}
    for d in (da, doff, didx, dmp, dseq, dlen, dscore):
        d.free()
    return out


@pytest.mark.parametrize("mode", [2, 0])
def test_noalloc_matches_decode_dev_two_calls(orc, rh, mode):
    from ppocr_rechead import workloads as wl
    L = rh._lib.lib()
    w_t, bias = wl.weights()
    q, s = orc.pack_int8(w_t)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    rng = np.random.default_rng(41)
    # first a larger ragged batch (some rows x30: the precision guard's list is used),
    # then a smaller one that finds the first call's contents in the scratch array
    for call, lens in enumerate(([120] * 40 + [77, 5, 1], [37, 120])):
        off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        m = int(off[-1])
        a = rng.standard_normal((m, 120)).astype(np.float32)
        a[rng.choice(m, max(1, m // 25), replace=False)] *= np.float32(30.0)
        print(f"noalloc call {call} mode={mode} m={m} lines={len(lens)}", flush=True)
        got = _run(rh, L, head, a, off, mode, noalloc=True)
        ref = _run(rh, L, head, a, off, mode, noalloc=False)
        for key in ("idx", "seq_len"):
            assert np.array_equal(got[key], ref[key]), (call, key)
        for key in ("maxprob", "score"):
            assert np.array_equal(got[key].view(np.uint32), ref[key].view(np.uint32)), (call, key)
        for b in range(len(lens)):
            n = int(ref["seq_len"][b])
            assert np.array_equal(got["seq"][off[b]:off[b] + n], ref["seq"][off[b]:off[b] + n]), (call, b)
        # and the oracle, within the parity bars
        r = orc.rechead_lines(a, off, q, s, bias)
        assert np.abs(got["maxprob"] - r["maxprob"]).max() < 1e-4
    head.close()


def test_noalloc_refuses_a_batch_beyond_its_scratch(rh):
    """A batch whose scratch (the workspace ppocr_rh_decode_dev would take) exceeds the
    32 MiB array is refused with an argument error before any launch.  The buffers are
    real and of the full size, so nothing could read out of bounds even if a launch
    happened."""
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray
    L = rh._lib.lib()
    w_t, bias = wl.weights()
    head = rh.RecHead(qw=rh.QuantizedWeight.from_f32_transposed(w_t), bias=bias)
    m = 600000
    while head.workspace_bytes(m, 2) <= (32 << 20):
        m *= 2
    ws = head.workspace_bytes(m, 2)
    print(f"noalloc refusal m={m} (workspace {ws} bytes)", flush=True)
    da = DeviceArray((m, 120), np.float32)
    doff = DeviceArray.from_numpy(np.array([0, m], np.int64))
    didx, dmp, dseq = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32), DeviceArray((m,), np.int32)
    dlen, dscore = DeviceArray((1,), np.int64), DeviceArray((1,), np.float32)
    rc = L.ppocr_rh_decode_dev_noalloc(head.handle, da.p, m, doff.p, 1, 2, didx.p, dmp.p, dseq.p, dlen.p, dscore.p,
                                       None)
    assert rc == rh._lib.PPOCR_ERR_INVALID_ARG
    assert b"allocation-free" in L.ppocr_last_error()
    for d in (da, doff, didx, dmp, dseq, dlen, dscore):
        d.free()
    head.close()
