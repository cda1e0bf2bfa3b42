"""GPU parity: every HIP entry point against the CPU oracle on the same seeded inputs.

Bars: packed q and scales bit-exact; logits and probabilities within max-abs 1e-4
(BF16X2, BF16X3, FP32_FMA); argmax and CTC sequences identical except at top-2 logit gaps
below 1e-4, which are printed; CTC collapse bit-exact on identical per-step inputs."""
import os

import numpy as np
import pytest

from gpu_common import assert_close_rel, check_argmax, f64_logits_q, rel_scale, split_lines, top2_gap

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def head(orc):
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    q, s = orc.pack_int8(w_t)
    return {"w_t": w_t, "bias": bias, "q": q, "s": s}


@pytest.fixture(scope="module")
def rhead(rh, head):
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=head["bias"])
    yield h
    h.close()


def test_pack_bit_exact_synthetic_and_stress(orc, rh):
    from ppocr_rechead import workloads as wl
    for stress in (False, True):
        w_t, _ = wl.weights(stress=stress)
        print(f"pack 18710x120 stress={stress}", flush=True)
        qw = rh.QuantizedWeight.from_f32_transposed(w_t)
        q, s = orc.pack_int8(w_t)
        assert np.array_equal(qw.data, q)
        assert np.array_equal(qw.scales.view(np.uint32), s.view(np.uint32))


def test_pack_bit_exact_golden_rows(rh):
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "pack_rows.npz"))
    for key in ("small_rec", "tiny_rec", "special"):
        print(f"pack golden {key}", flush=True)
        qw = rh.QuantizedWeight.from_f32_transposed(g[f"{key}_w_t"])
        assert np.array_equal(qw.data, g[f"{key}_q"]), key
        assert np.array_equal(qw.scales.view(np.uint32), g[f"{key}_scales"].view(np.uint32)), key


def test_pack_edge_shapes(orc, rh):
    rng = np.random.default_rng(5)
    for n, k in ((1, 1), (3, 7), (5, 64), (2, 65), (7, 300)):
        w = rng.standard_normal((n, k), dtype=np.float32)
        w[0, 0] = np.nan
        print(f"pack n={n} k={k}", flush=True)
        qw = rh.QuantizedWeight.from_f32_transposed(w)
        q, s = orc.pack_int8(w)
        assert np.array_equal(qw.data, q) and np.array_equal(qw.scales.view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("m", [1, 33, 120, 257])
def test_int8_logits(orc, rh, head, rhead, mode, m):
    rng = np.random.default_rng(100 + m)
    a = rng.standard_normal((m, 120), dtype=np.float32)
    print(f"int8 logits mode={mode} m={m}", flush=True)
    got = rhead.logits(a, mode)
    ref = orc.matmul_quantized_b(a, head["q"], head["s"], head["bias"], partition_threads=1)
    err = np.abs(got - ref).max()
    print(f"  max|gpu-oracle| = {err:.3e}")
    assert got.shape == (m, 18710)
    if mode == 1:
        assert err < 2e-2  # a single bf16 term keeps ~8 bits of the activation
    else:
        assert err < TOL


def test_int8_logits_no_bias_small_n(orc, rh):
    rng = np.random.default_rng(7)
    for n, k in ((100, 120), (1000, 120), (33, 117), (64, 80), (6906, 80)):
        w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
        q, s = orc.pack_int8(w)
        a = rng.standard_normal((70, k), dtype=np.float32)
        head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=None)
        for mode in (0, 2, 3, 4):
            print(f"int8 logits n={n} k={k} mode={mode} no bias", flush=True)
            got = head.logits(a, mode)
            ref = orc.matmul_quantized_b(a, q, s, None)
            assert np.abs(got - ref).max() < TOL, (n, k, mode)
        head.close()


def test_tiny_head_real_rows(orc, rh):
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "pack_rows.npz"))
    q, s = g["tiny_rec_q"], g["tiny_rec_scales"]
    rng = np.random.default_rng(8)
    a = rng.standard_normal((50, 80), dtype=np.float32)
    bias = (rng.standard_normal(q.shape[0], dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    for mode in (0, 2, 3, 4):
        print(f"tiny real rows mode={mode}", flush=True)
        got = head.logits(a, mode)
        assert np.abs(got - orc.matmul_quantized_b(a, q, s, bias)).max() < TOL
    head.close()


@pytest.mark.parametrize("mode", [0, 2, 3, 4])
def test_small_head_real_rows_decode(orc, rh, mode):
    """The whole head on 512 classes of the small model's real weights (its first 256
    classes, blank included, 128 from the middle and the last 128; golden fixture): ragged
    lines of seeded activations, some rows x30 (guarded), against the oracle."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "pack_rows.npz"))
    q, s = g["small_rec_q"], g["small_rec_scales"]
    rng = np.random.default_rng(17)
    bias = (rng.standard_normal(q.shape[0], dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    lens = [120, 37, 1, 80]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    a = rng.standard_normal((int(off[-1]), 120), dtype=np.float32)
    a[rng.choice(a.shape[0], 12, replace=False)] *= np.float32(30.0)
    print(f"small real rows decode mode={mode}", flush=True)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    got = head.decode(a, off, mode)
    head.close()
    ref = orc.rechead_lines(a, off, q, s, bias)
    lg = f64_logits_q(a, q, s, bias)
    exempt = check_argmax(got["idx"], ref["idx"], top2_gap(lg), label=f"real rows mode {mode}")
    assert_close_rel(got["maxprob"], ref["maxprob"], f"real rows maxprob mode {mode}", row_scale=rel_scale(lg))
    for b in range(len(lens)):
        if np.any((exempt >= off[b]) & (exempt < off[b + 1])):
            continue
        assert np.array_equal(got["seqs"][b], ref["seqs"][b]), (mode, b)
        assert abs(float(got["score"][b]) - float(ref["score"][b])) < TOL, (mode, b)


@pytest.mark.parametrize("mode", [0, 1, 3, 4])
def test_fp32_head_logits(orc, rh, mode):
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    rng = np.random.default_rng(9)
    a = rng.standard_normal((300, 120), dtype=np.float32)
    head = rh.RecHead(w_t=w_t, bias=bias)
    print(f"fp32 head mode={mode}", flush=True)
    got = head.logits(a, mode)
    ref = orc.matmul_transposed_b(a, w_t, bias, partition_threads=1)
    err = np.abs(got - ref).max()
    print(f"  max|gpu-oracle| = {err:.3e}")
    assert err < (2e-2 if mode == 1 else TOL)
    head.close()


def test_fp32_head_rejects_bf16x2(rh):
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights(n=64)
    head = rh.RecHead(w_t=w_t, bias=bias)
    with pytest.raises(rh.OcrError):
        head.logits(np.zeros((2, 120), np.float32), 2)
    head.close()


def test_softmax_matches_oracle(orc, rh):
    rng = np.random.default_rng(10)
    for rows, cols in ((5, 18710), (3, 40), (2, 2049), (2, 30000), (1, 1), (4, 7)):
        x = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
        print(f"softmax {rows}x{cols}", flush=True)
        got = x.copy()
        rh.softmax_inplace(got)
        ref = orc.softmax_rows(x)
        assert np.abs(got - ref).max() < 1e-6
    big = np.array([[1000, 1001, 999, 1000.5], [-1000, -999, -1001, -1000.5]], np.float32)
    rh.softmax_inplace(big)
    assert np.all(np.isfinite(big)) and np.all(np.abs(big.sum(axis=1) - 1) < 1e-5)
    empty = np.zeros((3, 0), np.float32)
    rh.softmax_inplace(empty)


def test_softmax_dev_emits_argmax_of_probs(orc, rh, head):
    from ppocr_rechead.hip import DeviceArray, synchronize
    rng = np.random.default_rng(11)
    a = rng.standard_normal((64, 120), dtype=np.float32)
    logits = orc.matmul_quantized_b(a, head["q"], head["s"], head["bias"])
    d = DeviceArray.from_numpy(logits)
    di = DeviceArray((64,), np.int32)
    dp = DeviceArray((64,), np.float32)
    L = rh._lib.lib()
    print("softmax_dev + argmax", flush=True)
    assert L.ppocr_softmax_rows_dev(d.p, 64, 18710, di.p, dp.p, None) == 0
    synchronize()
    probs = orc.softmax_rows(logits)
    idx, val = orc.argmax_rows(probs)
    gap = top2_gap(f64_logits_q(a, head["q"], head["s"], head["bias"]))
    check_argmax(di.numpy(), idx, gap, label="softmax argmax")
    assert np.abs(dp.numpy() - val).max() < 1e-6
    assert np.abs(d.numpy() - probs).max() < 1e-6


def test_argmax_rows_first_occurrence(orc, rh):
    rng = np.random.default_rng(12)
    x = rng.integers(0, 40, (300, 1000)).astype(np.float32)
    x[5] = np.nan
    x[6, :] = np.nan
    x[6, 500] = 3.0
    print("argmax rows", flush=True)
    idx = np.empty(300, np.int32)
    val = np.empty(300, np.float32)
    rh._check(rh._lib.lib().ppocr_argmax_rows(rh._ptr(x), 300, 1000, rh._ptr(idx), rh._ptr(val)))
    ridx, rval = orc.argmax_rows(x)
    assert np.array_equal(idx, ridx)
    assert np.array_equal(val, rval)
    assert idx[5] == 0 and val[5] == -np.inf and idx[6] == 500


def test_ctc_collapse_matches_oracle(orc, rh):
    rng = np.random.default_rng(13)
    lengths = [0, 1, 2, 63, 64, 65, 127, 128, 129, 240, 0, 17, 500]
    off = np.zeros(len(lengths) + 1, np.int64)
    off[1:] = np.cumsum(lengths)
    steps = int(off[-1])
    idx = rng.integers(0, 4, steps).astype(np.int32)  # many blanks and repeats
    mask = rng.random(steps) < 0.3
    idx[mask] = rng.integers(0, 18710, int(mask.sum())).astype(np.int32)
    val = rng.random(steps).astype(np.float32)
    print("ctc collapse", flush=True)
    seqs, score = rh.CtcDecoder.collapse(idx, val, off)
    rseqs, rscore = orc.ctc_collapse(idx, val, off)
    assert all(np.array_equal(x, y) for x, y in zip(seqs, rseqs))
    assert np.array_equal(score.view(np.uint32), rscore.view(np.uint32))
    # the reference's known answers
    dec = rh.CtcDecoder.from_vocab(["blank", "a", "b", " "])
    t = np.zeros((1, 4, 4), np.float32)
    for tt, c in ((0, 1), (1, 1), (2, 0), (3, 2)):
        t[0, tt, c] = 1.0
    text, sc = dec.decode(t)
    assert text == "ab" and abs(sc - 1.0) < 1e-6
    d = np.zeros((2, 2, 4), np.float32)
    d[0, 0, 1] = d[0, 1, 2] = d[1, 0, 2] = d[1, 1, 0] = 1.0
    assert [x[0] for x in dec.decode_batch(d)] == ["ab", "b"]


def test_ctc_greedy_dev_clamps_device_offsets(orc, rh):
    """ppocr_ctc_greedy_dev reads the line offsets on the device and clamps them into
    [0, line_off[lines]]: a negative start, a line running backwards and one past the end
    give the results of the clamped lines, and nothing is written past the arrays (their
    tails hold sentinels)."""
    from ppocr_rechead.hip import DeviceArray, synchronize
    rng = np.random.default_rng(19)
    total = 300
    off = np.array([-7, 100, 60, 60, 250, 1000, total], np.int64)
    lines = off.size - 1
    idx = rng.integers(0, 5, total).astype(np.int32)
    idx[0:100:2] = 0  # line 0 emits at most 50 indices, so its output stays clear of line 3's at 60
    val = rng.random(total).astype(np.float32)
    pad = 256
    d_idx = DeviceArray.from_numpy(np.concatenate([idx, np.full(pad, 3, np.int32)]))
    d_val = DeviceArray.from_numpy(np.concatenate([val, np.full(pad, 0.5, np.float32)]))
    d_off = DeviceArray.from_numpy(off)
    d_seq = DeviceArray.from_numpy(np.full(total + pad, -123, np.int32))
    d_len = DeviceArray.from_numpy(np.full(lines + 8, -5, np.int64))
    d_score = DeviceArray.from_numpy(np.full(lines + 8, -7.0, np.float32))
    print("ctc_greedy_dev with out-of-range offsets", flush=True)
    rh._check(rh._lib.lib().ppocr_ctc_greedy_dev(d_idx.p, d_val.p, d_off.p, lines, 0, d_seq.p, d_len.p, d_score.p,
                                                 None))
    synchronize()
    seq, seq_len, score = d_seq.numpy(), d_len.numpy(), d_score.numpy()
    assert np.all(seq[total:] == -123) and np.all(seq_len[lines:] == -5) and np.all(score[lines:] == -7.0)
    t0 = np.minimum(np.maximum(off[:-1], 0), total)
    t1 = np.minimum(np.maximum(off[1:], t0), total)
    clamped = np.stack([t0, t1], axis=1)
    for b, (a0, a1) in enumerate(clamped):
        rs, rsc = orc.ctc_collapse(idx[a0:a1], val[a0:a1], np.array([0, a1 - a0], np.int64))
        assert seq_len[b] == rs[0].size, b
        assert score[b].view(np.uint32) == rsc[0].view(np.uint32), b
    # line 0 ([0, 100)) overlaps no other line's output region
    assert np.array_equal(seq[:seq_len[0]], orc.ctc_collapse(idx[:100], val[:100], np.array([0, 100]))[0][0])


@pytest.mark.parametrize("mode", [0, 2, 3, 4])
def test_fused_argmax_a4_page(orc, rh, head, rhead, mode):
    from ppocr_rechead import workloads as wl
    a = wl.activations("a4_page")
    print(f"fused argmax a4_page mode={mode} m={a.shape[0]}", flush=True)
    idx, mp = rhead.argmax(a, mode)
    ref = orc.rechead_lines(a, wl.line_offsets(wl.lines_for("a4_page")), head["q"], head["s"], head["bias"])
    gap = top2_gap(f64_logits_q(a, head["q"], head["s"], head["bias"]))
    check_argmax(idx, ref["idx"], gap, label=f"a4_page mode {mode}")
    assert_close_rel(mp, ref["maxprob"], f"a4_page maxprob mode {mode}")


@pytest.mark.parametrize("mode", [0, 2, 3, 4])
def test_fused_probs_single_line(orc, rh, head, rhead, mode):
    from ppocr_rechead import workloads as wl
    a = wl.activations("single_line")
    print(f"fused probs single_line mode={mode}", flush=True)
    got = rhead.probs(a, mode)
    ref = orc.rechead_lines(a, np.array([0, 120], np.int64), head["q"], head["s"], head["bias"], want_probs=True)
    assert_close_rel(got, ref["probs"], f"single_line probs mode {mode}")


def test_decode_a4_page_end_to_end(orc, rh, head, rhead):
    from ppocr_rechead import workloads as wl
    a = wl.activations("a4_page")
    off = wl.line_offsets(wl.lines_for("a4_page"))
    print("decode a4_page", flush=True)
    got = rhead.decode(a, off)
    ref = orc.rechead_lines(a, off, head["q"], head["s"], head["bias"])
    gap = top2_gap(f64_logits_q(a, head["q"], head["s"], head["bias"]))
    exempt = set(check_argmax(got["idx"], ref["idx"], gap, label="decode a4_page").tolist())
    for b in range(len(off) - 1):
        if not any(off[b] <= r < off[b + 1] for r in exempt):
            assert np.array_equal(got["seqs"][b], ref["seqs"][b]), b
            assert abs(got["score"][b] - ref["score"][b]) < TOL


def test_decode_dev_matches_unfused_path(orc, rh, head, rhead):
    """MatMul.12 -> softmax_inplace -> argmax (three launches, logits through HBM) and the
    fused head agree on the dense 256-line batch (m = 30720), row by row."""
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray, synchronize
    a = wl.activations("dense_256")
    m = a.shape[0]
    L = rh._lib.lib()
    da = DeviceArray.from_numpy(a)
    dl = DeviceArray((m, 18710), np.float32)
    di1, dp1 = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
    di2, dp2 = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
    print("dense_256 unfused vs fused", flush=True)
    rh._check(L.ppocr_rh_logits_dev(rhead.handle, da.p, m, 2, dl.p, None, 0, None))
    rh._check(L.ppocr_softmax_rows_dev(dl.p, m, 18710, di1.p, dp1.p, None))
    rh._check(L.ppocr_rh_argmax_dev(rhead.handle, da.p, m, 2, di2.p, dp2.p, None, 0, None))
    synchronize()
    i1, p1, i2, p2 = di1.numpy(), dp1.numpy(), di2.numpy(), dp2.numpy()
    sample = np.random.default_rng(14).choice(m, 1024, replace=False)
    gap_s = top2_gap(f64_logits_q(a[sample], head["q"], head["s"], head["bias"]))
    diff = np.nonzero(i1 != i2)[0]
    print(f"  fused/unfused argmax differences: {diff.size}; max|maxprob diff| {np.abs(p1 - p2).max():.3e}")
    assert diff.size <= 5
    assert np.abs(p1 - p2).max() < 1e-5
    ref = orc.rechead_lines(a[sample], split_lines(sample.size), head["q"], head["s"], head["bias"])
    check_argmax(i2[sample], ref["idx"], gap_s, label="dense_256 fused sample")
    check_argmax(i1[sample], ref["idx"], gap_s, label="dense_256 unfused sample")
    assert_close_rel(p2[sample], ref["maxprob"], "dense_256 fused maxprob sample")
    probs_rows = dl.numpy()[sample[:64]]
    ref_p = orc.rechead_lines(a[sample[:64]], np.array([0, 64], np.int64), head["q"], head["s"], head["bias"],
                              want_probs=True)["probs"]
    assert_close_rel(probs_rows, ref_p, "dense_256 unfused probs")


def test_large_batch_logits_and_probs_single_pass(orc, rh, head, rhead):
    """m = 16461 rows: enough row blocks for the writers to walk each row's vocabulary in
    one pass, with a partial last row block; logits and probabilities of sampled rows
    (including the last 77) against the oracle."""
    rng = np.random.default_rng(21)
    m = 16384 + 77
    a = rng.standard_normal((m, 120), dtype=np.float32)
    sample = np.unique(np.concatenate([rng.choice(m - 77, 183, replace=False), np.arange(m - 77, m)]))
    print(f"large-batch logits m={m}", flush=True)
    got = rhead.logits(a, 2)
    ref = orc.matmul_quantized_b(a[sample], head["q"], head["s"], head["bias"])
    err = np.abs(got[sample] - ref).max()
    print(f"  max|logits gpu-oracle| = {err:.3e}")
    assert err < TOL
    del got
    print(f"large-batch probs m={m}", flush=True)
    gotp = rhead.probs(a, 2)
    refp = orc.rechead_lines(a[sample], split_lines(sample.size), head["q"], head["s"], head["bias"],
                             want_probs=True)["probs"]
    assert_close_rel(gotp[sample], refp, "large-batch probs")


@pytest.mark.parametrize("mode", [None, 2], ids=["auto", "bf16x2"])
def test_stress_1024_fused(orc, rh, mode):
    """m = 245760, zero-weight rows, +-5 outliers, 1% rows x50, 2% near-tie rows.  In
    BF16X2 the +-5 outliers put the precision limit near max|a| = 1.6, so the guard sends
    nearly every row to the three-term rescue pass: the whole batch goes through the gather
    kernels."""
    from ppocr_rechead import workloads as wl
    print(f"stress_1024 build (mode {mode})", flush=True)
    wk = wl.make("stress_1024", pack=orc.pack_int8)
    a, q, s, bias = wk["a"], wk["q"], wk["scales"], wk["bias"]
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    m = a.shape[0]
    guarded = head.guarded_rows(a, mode)
    print(f"stress_1024 fused decode, {int(guarded.sum())} of {m} rows guarded", flush=True)
    if mode == 2:
        assert guarded.mean() > 0.9
    got = head.decode(a, wk["line_off"], mode)
    head.close()
    assert got["idx"].min() >= 0 and got["idx"].max() < 18710
    assert np.all((got["maxprob"] > 0) & (got["maxprob"] <= 1))
    rng = np.random.default_rng(15)
    sample = np.unique(np.concatenate([wk["scaled_rows"], wk["tie_rows"], rng.choice(m, 2000, replace=False)]))
    ref = orc.rechead_lines(a[sample], split_lines(sample.size), q, s, bias)
    lg = f64_logits_q(a[sample], q, s, bias)
    gap = top2_gap(lg)
    exempt = check_argmax(got["idx"][sample], ref["idx"], gap, label="stress sample")
    print(f"  near-tie rows built: {wk['tie_rows'].size}, exempt differences: {exempt.size}")
    err = np.abs(got["maxprob"][sample] - ref["maxprob"])
    scaled = np.isin(sample, wk["scaled_rows"])
    print(f"  max|maxprob diff|: x50 rows {err[scaled].max():.3e}, other rows {err[~scaled].max():.3e}")
    assert_close_rel(got["maxprob"][sample], ref["maxprob"], "stress maxprob", row_scale=rel_scale(lg))


@pytest.mark.parametrize("m", [1500, 9000])
def test_skipped_row_blocks_beside_computed_ones(orc, rh, m):
    """BF16X2 on the stress head (precision limit 1.59, below the max|a| of unit-variance
    rows): a scan marks the row blocks whose rows all go to the rescue, lists their rows, and
    the main pass skips those blocks.  Rows scaled x0.3 (max|a| under the limit) hold their
    blocks back; the main pass computes those blocks and lists their other rows itself.  The
    1500-row batch runs 128-row blocks (its partial last block held back), the 9000-row one
    256-row blocks (its partial last block skipped).  Decode (argmax,
    maximum probability, sequences) and probabilities against the oracle on the rows of the
    held-back blocks and a seeded sample of the others; the channels-first entry bit for bit
    against the row entry."""
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights(stress=True)
    q, s = orc.pack_int8(w_t)
    rng = np.random.default_rng(41)
    a = rng.standard_normal((m, 120)).astype(np.float32)
    rb = 128 if m <= 8192 else 256
    # row blocks held back: with 1500 rows the last (partial) one among them, with 9000 rows the
    # last (40 rows) is skipped
    held = np.array([1, 5, (m - 1) // rb] if m == 1500 else [1, 5])
    small = np.concatenate([b * rb + rng.choice(min(rb, m - b * rb), 3, replace=False) for b in held])
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    prec, ra, _ = head.guard_limits(2)
    print(f"m={m}: limits prec {prec:.3f} range_amax {ra:.3f}", flush=True)
    # below both max|a| limits the row is not guarded, whatever its norm
    a[small] *= (np.float32(0.9 * min(prec, ra)) / np.abs(a[small]).max(axis=1))[:, None]
    guarded = head.guarded_rows(a, 2)
    print(f"m={m}: {int(guarded.sum())} of {m} rows guarded, {small.size} held back", flush=True)
    assert not guarded[small].any() and guarded.mean() > 0.9
    off = split_lines(m, 120)
    got = head.decode(a, off, 2)
    probs = head.probs(a, 2)
    # the same rows channels first ([lines][k][T], T = 60): the scan reads them one thread per row
    nct = head.decode_nct(np.ascontiguousarray(a.reshape(m // 60, 60, 120).transpose(0, 2, 1)), 2)
    head.close()
    assert np.array_equal(nct["idx"], got["idx"])
    assert np.array_equal(nct["maxprob"].view(np.uint32), got["maxprob"].view(np.uint32))
    in_held = np.concatenate([np.arange(b * rb, min(m, (b + 1) * rb)) for b in held])
    last = np.arange(((m - 1) // rb) * rb, m)  # the partial last block, skipped or held back
    sample = np.unique(np.concatenate([in_held, last, rng.choice(m, 600, replace=False)]))
    ref = orc.rechead_lines(a[sample], split_lines(sample.size), q, s, bias, want_probs=True)
    lg = f64_logits_q(a[sample], q, s, bias)
    check_argmax(got["idx"][sample], ref["idx"], top2_gap(lg), label=f"skipped blocks m={m}")
    assert_close_rel(got["maxprob"][sample], ref["maxprob"], "skipped blocks maxprob", row_scale=rel_scale(lg))
    assert_close_rel(probs[sample], ref["probs"], "skipped blocks probs", row_scale=rel_scale(lg))


@pytest.mark.parametrize("m", [600, 240])
@pytest.mark.parametrize("mode", [2, 4], ids=["bf16x2", "f16x2"])
def test_small_batch_rescue_inside_the_main_pass(orc, rh, mode, m):
    """Small batches of the two-term modes recompute their guarded rows inside the main
    pass (each workgroup its chunk of its rows, three bf16 terms) instead of in a rescue
    launch.  600 rows (five 128-row blocks): rows x30 and x300 in blocks 1 and 3 only, so
    blocks with and without guarded rows meet in one call; 240 rows (two blocks, the
    second a partial one): x30 rows in block 0, x300 rows in block 1.  Argmax,
    maximum probability, sequences and probabilities against the oracle, and the statistics
    pass's maxima against the probabilities pass's (each pass rescues the same rows)."""
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    q, s = orc.pack_int8(w_t)
    rng = np.random.default_rng(77)
    a = rng.standard_normal((m, 120)).astype(np.float32)
    if m == 600:
        big = np.concatenate([128 + rng.choice(128, 5, replace=False), 384 + rng.choice(128, 5, replace=False)])
    else:
        big = np.concatenate([rng.choice(128, 5, replace=False), 128 + rng.choice(m - 128, 5, replace=False)])
    a[big[:5]] *= np.float32(30.0)
    a[big[5:]] *= np.float32(300.0)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    guarded = head.guarded_rows(a, mode)
    print(f"mode {mode}: {int(guarded.sum())} of {m} rows guarded", flush=True)
    assert guarded[big[5:]].all() and not guarded[np.setdiff1d(np.arange(m), big)].any()
    off = split_lines(m, 120)
    got = head.decode(a, off, mode)
    idx2, mp2 = head.argmax(a, mode)
    probs = head.probs(a, mode)
    head.close()
    assert np.array_equal(got["idx"], idx2) and np.array_equal(got["maxprob"].view(np.uint32), mp2.view(np.uint32))
    ref = orc.rechead_lines(a, off, q, s, bias, want_probs=True)
    lg = f64_logits_q(a, q, s, bias)
    exempt = check_argmax(got["idx"], ref["idx"], top2_gap(lg), label=f"fused rescue mode {mode}")
    assert_close_rel(got["maxprob"], ref["maxprob"], "fused rescue maxprob", row_scale=rel_scale(lg))
    assert_close_rel(probs, ref["probs"], "fused rescue probs", row_scale=rel_scale(lg))
    np.testing.assert_allclose(probs.max(axis=1), got["maxprob"], rtol=1e-6, atol=1e-7)
    for b in range(len(off) - 1):
        if np.any((exempt >= off[b]) & (exempt < off[b + 1])):
            continue
        assert np.array_equal(got["seqs"][b], ref["seqs"][b]), b


def test_precision_guard_on_large_activations(orc, rh):
    """BF16X2 recomputes rows whose max|a| * max|w| exceeds the guard with three terms:
    x50 rows against the stress weights (+-5 outliers) stay as accurate as BF16X3."""
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights(stress=True)
    q, s = orc.pack_int8(w_t)
    rng = np.random.default_rng(16)
    a = rng.standard_normal((300, 120), dtype=np.float32)
    big = rng.choice(300, 40, replace=False)
    a[big] *= np.float32(50.0)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    print("guard logits x2 vs x3 vs oracle", flush=True)
    x2 = head.logits(a, 2)
    x3 = head.logits(a, 3)
    ref = orc.matmul_quantized_b(a, q, s, bias)
    tol = 1e-4 + 1e-5 * np.abs(ref)  # f32 rounding of |logits| ~ 1e3 alone is ~1e-4
    print(f"  max rel err x2 {np.max(np.abs(x2 - ref) / tol):.3f}, x3 {np.max(np.abs(x3 - ref) / tol):.3f}")
    assert np.all(np.abs(x2 - ref) <= tol)
    assert np.all(np.abs(x3 - ref) <= tol)
    idx, mp = head.argmax(a, 2)
    r = orc.rechead_lines(a, np.array([0, 300], np.int64), q, s, bias)
    assert_close_rel(mp, r["maxprob"], "guard maxprob", row_scale=rel_scale(f64_logits_q(a, q, s, bias)))
    head.close()


@pytest.mark.parametrize("bias_shift", [0.0, 55.0, 70.0])
def test_logit_range_guard(orc, rh, head, bias_shift):
    """The statistics pass skips its reference shift for rows whose logits are bounded by
    max|a| * max_c sum_k |w_ck| + max|b| <= 60; other rows go to the rescue pass.  Rows
    scaled x1 .. x48 straddle that limit and the precision limit; a bias shift of 55 leaves
    almost no room (nearly every row rescued), 70 none (the shift-keeping main pass).  A
    constant bias shift leaves the probabilities and the argmax unchanged."""
    rng = np.random.default_rng(21)
    factors = np.repeat(np.array([1, 2, 4, 8, 12, 16, 24, 48], np.float32), 16)
    a = rng.standard_normal((factors.size, 120), dtype=np.float32) * factors[:, None]
    bias = (head["bias"] + np.float32(bias_shift)).astype(np.float32)
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=bias)
    print(f"range guard bias_shift={bias_shift}", flush=True)
    idx, mp = h.argmax(a, 2)
    probs = h.probs(a[::8], 2)
    h.close()
    ref = orc.rechead_lines(a, split_lines(a.shape[0], 16), head["q"], head["s"], bias)
    lg = f64_logits_q(a, head["q"], head["s"], bias)
    check_argmax(idx, ref["idx"], top2_gap(lg), label=f"range guard shift {bias_shift}")
    err = np.abs(mp - ref["maxprob"])
    print(f"  max|maxprob diff| per factor: {[f'{e:.1e}' for e in err.reshape(8, 16).max(axis=1)]}")
    # a constant bias shift moves every logit by the same amount: the bar's allowance
    # follows the logits without it
    rs = rel_scale(lg - bias_shift)
    assert_close_rel(mp, ref["maxprob"], f"range guard maxprob shift {bias_shift}", row_scale=rs)
    refp = orc.rechead_lines(a[::8], split_lines(a[::8].shape[0], 8), head["q"], head["s"], bias, want_probs=True)
    assert_close_rel(probs, refp["probs"], f"range guard probs shift {bias_shift}", row_scale=rs[::8])


def _ctc_lines_host(idx, val, off, m, blank=0):
    """CTC collapse per line (CtcDecoder::decode_batch rules, src/postprocess/ctc.rs:151-163)
    with the device entry's offset clamping; f32 score summed in step order."""
    seqs, lens, scores = [], [], []
    for i in range(len(off) - 1):
        t0 = min(max(int(off[i]), 0), m)
        t1 = min(max(int(off[i + 1]), t0), m)
        prev, out, s = blank, [], np.float32(-0.0)
        for t in range(t0, t1):
            if idx[t] != blank and idx[t] != prev:
                out.append(int(idx[t]))
                s = np.float32(s + val[t])
            prev = idx[t]
        seqs.append((t0, out))
        lens.append(len(out))
        scores.append(np.float32(s / np.float32(len(out))) if out else np.float32(0.0))
    return seqs, np.array(lens, np.int64), np.array(scores, np.float32)


def test_decode_dev_one_merge_ctc_kernel(orc, rh, head, rhead):
    """ppocr_rh_decode_dev (chunk merge and CTC collapse in one kernel) equals
    ppocr_rh_argmax_dev + ppocr_ctc_greedy_dev bit for bit on the dense batch, and the
    restated collapse on ragged and malformed offsets (empty, reversed, past m, 300 rows)."""
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray, synchronize
    L = rh._lib.lib()
    a = wl.activations("dense_256")
    m = a.shape[0]
    off = wl.line_offsets([120] * 256)
    lines = len(off) - 1
    da, doff = DeviceArray.from_numpy(a), DeviceArray.from_numpy(off)
    di1, dp1 = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
    ds1, dl1, dc1 = DeviceArray((m,), np.int32), DeviceArray((lines,), np.int64), DeviceArray((lines,), np.float32)
    di2, dp2 = DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
    ds2, dl2, dc2 = DeviceArray((m,), np.int32), DeviceArray((lines,), np.int64), DeviceArray((lines,), np.float32)
    print("decode_dev vs argmax_dev + ctc_greedy_dev, dense_256", flush=True)
    rh._check(L.ppocr_rh_argmax_dev(rhead.handle, da.p, m, 2, di1.p, dp1.p, None, 0, None))
    rh._check(L.ppocr_ctc_greedy_dev(di1.p, dp1.p, doff.p, lines, 0, ds1.p, dl1.p, dc1.p, None))
    rh._check(L.ppocr_rh_decode_dev(rhead.handle, da.p, m, doff.p, lines, 2, di2.p, dp2.p, ds2.p, dl2.p, dc2.p,
                                    None, 0, None))
    synchronize()
    assert np.array_equal(di1.numpy(), di2.numpy())
    assert np.array_equal(dp1.numpy().view(np.uint32), dp2.numpy().view(np.uint32))
    l1, l2 = dl1.numpy(), dl2.numpy()
    assert np.array_equal(l1, l2)
    assert np.array_equal(dc1.numpy().view(np.uint32), dc2.numpy().view(np.uint32))
    s1, s2 = ds1.numpy(), ds2.numpy()
    for b in range(lines):
        assert np.array_equal(s1[off[b]:off[b] + l1[b]], s2[off[b]:off[b] + l2[b]]), b

    # ragged and malformed offsets on a small batch; idx/maxprob not requested
    rng = np.random.default_rng(31)
    mm = 700
    a2 = rng.standard_normal((mm, 120), dtype=np.float32)
    # empty lines, a 300-row line, offsets past m, a reversed and negative pair at the end
    off2 = np.array([0, 0, 5, 305, 420, 690, 700, 900, 950, -3], np.int64)
    n2 = len(off2) - 1
    da2, doff2 = DeviceArray.from_numpy(a2), DeviceArray.from_numpy(off2)
    ds3, dl3, dc3 = DeviceArray((mm,), np.int32), DeviceArray((n2,), np.int64), DeviceArray((n2,), np.float32)
    di4, dp4 = DeviceArray((mm,), np.int32), DeviceArray((mm,), np.float32)
    print("decode_dev ragged / malformed offsets", flush=True)
    rh._check(L.ppocr_rh_decode_dev(rhead.handle, da2.p, mm, doff2.p, n2, 2, None, None, ds3.p, dl3.p, dc3.p,
                                    None, 0, None))
    rh._check(L.ppocr_rh_argmax_dev(rhead.handle, da2.p, mm, 2, di4.p, dp4.p, None, 0, None))
    synchronize()
    seqs, lens, scores = _ctc_lines_host(di4.numpy(), dp4.numpy(), off2, mm)
    assert np.array_equal(dl3.numpy(), lens)
    assert np.array_equal(dc3.numpy().view(np.uint32), scores.view(np.uint32))
    s3 = ds3.numpy()
    for b, (t0, out) in enumerate(seqs):
        assert np.array_equal(s3[t0:t0 + len(out)], np.array(out, np.int32)), b

    # no rows at all: every line empty
    offz = np.zeros(4, np.int64)
    doffz = DeviceArray.from_numpy(offz)
    dlz, dcz = DeviceArray.from_numpy(np.full(3, 7, np.int64)), DeviceArray.from_numpy(np.full(3, 9.0, np.float32))
    rh._check(L.ppocr_rh_decode_dev(rhead.handle, None, 0, doffz.p, 3, 2, None, None, None, dlz.p, dcz.p,
                                    None, 0, None))
    synchronize()
    assert np.array_equal(dlz.numpy(), np.zeros(3, np.int64))
    assert np.array_equal(dcz.numpy(), np.zeros(3, np.float32))


def test_guard_list_in_a_reused_workspace(orc, rh):
    """The guarded-row list lives in the caller's workspace with an epoch-tagged header,
    so a workspace filled with 0xff bytes, or left by a larger guarded call, must not leak
    rows into the next call: argmax, decode and probabilities through one reused workspace
    equal those of calls with their own fresh workspace, bit for bit.  The stress weights
    (+-5 outliers) put many rows over the precision guard."""
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray, synchronize
    L = rh._lib.lib()
    w_t, bias = wl.weights(stress=True)
    q, s = orc.pack_int8(w_t)
    h = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    rng = np.random.default_rng(41)
    big = rng.standard_normal((1500, 120), dtype=np.float32)
    big[rng.choice(1500, 200, replace=False)] *= np.float32(50.0)
    small = rng.standard_normal((130, 120), dtype=np.float32)
    ws_bytes = max(h.workspace_bytes(1500, mode) for mode in (2, 3))
    ws = DeviceArray((ws_bytes,), np.uint8)
    ws.fill_bytes(0xFF)

    def argmax(a, mode, use_ws):
        m = a.shape[0]
        da, di, dp = DeviceArray.from_numpy(a), DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
        rh._check(L.ppocr_rh_argmax_dev(h.handle, da.p, m, mode, di.p, dp.p, ws.p if use_ws else None,
                                        ws_bytes if use_ws else 0, None))
        synchronize()
        return di.numpy(), dp.numpy().view(np.uint32)

    def decode(a, mode, use_ws):
        m = a.shape[0]
        off = np.array([0, m // 3, m // 3, m], np.int64)
        da, doff = DeviceArray.from_numpy(a), DeviceArray.from_numpy(off)
        dsq, dln, dsc = DeviceArray((m,), np.int32), DeviceArray((3,), np.int64), DeviceArray((3,), np.float32)
        rh._check(L.ppocr_rh_decode_dev(h.handle, da.p, m, doff.p, 3, mode, None, None, dsq.p, dln.p, dsc.p,
                                        ws.p if use_ws else None, ws_bytes if use_ws else 0, None))
        synchronize()
        ln = dln.numpy()
        # only seq[off[b] .. off[b] + len[b]) is defined; the rest of the array is not written
        emitted = np.concatenate([dsq.numpy()[off[b]:off[b] + ln[b]] for b in range(3)])
        return emitted, ln, dsc.numpy().view(np.uint32)

    def probs(a, mode, use_ws):
        m = a.shape[0]
        da, dpr = DeviceArray.from_numpy(a), DeviceArray((m, 18710), np.float32)
        rh._check(L.ppocr_rh_probs_dev(h.handle, da.p, m, mode, dpr.p, ws.p if use_ws else None,
                                       ws_bytes if use_ws else 0, None))
        synchronize()
        return (dpr.numpy().view(np.uint32),)

    for fn in (argmax, decode, probs):
        for a in (big, small, big[:700], small):
            print(f"reused workspace: {fn.__name__} m={a.shape[0]}", flush=True)
            for got, want in zip(fn(a, 2, True), fn(a, 2, False)):
                assert np.array_equal(got, want), (fn.__name__, a.shape[0])
    idx, _ = argmax(big, 2, True)
    ref = orc.rechead_lines(big[:64], np.array([0, 64], np.int64), q, s, bias)
    gap = top2_gap(f64_logits_q(big[:64], q, s, bias))
    check_argmax(idx[:64], ref["idx"], gap, label="reused workspace, stress head")
    h.close()


def test_workspace_holding_small_integers(orc, rh):
    """A caller workspace may hold anything before a call, in particular what calls of other
    sizes leave there: row and class indices, counts.  The guard header is the workspace's
    first 8 bytes and every epoch has its top bit set, so no such word reads as a list of
    the current call: with the workspace filled with small integers before each call, the
    fused head gives the results of a zeroed workspace, bit for bit."""
    from ppocr_rechead import workloads as wl
    from ppocr_rechead.hip import DeviceArray, hip, check, synchronize
    import ctypes
    L = rh._lib.lib()
    w_t, bias = wl.weights(stress=True)
    q, s = orc.pack_int8(w_t)
    h = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    rng = np.random.default_rng(43)
    a = rng.standard_normal((900, 120), dtype=np.float32)
    a[rng.choice(900, 120, replace=False)] *= np.float32(50.0)  # many guarded rows
    ws_bytes = h.workspace_bytes(900, 2)
    ws = DeviceArray((ws_bytes // 4 + 1,), np.int32)

    def run(m, fill):
        check(hip().hipMemcpy(ws.p, np.full(ws_bytes // 4 + 1, fill, np.int32).ctypes.data_as(ctypes.c_void_p),
                              ctypes.c_size_t(ws_bytes), 1), "hipMemcpy H2D")
        da, di, dp = DeviceArray.from_numpy(a[:m]), DeviceArray((m,), np.int32), DeviceArray((m,), np.float32)
        rh._check(L.ppocr_rh_argmax_dev(h.handle, da.p, m, 2, di.p, dp.p, ws.p, ws_bytes, None))
        synchronize()
        return di.numpy(), dp.numpy().view(np.uint32)

    for m in (900, 333, 64):
        want = run(m, 0)
        for fill in (1, 2, 3, 37, 1000, 0x7FFFFFFF):
            print(f"workspace of small integers: m={m} fill={fill}", flush=True)
            got = run(m, fill)
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), (m, fill)
    h.close()


def test_host_calls_from_many_threads(rh, rhead):
    """The handle is shared by threads (the reference's rec_pool workers): 8 threads
    decoding different line batches at once through the host-pointer entry point (each
    call takes its own device arena) get exactly the results of serial calls."""
    import threading
    from ppocr_rechead import workloads as wl
    rng = np.random.default_rng(23)
    jobs = []
    for t in range(8):
        lens = rng.integers(1, 130, size=int(rng.integers(1, 12)))
        off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        jobs.append((rng.standard_normal((int(off[-1]), 120)).astype(np.float32), off))
    print("host calls from 8 threads", flush=True)
    serial = [rhead.decode(a, off) for a, off in jobs]
    got = [None] * len(jobs)
    errors = []

    def work(t):
        try:
            for _ in range(5):
                got[t] = rhead.decode(*jobs[t])
        except Exception as e:  # reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(len(jobs))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for s, g in zip(serial, got):
        assert np.array_equal(s["idx"], g["idx"])
        assert np.array_equal(s["maxprob"].view(np.uint32), g["maxprob"].view(np.uint32))
        assert np.array_equal(s["score"].view(np.uint32), g["score"].view(np.uint32))
        for a, b in zip(s["seqs"], g["seqs"]):
            assert np.array_equal(a, b)


def test_probs_consistent_with_the_statistics_pass(orc, rh):
    """The probabilities pass recomputes every logit; it must take the same activation
    terms as the statistics pass for each row (rows between the range limit and the
    precision limit get three terms in both), or a row's own maximum stops mapping to
    exp2(0).  With a single class every probability is 1 (within f32 rounding of 1/sum)."""
    rng = np.random.default_rng(29)
    w = (rng.standard_normal((1, 120)) * 0.05).astype(np.float32)
    q, s = orc.pack_int8(w)
    bias = np.array([0.003], np.float32)
    factors = np.repeat(np.array([1, 4, 12, 24, 30, 48, 90], np.float32), 8)
    a = rng.standard_normal((factors.size, 120)).astype(np.float32) * factors[:, None]
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    print("probs of a one-class head", flush=True)
    for mode in (2, 3):
        p = head.probs(a, mode)
        err = np.abs(p - 1.0).max()
        print(f"  mode {mode}: max|p - 1| = {err:.2e}")
        assert err < 1e-6, (mode, err)
    head.close()


def test_free_functions_run_auto_on_a_resident_head(orc, rh, head):
    """The mirror's operator functions: matmul_quantized_b runs the library's default
    arithmetic (AUTO) on a head built once per QuantizedWeight and bias (a second call reuses
    it: same handle, same results) and stays within the bar of the oracle; an explicit mode
    and another bias get heads of their own; matmul_transposed_b runs AUTO on an FP32 head."""
    rng = np.random.default_rng(41)
    a = rng.standard_normal((300, 120)).astype(np.float32)
    qw = rh.QuantizedWeight(head["q"], head["s"])
    got1 = rh.matmul_quantized_b(a, qw, head["bias"])
    h1 = qw._gpu_heads[head["bias"].tobytes()].handle.value
    got2 = rh.matmul_quantized_b(a, qw, head["bias"])
    assert qw._gpu_heads[head["bias"].tobytes()].handle.value == h1 and np.array_equal(got1, got2)
    ref = orc.matmul_quantized_b(a, head["q"], head["s"], head["bias"], partition_threads=1)
    assert np.abs(got1 - ref).max() < TOL
    auto = qw._gpu_heads[head["bias"].tobytes()].auto_mode()
    assert np.array_equal(got1, rh.matmul_quantized_b(a, qw, head["bias"], mode=auto))
    got_nb = rh.matmul_quantized_b(a, qw)
    assert len(qw._gpu_heads) == 2
    assert np.abs(got_nb - orc.matmul_quantized_b(a, head["q"], head["s"], None, partition_threads=1)).max() < TOL
    w_t = (rng.standard_normal((500, 120)) * 0.05).astype(np.float32)
    b = (rng.standard_normal(500) * 0.01).astype(np.float32)
    got_f = rh.matmul_transposed_b(a, w_t, b)
    assert np.abs(got_f - orc.matmul_transposed_b(a, w_t, b, partition_threads=1)).max() < TOL
    for hd in qw._gpu_heads.values():
        hd.close()
