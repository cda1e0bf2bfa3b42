"""GPU parity where the bars bite: the FP32 head at the 64-line batch size (m = 7680),
peaked outputs (one class near probability 1, as the real model gives), rows sized
around the precision guards' limits, and the whole dense 256-line batch.

Probabilities and maximum probabilities are held to 1e-4 absolute and 1e-4 relative
(rows whose logits exceed 10 in magnitude get a proportionally wider relative bar for the
fp32 rounding both sides carry); logits to 1e-4; argmax and CTC sequences identical except
at top-2 logit gaps below 1e-4, which are printed."""
import numpy as np
import pytest

from gpu_common import (assert_close_rel, check_argmax, dot_tol, f64_logits_f32, f64_logits_q, oracle_head_f32,
                        peaked_rows, rel_scale, split_lines, top2_gap)

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def head(orc):
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    q, s = orc.pack_int8(w_t)
    return {"w_t": w_t, "bias": bias, "q": q, "s": s, "wd": q.astype(np.float64) * s.astype(np.float64)[:, None]}


def _int8_limit(q, s):
    """The INT8 head's precision limit on max|a| (two activation terms), computed as the
    library does: min(16 / max|w|, 8 / max_c ||w_c||_2) on the dequantised weight."""
    qa = np.abs(q.astype(np.int64))
    wmax = float(np.max((qa.max(axis=1).astype(np.float32) * s).astype(np.float32)))
    l2 = float(np.max(np.sqrt((qa * qa).sum(axis=1).astype(np.float64)) * s.astype(np.float64)))
    return min(16.0 / wmax, 8.0 / l2)


def _f32_limit(w_t):
    w = np.abs(w_t.astype(np.float64))
    return min(16.0 / float(np.abs(w_t).max()), 4.0 / float(np.sqrt((w * w).sum(axis=1)).max()))


def _f16_limit_f32(w_t):
    """An FP32 head's limit with fp16 halves of both operands (F16X2): min(32768, 64 / L2)."""
    w = np.abs(w_t.astype(np.float64))
    return min(32768.0, 64.0 / float(np.sqrt((w * w).sum(axis=1)).max()))


def _f16_limit_int8(q, s):
    """The INT8 head's limit with two fp16 activation terms: min(32768, 512 / L2)."""
    qa = np.abs(q.astype(np.int64))
    l2 = float(np.max(np.sqrt((qa * qa).sum(axis=1).astype(np.float64)) * s.astype(np.float64)))
    return min(32768.0, 512.0 / l2)


@pytest.mark.parametrize("mode", [0, 3, 4])
def test_fp32_head_m7680_logits(orc, rh, mode):
    """The FP32 head at 64 lines x T=120 (m = 7680), every row's logits from the GPU, sampled
    rows (the last row block among them) against matmul_transposed_b."""
    from ppocr_rechead import workloads as wl
    wk = wl.make("fp32_64")
    a, w_t, bias = wk["a"], wk["w_t"], wk["bias"]
    m = a.shape[0]
    assert m == 7680
    head = rh.RecHead(w_t=w_t, bias=bias)
    print(f"fp32 head m={m} mode={mode} logits", flush=True)
    got = head.logits(a, mode)
    head.close()
    rng = np.random.default_rng(31)
    sample = np.unique(np.concatenate([rng.choice(m - 128, 256, replace=False), np.arange(m - 128, m)]))
    ref = orc.matmul_transposed_b(a[sample], w_t, bias, partition_threads=1)
    err = np.abs(got[sample] - ref).max()
    print(f"  max|logits gpu-oracle| = {err:.3e} over {sample.size} rows")
    assert err < TOL


@pytest.mark.parametrize("mode", [0, 3, 4])
def test_fp32_head_m7680_decode(orc, rh, mode):
    """The fused head (statistics pass, chunk merge, CTC) with the FP32 weight at m = 7680:
    every row's argmax and maximum probability and every line's sequence and score against
    the oracle's FP32 head (matmul_transposed_b, softmax, find_argmax, collapse)."""
    from ppocr_rechead import workloads as wl
    wk = wl.make("fp32_64")
    a, w_t, bias, off = wk["a"], wk["w_t"], wk["bias"], wk["line_off"]
    head = rh.RecHead(w_t=w_t, bias=bias)
    print(f"fp32 head m={a.shape[0]} mode={mode} decode", flush=True)
    got = head.decode(a, off, mode)
    head.close()
    ref = oracle_head_f32(orc, a, w_t, bias, off)
    mis = np.nonzero(got["idx"] != ref["idx"])[0]
    gap = np.full(a.shape[0], np.inf)
    if mis.size:
        gap[mis] = top2_gap(f64_logits_f32(a[mis], w_t, bias))
    exempt = check_argmax(got["idx"], ref["idx"], gap, label=f"fp32 m7680 mode {mode}")
    assert_close_rel(got["maxprob"], ref["maxprob"], f"fp32 m7680 maxprob mode {mode}")
    for b in range(len(off) - 1):
        if np.any((exempt >= off[b]) & (exempt < off[b + 1])):
            continue
        assert np.array_equal(got["seqs"][b], ref["seqs"][b]), b
        assert abs(float(got["score"][b]) - float(ref["score"][b])) <= TOL * max(1e-3, abs(float(ref["score"][b])))


@pytest.mark.parametrize("mode", [2, 3, 4])
def test_peaked_outputs_decode_and_probs(orc, rh, head, mode):
    """Rows built so that one class dominates (maximum probability ~0.5 .. 0.99, blank and
    repeated classes among the targets, as in real CTC output): decode and probabilities
    against the oracle.  Here the 1e-4 bar on the maximum probability is what a lost or
    doubled term of the softmax sum would break."""
    rng = np.random.default_rng(32)
    lens = [120, 80, 37, 1, 120]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    m = int(off[-1])
    # a text-like target sequence: runs of the same class separated by blanks
    targets = np.zeros(m, np.int64)
    t = 0
    while t < m:
        run = int(rng.integers(1, 5))
        targets[t:t + run] = 0 if rng.random() < 0.4 else int(rng.integers(1, 18710))
        t += run
    alpha = rng.uniform(15.0, 30.0, m)
    a = peaked_rows(head["wd"], targets, alpha, rng)
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=head["bias"])
    print(f"peaked rows m={m} mode={mode}", flush=True)
    got = h.decode(a, off, mode)
    probs = h.probs(a[:200], mode)
    h.close()
    ref = orc.rechead_lines(a, off, head["q"], head["s"], head["bias"])
    lg = f64_logits_q(a, head["q"], head["s"], head["bias"])
    print(f"  maxprob range {ref['maxprob'].min():.3f} .. {ref['maxprob'].max():.4f}, "
          f"median {np.median(ref['maxprob']):.3f}; targets hit {np.mean(ref['idx'] == targets):.3f}")
    assert np.median(ref["maxprob"]) > 0.8
    exempt = check_argmax(got["idx"], ref["idx"], top2_gap(lg), label=f"peaked mode {mode}")
    assert_close_rel(got["maxprob"], ref["maxprob"], f"peaked maxprob mode {mode}", row_scale=rel_scale(lg))
    for b in range(len(lens)):
        if np.any((exempt >= off[b]) & (exempt < off[b + 1])):
            continue
        assert np.array_equal(got["seqs"][b], ref["seqs"][b]), b
        assert abs(float(got["score"][b]) - float(ref["score"][b])) <= TOL * max(1e-3, abs(float(ref["score"][b])))
    refp = orc.rechead_lines(a[:200], split_lines(200, 50), head["q"], head["s"], head["bias"], want_probs=True)
    assert_close_rel(probs, refp["probs"], f"peaked probs mode {mode}", row_scale=rel_scale(lg[:200]))


def test_int8_logits_around_the_precision_limit(orc, rh, head):
    """BF16X2 logits of rows whose max|a| is 0.5 .. 0.99 of the precision limit (two
    activation terms) and 1.01 .. 3 of it (recomputed with three) against the oracle."""
    lim = _int8_limit(head["q"], head["s"])
    rng = np.random.default_rng(33)
    fr = np.concatenate([np.linspace(0.5, 0.99, 96), np.linspace(1.01, 3.0, 32)])
    a = rng.standard_normal((fr.size, 120)).astype(np.float32)
    a = (a / np.abs(a).max(axis=1, keepdims=True) * (fr * lim)[:, None]).astype(np.float32)
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=head["bias"])
    print(f"int8 logits around the limit {lim:.3f}", flush=True)
    got = h.logits(a, 2)
    idx, mp = h.argmax(a, 2)
    h.close()
    ref = orc.matmul_quantized_b(a, head["q"], head["s"], head["bias"])
    err = np.abs(got - ref).max(axis=1)
    print(f"  max|logits diff| under the limit {err[:96].max():.2e}, over it {err[96:].max():.2e}")
    assert err.max() < TOL
    r = orc.rechead_lines(a, split_lines(a.shape[0], 32), head["q"], head["s"], head["bias"])
    check_argmax(idx, r["idx"], top2_gap(f64_logits_q(a, head["q"], head["s"], head["bias"])), label="int8 limit")
    assert_close_rel(mp, r["maxprob"], "int8 limit maxprob")


@pytest.mark.parametrize("mode", [3, 4], ids=["bf16x3", "f16x2"])
def test_fp32_head_precision_guard(orc, rh, mode):
    """BF16X3 and F16X2 on an FP32 head: rows of max|a| 0.5 .. 0.99 of the mode's precision
    limit stay on the MFMA path, rows above it (to 3x the limit, and x50 of an N(0,1) row)
    are recomputed in fp32 FMA.  Logits, the fused argmax and the probabilities against the
    oracle.  The limit is computed here from the weights and checked against the library's."""
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights()
    lim = _f32_limit(w_t) if mode == 3 else _f16_limit_f32(w_t)
    rng = np.random.default_rng(34)
    fr = np.concatenate([np.linspace(0.5, 0.99, 64), np.linspace(1.01, 3.0, 32)])
    a = rng.standard_normal((fr.size, 120)).astype(np.float32)
    a = (a / np.abs(a).max(axis=1, keepdims=True) * (fr * lim)[:, None]).astype(np.float32)
    big = rng.standard_normal((32, 120)).astype(np.float32) * np.float32(50.0)
    a = np.concatenate([a, big]).astype(np.float32)
    head = rh.RecHead(w_t=w_t, bias=bias)
    print(f"fp32 head guard, mode {mode}, limit {lim:.3f}", flush=True)
    assert head.guard_limits(mode)[0] == pytest.approx(lim, rel=1e-5)
    got = head.logits(a, mode)
    idx, mp = head.argmax(a, mode)
    probs = head.probs(a, mode)
    head.close()
    ref = oracle_head_f32(orc, a, w_t, bias, np.array([0, a.shape[0]], np.int64), want_probs=True)
    lg = f64_logits_f32(a, w_t, bias)
    tol = 1e-4 + 1e-5 * np.abs(ref["logits"])  # f32 rounding of |logits| ~ 1e2 alone is ~1e-5
    err = np.abs(got - ref["logits"])
    print(f"  max|logits diff|: under {err[:64].max():.2e}, over {err[64:96].max():.2e}, x50 {err[96:].max():.2e}")
    assert np.all(err <= tol)
    check_argmax(idx, ref["idx"], top2_gap(lg), label=f"fp32 guard mode {mode}")
    assert_close_rel(mp, ref["maxprob"], f"fp32 guard maxprob mode {mode}", row_scale=rel_scale(lg))
    assert_close_rel(probs, ref["probs"], f"fp32 guard probs mode {mode}", row_scale=rel_scale(lg))


def test_dense_256_whole_batch(orc, rh, head):
    """The fused decode of the dense 256-line batch (m = 30720) against the oracle on every
    row and every line."""
    from ppocr_rechead import workloads as wl
    a = wl.activations("dense_256")
    off = wl.line_offsets(wl.lines_for("dense_256"))
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=head["bias"])
    print("dense_256 whole batch decode", flush=True)
    got = h.decode(a, off, 2)
    h.close()
    ref = orc.rechead_lines(a, off, head["q"], head["s"], head["bias"])
    mis = np.nonzero(got["idx"] != ref["idx"])[0]
    gap = np.full(a.shape[0], np.inf)
    if mis.size:
        gap[mis] = top2_gap(f64_logits_q(a[mis], head["q"], head["s"], head["bias"]))
    exempt = check_argmax(got["idx"], ref["idx"], gap, label="dense_256 all rows")
    assert_close_rel(got["maxprob"], ref["maxprob"], "dense_256 maxprob")
    same = 0
    for b in range(len(off) - 1):
        if np.any((exempt >= off[b]) & (exempt < off[b + 1])):
            continue
        assert np.array_equal(got["seqs"][b], ref["seqs"][b]), b
        assert abs(float(got["score"][b]) - float(ref["score"][b])) <= TOL * max(1e-3, abs(float(ref["score"][b])))
        same += 1
    print(f"  {same} of {len(off) - 1} lines identical (the rest hold near-tie rows)")


def test_f16x2_around_its_limit_and_range(orc, rh, head):
    """F16X2 (two fp16 activation terms) logits and fused argmax for rows of max|a| 0.5 ..
    0.99 of its precision limit, 1.01 .. 3 of it (recomputed with three bf16 terms), and
    rows beyond the fp16 range (|a| up to 1e5, recomputed) against the oracle; the logits'
    bar grows with the magnitude of the products by the fp32 rounding the reference itself
    carries (dot_tol)."""
    lim = _f16_limit_int8(head["q"], head["s"])
    rng = np.random.default_rng(35)
    fr = np.concatenate([np.linspace(0.5, 0.99, 64), np.linspace(1.01, 3.0, 32)])
    a = rng.standard_normal((fr.size, 120)).astype(np.float32)
    a = (a / np.abs(a).max(axis=1, keepdims=True) * (fr * lim)[:, None]).astype(np.float32)
    huge = rng.standard_normal((16, 120)).astype(np.float32) * np.float32(3e4)
    a = np.concatenate([a, huge]).astype(np.float32)
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=head["bias"])
    print(f"f16x2 around the limit {lim:.1f} and beyond the fp16 range", flush=True)
    got = h.logits(a, 4)
    idx, mp = h.argmax(a, 4)
    h.close()
    ref = orc.matmul_quantized_b(a, head["q"], head["s"], head["bias"])
    tol = dot_tol(a, head["wd"])
    err = np.abs(got - ref)
    print(f"  max|logits diff|: under {err[:64].max():.2e}, over {err[64:96].max():.2e}, beyond range "
          f"{err[96:].max():.2e} (|logit| up to {np.abs(ref).max():.0f})")
    assert np.all(err <= tol)
    lg = f64_logits_q(a, head["q"], head["s"], head["bias"])
    r = orc.rechead_lines(a, split_lines(a.shape[0], 16), head["q"], head["s"], head["bias"])
    check_argmax(idx, r["idx"], top2_gap(lg), label="f16x2 limit")
    assert_close_rel(mp, r["maxprob"], "f16x2 limit maxprob", row_scale=rel_scale(lg))


@pytest.mark.parametrize("mode", [2, 4])
def test_tiny_activations(orc, rh, head, mode):
    """Rows of magnitude 1e-3 .. 1e-7 (fp16 terms in and below the subnormal range, bf16
    terms far from it): logits within 1e-4 and the fused argmax against the oracle."""
    rng = np.random.default_rng(36)
    a = np.concatenate([rng.standard_normal((32, 120)) * sc for sc in (1e-3, 1e-4, 1e-5, 1e-7)]).astype(np.float32)
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=head["bias"])
    print(f"tiny activations mode {mode}", flush=True)
    got = h.logits(a, mode)
    idx, mp = h.argmax(a, mode)
    h.close()
    ref = orc.matmul_quantized_b(a, head["q"], head["s"], head["bias"])
    err = np.abs(got - ref).max()
    print(f"  max|logits diff| {err:.2e}")
    assert err < TOL
    r = orc.rechead_lines(a, split_lines(a.shape[0], 32), head["q"], head["s"], head["bias"])
    check_argmax(idx, r["idx"], top2_gap(f64_logits_q(a, head["q"], head["s"], head["bias"])), label="tiny")
    assert_close_rel(mp, r["maxprob"], f"tiny maxprob mode {mode}")


def test_guard_limits_query(orc, rh):
    """ppocr_rh_guard_limits reports the limits the kernels apply: for the INT8 head the
    precision limits of the bf16 and fp16 splits and, for the statistics pass, the logit
    range bounds (60 - 1.001 max|bias|) / (1.001 max_c ||w_c||_1) on max|a| and
    (60 - 1.001 max|bias|) / (1.001 max_c ||w_c||_2) on ||a||_2 (the latter squared with a
    0.1% margin); no guard (inf) in the one- and three-term modes and in fp32 FMA."""
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights(stress=True)
    q, s = orc.pack_int8(w_t)
    h = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    wd = np.abs(q.astype(np.float64)) * s.astype(np.float64)[:, None]
    room = 60.0 - 1.001 * float(np.abs(bias).max())
    rng_amax = room / (1.001 * float(wd.sum(axis=1).max()))
    rng_norm = room / (1.001 * float(np.sqrt((wd * wd).sum(axis=1)).max())) * np.sqrt(0.999)
    for mode, prec in ((2, _int8_limit(q, s)), (4, _f16_limit_int8(q, s))):
        p, ra, rn = h.guard_limits(mode)
        print(f"mode {mode}: precision {p:.4f} ({prec:.4f}), range max|a| {ra:.4f} ({rng_amax:.4f}), "
              f"range ||a|| {rn:.4f} ({rng_norm:.4f})")
        assert abs(p - prec) <= 1e-5 * prec
        assert abs(ra - rng_amax) <= 1e-5 * rng_amax and abs(rn - rng_norm) <= 1e-5 * rng_norm
    for mode in (0, 1, 3):
        assert h.guard_limits(mode) == (np.inf, np.inf, np.inf)
    h.close()


def test_rows_over_the_range_bound_but_within_the_norm_bound(orc, rh, head):
    """Rows whose max|a| exceeds the logit range bound on max|a| but whose ||a||_2 proves
    the range (a few large entries, or many moderate ones, as the activations after the
    SVTR tail's final LayerNorm have) stay on the split path of decode and probabilities
    and meet the bars there."""
    h = rh.RecHead(qw=rh.QuantizedWeight(head["q"], head["s"]), bias=head["bias"])
    prec, ra, rn = h.guard_limits(4)
    rng = np.random.default_rng(43)
    a = rng.standard_normal((512, 120)).astype(np.float32)
    # moderate entries everywhere, scaled so max|a| lies between the two range bounds
    a *= (np.float32(ra * 1.3) / np.abs(a).max(axis=1))[:, None]
    keep = np.sqrt((a.astype(np.float64) ** 2).sum(1)) < rn * 0.98
    a = a[keep][:256]
    assert a.shape[0] >= 64 and not h.guarded_rows(a, 4).any() and (np.abs(a).max(1) > ra).all()
    off = np.array([0, 100, a.shape[0]], np.int64)
    for mode in (4, 2):
        got = h.decode(a, off, mode=mode)
        ref = orc.rechead_lines(a, off, head["q"], head["s"], head["bias"])
        lg = f64_logits_q(a, head["q"], head["s"], head["bias"])
        check_argmax(got["idx"], ref["idx"], top2_gap(lg), label=f"range by norm, mode {mode}")
        assert_close_rel(got["maxprob"], ref["maxprob"], f"range by norm maxprob mode {mode}", row_scale=rel_scale(lg))
        probs = h.probs(a[:64], mode)
        refp = orc.softmax_rows(orc.matmul_quantized_b(a[:64], head["q"], head["s"], head["bias"]))
        assert_close_rel(probs, refp, f"range by norm probs mode {mode}", row_scale=rel_scale(lg[:64]))
    h.close()


def test_f16x2_outlier_head_needs_no_rescue_for_ordinary_rows(orc, rh):
    """The stress head (0.5% of its classes hold a single +-5 weight): with fp16 terms its
    precision limit stays far above ordinary rows' magnitudes, and the logits of N(0,1) rows
    (max|a| ~ 3..5) meet the bar on the two-term path itself.  Checked on rows that the
    bf16 limit would send to the rescue."""
    from ppocr_rechead import workloads as wl
    w_t, bias = wl.weights(stress=True)
    q, s = orc.pack_int8(w_t)
    lim16 = _f16_limit_int8(q, s)
    lim_bf = _int8_limit(q, s)
    rng = np.random.default_rng(37)
    a = rng.standard_normal((256, 120)).astype(np.float32)
    amax = np.abs(a).max(axis=1)
    print(f"stress head: bf16 limit {lim_bf:.2f}, fp16 limit {lim16:.1f}; rows over the bf16 limit "
          f"{int((amax > lim_bf).sum())}/256, over the fp16 limit {int((amax > lim16).sum())}/256", flush=True)
    assert (amax > lim_bf).mean() > 0.9 and not np.any(amax > lim16)
    h = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    got = h.logits(a, 4)
    h.close()
    err = np.abs(got - orc.matmul_quantized_b(a, q, s, bias)).max()
    print(f"  max|logits diff| {err:.2e}")
    assert err < TOL


def test_auto_mode_picks_per_head_and_matches_the_explicit_mode(orc, rh):
    """MODE_AUTO, the default: the fp16 split unless the bf16 limit is at least 32 (then the
    bf16 split): the synthetic INT8 head (~11.7), the stress head (~1.6) and the synthetic
    FP32 head (~5.8) all take the fp16 split, a head with weights 1/8 as large (limit ~94)
    the bf16 one.  Its results are those of the explicit mode, bit for bit, on logits and
    on the decode."""
    from ppocr_rechead import workloads as wl
    rng = np.random.default_rng(41)
    a = rng.standard_normal((512, 120)).astype(np.float32)
    off = np.array([0, 40, 40, 300, 512], np.int64)
    cases = []
    w_t, bias = wl.weights()
    q, s = orc.pack_int8(w_t)
    cases.append(("int8", rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias), _int8_limit(q, s)))
    w_t2, bias2 = wl.weights(stress=True)
    q2, s2 = orc.pack_int8(w_t2)
    cases.append(("int8 stress", rh.RecHead(qw=rh.QuantizedWeight(q2, s2), bias=bias2), _int8_limit(q2, s2)))
    cases.append(("fp32", rh.RecHead(w_t=w_t, bias=bias), _f32_limit(w_t)))
    w_s = (w_t / np.float32(8.0)).astype(np.float32)
    q3, s3 = orc.pack_int8(w_s)
    cases.append(("int8 small weights", rh.RecHead(qw=rh.QuantizedWeight(q3, s3), bias=bias), _int8_limit(q3, s3)))
    for name, h, lim in cases:
        want = (rh.MODE_BF16X2 if h.quantized else rh.MODE_BF16X3) if lim >= 32.0 else rh.MODE_F16X2
        print(f"{name}: bf16 limit {lim:.2f} -> auto mode {h.auto_mode()}", flush=True)
        assert h.auto_mode() == want
        assert h.default_mode == rh.MODE_AUTO
        prec, ra, rn = h.guard_limits(want)
        assert h.quantized or (ra == np.inf and rn == np.inf)
        if want != rh.MODE_F16X2:
            assert abs(prec - lim) <= 1e-5 * lim, (prec, lim)
        np.testing.assert_array_equal(h.logits(a), h.logits(a, want))
        d_auto, d_want = h.decode(a, off), h.decode(a, off, mode=want)
        for key in ("idx", "maxprob", "score"):
            np.testing.assert_array_equal(d_auto[key], d_want[key])
        for x, y in zip(d_auto["seqs"], d_want["seqs"]):
            np.testing.assert_array_equal(x, y)
        h.close()
