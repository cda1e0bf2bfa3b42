"""Shared helpers of the GPU parity tests."""
import numpy as np


def f64_logits_q(a, q, s, bias):
    wd = q.astype(np.float64) * s.astype(np.float64)[:, None]
    return a.astype(np.float64) @ wd.T + (0.0 if bias is None else bias.astype(np.float64))


def top2_gap(logits64):
    """Top-1 minus top-2 logit per row (f64)."""
    part = np.partition(logits64, -2, axis=1)[:, -2:]
    return part[:, 1] - part[:, 0]


def check_argmax(got_idx, ref_idx, gap, tol=1e-4, label=""):
    """Indices must match except where the top-2 gap is below tol; returns the exempt rows."""
    diff = np.nonzero(got_idx != ref_idx)[0]
    bad = diff[gap[diff] >= tol]
    assert bad.size == 0, f"{label}: {bad.size} argmax mismatches with top-2 gap >= {tol}: rows {bad[:10]}"
    if diff.size:
        print(f"[{label}] {diff.size} near-tie argmax differences (gaps {np.sort(gap[diff])[:5]})")
    return diff


def split_lines(rows, t=64):
    """Offsets cutting `rows` independent rows into lines of t, so the oracle runs them in
    parallel (per-row results do not depend on the line split)."""
    off = list(range(0, rows, t)) + [rows]
    return np.asarray(off, dtype=np.int64)


def f64_logits_f32(a, w_t, bias):
    return a.astype(np.float64) @ w_t.astype(np.float64).T + (0.0 if bias is None else bias.astype(np.float64))


def rel_scale(logits64):
    """Per-row allowance factor of the relative bar: 1 for rows whose logits stay within
    +-10, |logit|max / 10 above.  fp32 logits of magnitude L carry rounding of ~L * 2^-23 *
    sqrt(k) on both sides (the reference's own arithmetic included), which becomes relative
    error of the probabilities; rows of ordinary magnitude get the plain bar."""
    return np.maximum(1.0, np.abs(logits64).max(axis=1) / 10.0)


def assert_close_rel(got, ref, label, abs_tol=1e-4, rel_tol=1e-4, row_scale=None):
    """Probabilities and maximum probabilities: |got - ref| <= abs_tol, and <= rel_tol * |ref|
    (times row_scale per row, when given; a floor of 1e-30 covers denormals flushed to 0).
    On the synthetic workloads every probability is ~4e-4 or less, so the absolute bar alone
    would allow ~25% relative error; the relative bar is what a lost term of a sum trips."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    tol = rel_tol * np.abs(ref)
    if row_scale is not None:
        rs = np.asarray(row_scale, np.float64)
        tol = tol * (rs if got.ndim == 1 else rs[:, None])
    tol = tol + 1e-30
    worst = float(np.max(d / tol)) if d.size else 0.0
    print(f"  [{label}] max abs diff {float(d.max()) if d.size else 0.0:.3e}, "
          f"max diff / relative bar {worst:.3f}")
    assert d.size == 0 or float(d.max()) < abs_tol, label
    assert np.all(d <= tol), f"{label}: relative bar exceeded ({worst:.2f} x)"


def oracle_head_f32(orc, a, w_t, bias, line_off, want_probs=False):
    """The whole head with an FP32 weight through the oracle's parts: matmul_transposed_b,
    softmax, find_argmax per row, CTC collapse (the per-line composition of
    src/pipeline.rs:395-436 with the FP32 MatMul.12)."""
    logits = orc.matmul_transposed_b(a, w_t, bias, partition_threads=1)
    probs = orc.softmax_rows(logits)
    idx, mp = orc.argmax_rows(probs)
    seqs, score = orc.ctc_collapse(idx, mp, line_off)
    return {"idx": idx, "maxprob": mp, "seqs": seqs, "score": score, "probs": probs if want_probs else None,
            "logits": logits}


def peaked_rows(wd, targets, alpha, rng, noise=0.3):
    """Activations whose head output is dominated by one class: a = alpha * w_c / ||w_c||
    + noise for target class c of each row (wd the dequantised weight [n][k]).  With the
    synthetic N(0, 0.05^2) head, alpha 15 .. 30 gives maximum probabilities ~0.5 .. 0.99."""
    w = wd[targets].astype(np.float64)
    w /= np.linalg.norm(w, axis=1, keepdims=True)
    a = alpha[:, None] * w + noise * rng.standard_normal(w.shape)
    return a.astype(np.float32)


def dot_tol(a, wd, base=1e-4):
    """Logit bar for rows of large magnitude: base plus the fp32 rounding a length-k dot
    product carries, 8 sqrt(k) ulps (2^-24) of the magnitude of its terms sum_k |a_k w_k|
    (the reference's own arithmetic carries that much; for ordinary rows it adds ~2e-5)."""
    k = a.shape[1]
    mag = np.abs(a.astype(np.float64)) @ np.abs(wd.astype(np.float64)).T
    return base + 8.0 * np.sqrt(k) * 2.0 ** -24 * mag
