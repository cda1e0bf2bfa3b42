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
