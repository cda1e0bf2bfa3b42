"""Exact ties of the fused argmax, the case that tells `find_argmax`'s first-occurrence rule
(src/postprocess/ctc.rs:178-258) from any other: identical weight rows (identical int8 rows,
scales and biases, so identical logits in every arithmetic) inside one lane half of a
32-class tile of the statistics pass, across the two halves of a tile (the lower class sits
in the half whose lanes hold the higher classes of the other quads), and across tiles.  The
statistics pass saves a raised maximum's tile values and takes the first class equal to the
maximum; its small-batch (one row block per wave) and large-batch (two per wave, above 8192
rows) kernels, every mode and every entry point (argmax, decode, channels-first decode) must
give the first class on every row.  Random rows of a large batch are held to the oracle as
elsewhere (argmax except top-2 gaps below 1e-4)."""
import numpy as np
import pytest

from gpu_common import assert_close_rel, check_argmax, f64_logits_q, rel_scale, split_lines, top2_gap

pytestmark = pytest.mark.gpu

K = 120
# tie groups: (classes with identical weight rows, k range of the group's weights); the
# expected index is the group's lowest class.  Class c of a tile sits in lane half
# (c % 32 // 4) % 2.
GROUPS = [
    ((3, 1), (0, 24)),           # tile 0, both in half 0
    ((8, 5), (24, 48)),          # tile 0, halves 0 and 1: the first class (5) is in half 1
    ((70, 40), (48, 72)),        # tiles 2 and 1
    ((101, 100, 96), (72, 96)),  # tile 3: half 0 holds the first (96), half 1 two more
    ((157, 150), (96, 120)),     # tile 4, both in half 1
]
N = 200


def _tie_head(orc):
    rng = np.random.default_rng(21)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    for classes, (k0, k1) in GROUPS:
        row = np.zeros(K, np.float32)
        row[k0:k1] = 0.5
        for c in classes:
            w[c] = row
            bias[c] = 0.0
    q, s = orc.pack_int8(w)
    for classes, _ in GROUPS:
        for c in classes[1:]:
            assert np.array_equal(q[c], q[classes[0]]) and s[c] == s[classes[0]]
    return q, s, bias


def _tie_rows(m, seed):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((m, K)) * 0.3).astype(np.float32)
    group = np.arange(m) % len(GROUPS)
    for g, (_, (k0, k1)) in enumerate(GROUPS):
        a[group == g, k0:k1] += 2.0
    expect = np.array([min(GROUPS[g][0]) for g in group], np.int32)
    return a, expect


@pytest.mark.parametrize("m", [3000, 10000])
@pytest.mark.parametrize("mode", [2, 4, 5, 3, 0])
def test_exact_ties_resolve_to_the_first_class(orc, rh, mode, m):
    q, s, bias = _tie_head(orc)
    a, expect = _tie_rows(m, 5)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    try:
        idx, mp = head.argmax(a, mode)
        bad = np.nonzero(idx != expect)[0]
        assert bad.size == 0, f"mode {mode}: {bad.size} rows off the first tied class, e.g. rows {bad[:5]} " \
                              f"got {idx[bad[:5]]} expected {expect[bad[:5]]}"
        lines = 40 if m == 3000 else 80
        off = np.arange(0, m + 1, m // lines, dtype=np.int64)
        dec = head.decode(a, off, mode)
        assert np.array_equal(dec["idx"], idx) and np.array_equal(dec["maxprob"], mp)
        nct = head.decode_nct(a.reshape(lines, m // lines, K).transpose(0, 2, 1).copy(), mode)
        assert np.array_equal(nct["idx"], idx) and np.array_equal(nct["maxprob"], mp)
    finally:
        head.close()
    ref = orc.rechead_lines(a[:500], split_lines(500), q, s, bias)
    assert np.array_equal(ref["idx"], expect[:500]), "the oracle's first occurrence"
    assert_close_rel(mp[:500], ref["maxprob"], f"tie rows maxprob mode {mode}")


@pytest.mark.parametrize("mode", [2, 4])
def test_large_batch_argmax_matches_oracle(orc, rh, mode):
    from test_gpu_random_shapes import _head
    rng = np.random.default_rng(31 + mode)
    n, m = 4000, 12000
    q, s, bias = _head(orc, rng, n, K)
    a = rng.standard_normal((m, K)).astype(np.float32)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    try:
        idx, mp = head.argmax(a, mode)
    finally:
        head.close()
    ref = orc.rechead_lines(a, split_lines(m), q, s, bias)
    lg = f64_logits_q(a, q, s, bias)
    check_argmax(idx, ref["idx"], top2_gap(lg), label=f"large batch mode {mode}")
    assert_close_rel(mp, ref["maxprob"], f"large batch maxprob mode {mode}", row_scale=rel_scale(lg))


# Ties inside one vocabulary chunk of the small-batch kernel (a single line to 512 rows of
# the 18710-class head: chunks of 10 tiles): across neighbouring tiles, the first class in
# the earlier tile or in the later tile's neighbour, two tiles apart, inside one tile, and
# across two chunks (the merge's choice).
GROUPS_SETS = [
    ((40, 10), (0, 24)),           # tiles 1 and 0 of chunk 0
    ((70, 50), (24, 48)),          # tiles 2 and 1
    ((72, 20), (48, 72)),          # tiles 2 and 0
    ((101, 100, 96), (72, 96)),    # tile 3
    ((1610, 1590), (96, 120)),     # tiles 50 and 49: chunks 5 and 4
]


@pytest.mark.parametrize("m", [120, 480])
@pytest.mark.parametrize("mode", [2, 4])
def test_exact_ties_across_tiles_of_a_chunk(orc, rh, mode, m):
    from ppocr_rechead import workloads as wl
    w, bias = wl.weights()
    w, bias = w.copy(), bias.copy()
    for classes, (k0, k1) in GROUPS_SETS:
        row = np.zeros(K, np.float32)
        row[k0:k1] = 0.5
        for c in classes:
            w[c] = row
            bias[c] = 0.0
    q, s = orc.pack_int8(w)
    rng = np.random.default_rng(8)
    a = (rng.standard_normal((m, K)) * 0.3).astype(np.float32)
    group = np.arange(m) % len(GROUPS_SETS)
    for g, (_, (k0, k1)) in enumerate(GROUPS_SETS):
        a[group == g, k0:k1] += 2.0
    expect = np.array([min(GROUPS_SETS[g][0]) for g in group], np.int32)
    print(f"ties across tiles of a chunk: mode {mode}, {m} rows", flush=True)
    head = rh.RecHead(qw=rh.QuantizedWeight(q, s), bias=bias)
    try:
        idx, mp = head.argmax(a, mode)
        bad = np.nonzero(idx != expect)[0]
        assert bad.size == 0, f"mode {mode}: {bad.size} rows off the first tied class, e.g. rows {bad[:5]} " \
                              f"got {idx[bad[:5]]} expected {expect[bad[:5]]}"
        off = split_lines(m, 120)
        dec = head.decode(a, off, mode)
        assert np.array_equal(dec["idx"], idx) and np.array_equal(dec["maxprob"], mp)
    finally:
        head.close()
    ref = orc.rechead_lines(a, split_lines(m, 120), q, s, bias)
    assert np.array_equal(ref["idx"], expect), "the oracle's first occurrence"
    assert_close_rel(mp, ref["maxprob"], f"tie rows maxprob mode {mode}", row_scale=rel_scale(f64_logits_q(a, q, s, bias)))
