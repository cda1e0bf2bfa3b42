"""Pins the oracle's INT8 packer (QuantizedWeight::from_f32_transposed,
src/ops/matmul.rs:1173-1202) against closed forms, hand-derived known answers, exact
rational arithmetic and an independent numpy restatement."""
import os
from fractions import Fraction

import numpy as np
import pytest

from conftest import REFERENCE, reference_available
from packref import pack_numpy


def test_random_rows_match_numpy_restatement(orc):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((2000, 120), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    q, s = orc.pack_int8(w)
    qn, sn = pack_numpy(w)
    assert np.array_equal(q, qn)
    assert np.array_equal(s.view(np.uint32), sn.view(np.uint32))


def test_half_way_values_round_away_from_zero(orc):
    # max |w| = 127 -> scale = 1, inv = 1: q is round(w) with ties away from zero.
    row = np.array([127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -0.49999997], np.float32)
    q, s = orc.pack_int8(row[None, :])
    assert s[0] == 1.0
    assert q[0].tolist() == [127, 3, -3, 1, -1, 2, -2, 127, 0]  # rint would give 2, -2, 0, 0, 2, -2, 126


def test_scale_rule_and_special_rows(orc):
    rows = np.zeros((6, 16), np.float32)
    rows[1, :] = 5e-9                      # max_abs <= 1e-8 -> scale 1.0, q = round(5e-9) = 0
    rows[2, 3] = 5.0                       # single outlier -> q = 127 there
    rows[3, 7] = -5.0
    rows[3, 0] = 0.01
    rows[4, :] = np.float32(1e-8)          # exactly 1e-8 is not > 1e-8
    rows[5, 0] = np.nan                    # NaN ignored by the max and packed as 0
    rows[5, 1] = 0.5
    q, s = orc.pack_int8(rows)
    assert s[0] == 1.0 and not q[0].any()
    assert s[1] == 1.0 and not q[1].any()
    assert s[2] == np.float32(5.0) / np.float32(127.0) and q[2, 3] == 127 and q[2].sum() == 127
    assert q[3, 7] == -127
    # 0.01 / (5/127) = 0.254 -> 0
    assert q[3, 0] == 0
    assert s[4] == 1.0 and not q[4].any()
    assert q[5, 0] == 0 and q[5, 1] == 127 and s[5] == np.float32(0.5) / np.float32(127.0)


def test_infinite_row_packs_to_zero(orc):
    row = np.array([[np.inf, 1.0, -2.0, 0.0]], np.float32)
    q, s = orc.pack_int8(row)
    # scale = inf/127 = inf, inv = 0, inf*0 = NaN -> 0, finite*0 = 0
    assert np.isinf(s[0]) and not q.any()


def _exact_round_half_away(fr):
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    fl = a.numerator // a.denominator
    return sign * (fl + 1 if a - fl >= Fraction(1, 2) else fl)


def test_multiplies_by_the_rounded_reciprocal(orc):
    """q is round(f32(w * f32(1/scale))), not round(w / scale).  Construct elements whose
    f32 product lands on a half-way point while the exact quotient does not (or the other
    way round) and check the oracle against exact rational arithmetic of the reference rule."""
    rows, expect_rows = [], []
    for max_abs in (np.float32(0.1538154), np.float32(0.123), np.float32(5.0), np.float32(0.0731)):
        scale = np.float32(max_abs / np.float32(127))
        inv = np.float32(np.float32(1) / scale)
        for kk in range(0, 127):
            w0 = np.float32((kk + 0.5) / float(inv))
            for d in range(-6, 7):
                w = np.float32(np.nextafter(w0, np.float32(np.inf if d > 0 else -np.inf)) if d else w0)
                for _ in range(abs(d) - 1 if d else 0):
                    w = np.nextafter(w, np.float32(np.inf if d > 0 else -np.inf))
                prod = np.float32(w * inv)
                via_mul = _exact_round_half_away(Fraction(float(prod)))
                via_div = _exact_round_half_away(Fraction(float(w)) / Fraction(float(scale)))
                if via_mul != via_div and abs(via_mul) <= 127:
                    row = np.zeros(8, np.float32)
                    row[0] = max_abs
                    row[1] = w
                    row[2] = -w
                    rows.append(row)
                    expect_rows.append((via_mul, -via_mul))
                    break
            if len(rows) >= 40:
                break
    assert len(rows) >= 4, "no distinguishing element found"
    q, s = orc.pack_int8(np.stack(rows))
    for j, (e1, e2) in enumerate(expect_rows):
        assert q[j, 0] == 127
        assert (q[j, 1], q[j, 2]) == (e1, e2), j


def test_reconstruction_within_half_a_step(orc):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((500, 120), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    q, s = orc.pack_int8(w)
    err = np.abs(q.astype(np.float64) * s[:, None].astype(np.float64) - w.astype(np.float64))
    # |q*s - w| <= s/2 plus the f32 rounding of w * inv (|w*inv| <= 127, one ulp = 2^-17 of it)
    assert np.all(err <= s[:, None] * (0.5 + 127 * 2.0**-23))
    assert np.all(np.abs(q).max(axis=1) == 127)


def test_golden_fixture(orc):
    path = os.path.join(os.path.dirname(__file__), "golden", "pack_rows.npz")
    g = np.load(path)
    for key in ("small_rec", "tiny_rec", "special"):
        q, s = orc.pack_int8(g[f"{key}_w_t"])
        assert np.array_equal(q, g[f"{key}_q"]), key
        assert np.array_equal(s.view(np.uint32), g[f"{key}_scales"].view(np.uint32)), key


@pytest.mark.skipif(not reference_available(), reason="reference model files not mounted")
def test_real_head_weight_and_footprint(orc):
    from safetensors.numpy import load_file
    w = load_file(os.path.join(REFERENCE, "models", "PP-OCRv6_small_rec.safetensors"))["linear_8.w_0"]
    assert w.shape == (120, 18710)
    w_t = np.ascontiguousarray(w.T)  # the transpose prepack, src/engine/model.rs:565-605
    q, s = orc.pack_int8(w_t)
    qn, sn = pack_numpy(w_t)
    assert np.array_equal(q, qn) and np.array_equal(s, sn)
    # weight_footprint_bytes contribution: data.len() + 4 * scales.len() (src/engine/model.rs:661-665)
    assert q.size + 4 * s.size == 2_320_040
    assert 4 * w_t.size == 8_980_800
