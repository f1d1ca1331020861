"""Pin the wide (i16) rmsnorm of the oracle (reference anvil/semantics.py:158-182, ADR-004) by its rational form, and
restate the reference's adversarial-row bound test (tests/lower/test_wide_residual.py:45-66).

For an i16 row x of d entries with square shift c, sum offset e, table lut (n entries), multiplier M and shift s:
    ss    = e + sum_j floor((x_j^2 + 2^(c-1)) / 2^c)                 (each square rounded half up at 2^c)
    (i,k) : i 4^k <= ss < (i + 1) 4^k, i < n, k minimal              (the table index after k steps of /4)
    out_j = clamp_i8(floor(x_j w_j lut[i] M / 2^(s+k) + 1/2))
The rational form is evaluated with Python integers and Fractions: no shift, no rsqrt_index call, no numpy int64.
"""
from fractions import Fraction

import numpy as np
import pytest

from anvil_mi355x import quantize as Q
from oracle import semantics as sem

RNG = np.random.default_rng(4242)
I16 = (-(1 << 15), (1 << 15) - 1)


def _rational_row(x, w, lut, M, s, c, e):
    n = len(lut)
    ss = e + sum(int(np.floor(Fraction(int(v) * int(v) + (1 << c >> 1), 1 << c))) for v in x)
    k = 0
    while not ss < n * 4 ** k:
        k += 1
    i = ss // 4 ** k
    assert i * 4 ** k <= ss < (i + 1) * 4 ** k
    return [max(-128, min(127, int(np.floor(Fraction(int(xj) * int(wj) * int(lut[i]) * M, 1 << (s + k))
                                             + Fraction(1, 2))))) for xj, wj in zip(x, w)]


def _wide_rows(d, count):
    rows = [RNG.integers(I16[0], I16[1] + 1, d) for _ in range(count)]
    for mag in (0, 1, 7, 300, 5000, I16[1]):                          # quiet, tiny, loud and saturated rows
        rows.append(np.full(d, mag))
        rows.append(np.r_[-mag if mag else 0, RNG.integers(-3, 4, d - 1)])
    rows.append(np.full(d, I16[0]))
    return np.array(rows)


@pytest.mark.parametrize("d,sx", [(32, 4e-4), (96, 2e-4), (7, 1e-3)])
def test_wide_rmsnorm_rational_form(d, sx):
    w = RNG.integers(-127, 128, d)
    lut, s, c, e = Q.wide_rsqrt_table(sx, 0.01, 0.02, 127, d, 1e-6, 1 << 15)
    assert c > 0 and e > 0                       # the wide path proper: shifted squares and a folded eps
    x = _wide_rows(d, 30)
    got = sem.rmsnorm_wide(x, w, lut, 1, s, c, e, "i16")
    for r in range(len(x)):
        assert list(got[r]) == _rational_row(x[r], w, lut, 1, s, c, e), r


def test_wide_rmsnorm_rational_form_with_a_multiplier():
    """M != 1 and a hand-made table: c = 5, e = 37, s = 9 on rows whose sums cross several k."""
    d, n = 16, 64
    lut = np.r_[0, RNG.integers(100, 20000, n - 1)]
    w = RNG.integers(-127, 128, d)
    x = _wide_rows(d, 40)
    got = sem.rmsnorm_wide(x // 128, w, lut, 3, 9, 5, 37, "i16")
    for r in range(len(x)):
        assert list(got[r]) == _rational_row(x[r] // 128, w, lut, 3, 9, 5, 37), r


def test_planted_wide_mistakes_fail_the_rational_form(monkeypatch):
    """A square shift that drops its rounding term, or an oracle that forgets ss_init, disagrees with the rational
    form on these rows: the pin is sharp enough to catch either."""
    d = 32
    w = RNG.integers(-127, 128, d)
    lut, s, c, e = Q.wide_rsqrt_table(4e-4, 0.01, 0.02, 127, d, 1e-6, 1 << 15)
    x = _wide_rows(d, 30)
    want = [_rational_row(x[r], w, lut, 1, s, c, e) for r in range(len(x))]
    monkeypatch.setattr(sem, "sq_shift", lambda v, cc: sem.check_i32(v * v, "x*x") >> int(cc))
    assert any(list(row) != wr for row, wr in zip(sem.rmsnorm_wide(x, w, lut, 1, s, c, e, "i16"), want))
    monkeypatch.undo()
    assert any(list(row) != wr for row, wr in zip(sem.rmsnorm_wide(x, w, lut, 1, s, c, 0, "i16"), want))


def test_wide_bound_holds_on_adversarial_rows():
    """Reference tests/lower/test_wide_residual.py:45-66: every x * w * r (+ round) the wide rmsnorm forms stays within
    the bound the quantizer proves, on rows built to maximise it (one loud entry, all entries equal, one loud entry
    over ones) at every magnitude from 1 to 2^15; each row's loudest entry is within WideRow's xmax."""
    D = 32
    lut, s, c, e = Q.wide_rsqrt_table(4e-4, 0.01, 0.02, 127, D, 1e-6, 1 << 15)
    row = Q.WideRow(D, len(lut), c, 1 << 15, e)
    bound = row.numerators(lut, 127, 1, s)
    assert max(bound.values()) <= Q.INT32_MAX and s + row.kmax <= 31
    rows = []
    for mag in np.unique(np.geomspace(1, 1 << 15, 200).astype(np.int64)):
        loud = min(int(mag), I16[1] + 1)
        one = np.zeros(D, np.int64)
        one[0] = loud
        rows += [one, -one, np.full(D, loud), np.r_[loud, np.ones(D - 1, np.int64)]]
    x = np.clip(np.array(rows), I16[0], I16[1])
    ss = sem.sq_shift(x, c).sum(axis=1) + e
    idx, k = sem.rsqrt_index(ss, len(lut))
    xwr = np.abs(x * 127) * lut[idx][:, None]
    for kv in np.unique(k):
        assert (xwr[k == kv] + sem.round_term(s + int(kv))).max() <= bound[int(kv)]
        assert (np.abs(x[k == kv]).max(axis=1) <= row.xmax[int(kv)][idx[k == kv]]).all()
    out = sem.rmsnorm_wide(x, np.full(D, 127), lut, 1, s, c, e, "i16")      # raises on any int32 overflow
    assert np.abs(out).max() <= 128
