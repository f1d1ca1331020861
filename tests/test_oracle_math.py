"""Pin the oracle by what the mathematics fixes: exact rational forms, closed forms, invariants, brute force, and an
independent second restatement (the scalar C oracle) on random graphs.

requant(acc, M, s) = clamp(floor(acc M / 2^s + 1/2))          (round half up of the exact quotient)
softmax p_j        = floor(e_j one / S + 1/2)                  (round half up of the exact share)
rsqrt_index(ss, n) = (i, k) with i 4^k <= ss < (i + 1) 4^k, i < n, and i >= n / 4 whenever k > 0
"""
from fractions import Fraction

import numpy as np
import pytest

import helpers
from anvil_mi355x import models
from anvil_mi355x import quantize as Q
from oracle import interp
from oracle import semantics as sem

RNG = np.random.default_rng(2024)


def _clamp(v, lo=-128, hi=127):
    return max(lo, min(hi, v))


def test_requant_is_round_half_up_of_the_exact_quotient():
    for _ in range(3000):
        s = int(RNG.integers(0, 32))
        acc = int(RNG.integers(-(1 << 20), 1 << 20))
        m = int(RNG.integers(-(1 << 10), 1 << 10))
        try:
            got = int(sem.requant(np.array([acc]), m, s)[0])
        except OverflowError:
            assert not -(1 << 31) <= acc * m + (1 << (s - 1) if s else 0) <= (1 << 31) - 1 or \
                not -(1 << 31) <= acc * m <= (1 << 31) - 1
            continue
        want = _clamp(int(np.floor(Fraction(acc * m, 1 << s) + Fraction(1, 2))))
        assert got == want, (acc, m, s)


def test_matmul_brute_force_and_fast_path():
    for (m, k, n) in [(1, 1, 1), (3, 7, 5), (8, 33, 4), (2, 300, 3)]:
        a, b = RNG.integers(-128, 128, (m, k)), RNG.integers(-128, 128, (k, n))
        brute = np.array([[sum(int(a[i, t]) * int(b[t, j]) for t in range(k)) for j in range(n)] for i in range(m)])
        assert np.array_equal(sem.matmul_i8(a, b), brute)
        assert np.array_equal(sem.matmul_i8(a, b, fast=True), brute)
    a, b = np.full((2, 4096), -128), np.full((4096, 2), -128)
    assert np.array_equal(sem.matmul_i8(a, b, fast=True), np.full((2, 2), 4096 * 16384))
    with pytest.raises(ValueError):
        sem.matmul_i8(np.array([[128]]), np.array([[1]]))


def test_softmax_is_round_half_up_of_the_exact_share():
    lut = Q.exp_table(0.07, 40)
    for causal in (False, True):
        x = RNG.integers(-128, 128, (3, 40, 40))
        p = sem.softmax_lut(x, lut, 127, causal)
        for b in range(3):
            for i in range(40):
                kept = i + 1 if causal else 40
                row = x[b, i, :kept]
                m = max(-128, int(row.max()))
                e = [int(lut[v - m + 255]) for v in row]
                S = sum(e)
                want = [int(np.floor(Fraction(ej * 127, S) + Fraction(1, 2))) for ej in e]
                assert list(p[b, i, :kept]) == want
                assert not p[b, i, kept:].any()


def test_softmax_closed_forms_and_mask():
    lut = Q.exp_table(0.05, 16)
    E = int(lut[255])
    for n in range(1, 17):                       # a constant row of n kept entries: round half up of one / n
        p = sem.softmax_lut(np.full((1, n), 7), lut, 127, False)
        assert (p == int(np.floor(Fraction(127, n) + Fraction(1, 2)))).all()
    onehot = np.full((1, 16), -128)
    onehot[0, 5] = 127
    sharp = Q.exp_table(0.2, 16)                   # exp(-51) 2^23 rounds to 0: only the maximum survives
    assert sharp[0] == 0
    p = sem.softmax_lut(onehot, sharp, 127, False)
    assert p[0, 5] == 127 and p.sum() == 127
    x = RNG.integers(-128, 128, (16, 16))        # a causal row equals the unmasked softmax of its kept prefix
    pc = sem.softmax_lut(x, lut, 127, True)
    for i in range(16):
        assert np.array_equal(pc[i, :i + 1], sem.softmax_lut(x[i:i + 1, :i + 1], lut, 127, False)[0])
    perm = RNG.permutation(16)                   # unmasked softmax commutes with a column permutation
    assert np.array_equal(sem.softmax_lut(x[:, perm], lut, 127, False), sem.softmax_lut(x, lut, 127, False)[:, perm])
    assert E > 0


def test_rsqrt_index_characterisation():
    for n in (64, 256, 1024):
        ss = np.concatenate([np.arange(0, 5000), RNG.integers(0, 1 << 31, 5000)])
        i, k = sem.rsqrt_index(ss, n)
        four_k = 4 ** k.astype(object)
        assert ((i * four_k <= ss.astype(object)) & (ss.astype(object) < (i + 1) * four_k)).all()
        assert (i < n).all() and ((k == 0) | (i >= n // 4)).all()


def test_rmsnorm_rational_form():
    d = 48
    w = RNG.integers(-127, 128, d)
    lut, s = Q.rsqrt_table(0.02, 0.01, 0.03, int(np.abs(w).max()), d, 1e-5)
    x = np.concatenate([RNG.integers(-128, 128, (20, d)), np.zeros((1, d), int), np.full((1, d), -128)])
    out = sem.rmsnorm_int(x, w, lut, 1, s)
    assert not out[20].any()                     # a zero row sums to 0 and maps to lut[0] = 0
    for r in range(len(x)):
        ss = int((x[r] ** 2).sum())
        i, k = int(sem.rsqrt_index(ss, len(lut))[0]), int(sem.rsqrt_index(ss, len(lut))[1])
        want = [_clamp(int(np.floor(Fraction(int(x[r, j]) * int(w[j]) * int(lut[i]), 1 << (s + k)) + Fraction(1, 2))))
                for j in range(d)]
        assert list(out[r]) == want


def test_lut_ops_brute_force():
    t = RNG.integers(-128, 128, 256)
    x, y = RNG.integers(-128, 128, 500), RNG.integers(-128, 128, 500)
    assert list(sem.lut_i8(x, t)) == [int(t[v + 128]) for v in x]
    got = sem.swiglu_lut(x, y, t, 300, 12)
    assert list(got) == [_clamp(int(np.floor(Fraction(int(t[a + 128]) * int(b) * 300, 1 << 12) + Fraction(1, 2))))
                         for a, b in zip(x, y)]


@pytest.mark.parametrize("seed", range(24))
def test_numpy_and_scalar_c_oracles_agree(seed):
    m, c, x, want = helpers.random_case(seed)
    got = helpers.scalar_run(m, x, c)
    for k, v in want.values.items():
        assert np.array_equal(got[k], v), k


def test_oracles_agree_on_config1_and_batch_equals_per_sample():
    built, _ = models.config(1)
    x = models.eval_inputs(built.spec, 4, 11)
    xq = np.clip(np.rint(x.astype(np.float64) / built.scales["x"]), -128, 127).astype(np.int64)
    batched = interp.run(built.module, {"x": xq}, built.consts, batch=True)
    scalar = helpers.scalar_run(built.module, {"x": xq}, built.consts, batch=True)
    for k, v in batched.values.items():
        assert np.array_equal(scalar[k], v), k
    for i in range(4):
        one = interp.run(built.module, {"x": xq[i]}, built.consts)
        for k, v in one.values.items():
            assert np.array_equal(v, batched.values[k] if k in built.consts else batched.values[k][i]), k


def test_fast_matmul_path_equals_literal_path_on_a_block():
    built, _ = models.config(1)
    xq = RNG.integers(-128, 128, (2, 32, 64))
    a = interp.run(built.module, {"x": xq}, built.consts, batch=True)
    b = interp.run(built.module, {"x": xq}, built.consts, batch=True, fast=True)
    assert all(np.array_equal(a.values[k], b.values[k]) for k in a.values)


_SOFTMAX, _MATMUL = sem.softmax_lut, sem.matmul_i8


def _softmax_wrong_mask(x, lut, one, causal):
    """The oracle's softmax with the causal mask off by one (keeps j < i instead of j <= i, i > 0)."""
    x = np.asarray(x)
    if not causal:
        return _SOFTMAX(x, lut, one, False)
    out = np.zeros(x.shape, dtype=np.int64)
    t1 = x.shape[-2]
    for i in range(t1):
        kept = max(i, 1)
        out[..., i, :kept] = _SOFTMAX(x[..., i:i + 1, :kept], lut, one, False)[..., 0, :]
    return out


def _matmul_transposed(a, b, fast=False):
    """The oracle's matmul reading its right operand transposed."""
    return _MATMUL(a, np.asarray(b).T if np.asarray(b).shape[0] == np.asarray(b).shape[1] else b, fast)


@pytest.mark.parametrize("plant", ["mask", "transpose"])
def test_planted_oracle_mistakes_fail_the_pins(monkeypatch, plant):
    """A wrong causal mask or a transposed matmul operand planted in the oracle makes the pins above fail."""
    if plant == "mask":
        monkeypatch.setattr(sem, "softmax_lut", _softmax_wrong_mask)
        with pytest.raises(AssertionError):
            test_softmax_closed_forms_and_mask()
    else:
        monkeypatch.setattr(sem, "matmul_i8", _matmul_transposed)
        with pytest.raises(AssertionError):
            a, b = RNG.integers(-128, 128, (4, 4)), RNG.integers(-128, 128, (4, 4))
            brute = np.array([[sum(int(a[i, t]) * int(b[t, j]) for t in range(4)) for j in range(4)]
                              for i in range(4)])
            assert np.array_equal(sem.matmul_i8(a, b), brute)
