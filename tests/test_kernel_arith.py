"""Host checks of the integer identities the HIP kernels rely on, evaluated exactly on the CPU.

The fused attention kernel (csrc/attention.hip) divides p = (e one + S // 2) // S as trunc(fma(e, A, B)) in float64
with A = fl(one / S) and B = fl(fl((S // 2) / S) + 2^-40). Here fma is emulated exactly (the exact rational e A + B
rounded once to the nearest double, which Python's float(Fraction) does) and compared with integer floor division on
the cases where a floating-point quotient is most fragile: exact multiples n = k S and their neighbours, the largest
divisors, and random draws.
"""
from fractions import Fraction

import numpy as np
import pytest


def fdiv(a, b):
    return a / b                                  # IEEE double division, correctly rounded


def kernel_quot(e, one, S):
    A = fdiv(float(one), float(S))
    B = fdiv(float(S >> 1), float(S)) + 2.0 ** -40
    y = float(Fraction(e) * Fraction(A) + Fraction(B))   # fma: one rounding of the exact value
    return int(y)                                         # truncation toward zero


def cases():
    rng = np.random.default_rng(77)
    out = []
    for S in [1, 2, 3, 7, 255, 256, 1 << 20, (1 << 23) + 1, (1 << 30) - 1, (1 << 31) - 1, 1000003, 123456789]:
        for one in (1, 3, 100, 127):
            h = S >> 1
            emax = ((1 << 31) - 1 - h) // one            # n = e one + h < 2^31, as the overflow proof guarantees
            for k in range(0, 128, 7):
                for delta in (-1, 0, 1):                 # e one + h near k S
                    target = k * S + delta - h
                    if target < 0:
                        continue
                    e = min(target // one, emax)
                    if e * one + h < (1 << 31):
                        out.append((e, one, S))
            for e in rng.integers(0, emax + 1, 20):
                out.append((int(e), one, S))
    return out


# exact quotients n = k S whose float64 estimate rounds just below k without the 2^-40 term (found by search)
NEEDS_EPSILON = [(344077939, 2, 458770585), (334444885, 3, 668889770), (335528144, 5, 479325920),
                 (18999029, 28, 151992232)]


def test_float64_division_is_exact_floor_division():
    bad = [(e, one, S) for e, one, S in cases() + NEEDS_EPSILON
           if kernel_quot(e, one, S) != (e * one + (S >> 1)) // S]
    assert not bad, bad[:5]


def test_the_epsilon_term_is_needed():
    """Dropping the 2^-40 term truncates an exact quotient k to k - 1: the cases above pin it."""
    for e, one, S in NEEDS_EPSILON:
        A, B = float(one) / float(S), float(S >> 1) / float(S)
        assert int(float(Fraction(e) * Fraction(A) + Fraction(B))) == (e * one + (S >> 1)) // S - 1


@pytest.mark.parametrize("S", [1, 2, 5, 1 << 16, (1 << 31) - 1])
def test_every_quotient_of_a_small_range(S):
    one = 127
    h = S >> 1
    top = min(((1 << 31) - 1 - h) // one, 4000)
    for e in range(top + 1):
        assert kernel_quot(e, one, S) == (e * one + h) // S, (e, S)
