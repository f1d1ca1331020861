"""Host checks of the integer identities the HIP kernels rely on, evaluated exactly on the CPU.

The fused attention kernel (csrc/attention.hip) divides p = (e one + S // 2) // S in float64 as
y = fma(e, A, B - 1/2) with A = fl(one / S) and B = fl(fl((S // 2) / S) + 2^-40), then takes the low dword of
fl(y + 1.5 2^52), i.e. y rounded to the nearest integer: floor(y + 1/2). Here fma is emulated exactly (the exact
rational e A + B' rounded once to the nearest double, which Python's float(Fraction) does), the addition is an IEEE
double addition, and the result is compared with integer floor division on the cases where a floating-point quotient
is most fragile: exact multiples n = k S and their neighbours, the largest divisors, and random draws.

The GEMM epilogues' fused add on byte multiplies (PackedAdd) and their widened LUT index are checked at the end of
the file, on every int8 operand pair and on int32 values at both ends of the range, and so is the closed form of the
rsqrt table index that the fused rmsnorm epilogue uses in place of the reference's shift loop. Last, the embedding
quantization's rounding of x / scale through a multiply by 1 / scale, guarded near the half-integers.
"""
import struct
from fractions import Fraction

import numpy as np
import pytest


def fdiv(a, b):
    return a / b                                  # IEEE double division, correctly rounded


MAGIC = 1.5 * 2.0 ** 52


def low_dword(x):
    """The low 32 bits of a double's bit pattern, as a signed int."""
    lo = struct.unpack("<Q", struct.pack("<d", x))[0] & 0xFFFFFFFF
    return lo - (1 << 32) if lo >= 1 << 31 else lo


def kernel_quot(e, one, S, eps=2.0 ** -40):
    A = fdiv(float(one), float(S))
    B = fdiv(float(S >> 1), float(S)) + eps - 0.5         # as the kernel: the - 0.5 is exact
    y = float(Fraction(e) * Fraction(A) + Fraction(B))   # fma: one rounding of the exact value
    return low_dword(y + MAGIC)                           # rounded to nearest, read from the mantissa


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


def in_domain(e, one, S):
    """The kernel divides only quotients below 128: S sums the row's exp values, this key's own included, so
    e <= S and n // S <= one <= 127 (the error bound assumes |y| < 128)."""
    return (e * one + (S >> 1)) // S < 128


def test_float64_division_is_exact_floor_division():
    todo = [c for c in cases() + NEEDS_EPSILON if in_domain(*c)]
    assert len(todo) > 500
    bad = [(e, one, S) for e, one, S in todo if kernel_quot(e, one, S) != (e * one + (S >> 1)) // S]
    assert not bad, bad[:5]


def test_the_epsilon_term_is_needed():
    """Dropping the 2^-40 term rounds an exact quotient k to k - 1: the cases above pin it."""
    for e, one, S in NEEDS_EPSILON:
        assert kernel_quot(e, one, S, eps=0.0) == (e * one + (S >> 1)) // S - 1


def test_the_rounding_constant_reads_back_small_integers():
    """fl(y + 1.5 2^52) holds round(y) in its low dword for y in (-1/2, 128), the kernel's range (never a tie)."""
    for k in range(128):
        for y in (k - 0.499, k - 0.25, float(k), k + 0.25, k + 0.499):
            if y > -0.5:
                assert low_dword(y + MAGIC) == round(y), y


@pytest.mark.parametrize("S", [1, 2, 5, 1 << 16, (1 << 31) - 1])
def test_every_quotient_of_a_small_range(S):
    one = 127
    h = S >> 1
    top = min(((1 << 31) - 1 - h) // one, 4000)
    for e in range(top + 1):
        if in_domain(e, one, S):
            assert kernel_quot(e, one, S) == (e * one + h) // S, (e, S)


# ---------------------------------------------------------------------------------------------------------------
# The GEMM epilogues' byte-multiply add and widened LUT index (csrc/common.h PackedAdd, csrc/gemm.hip plain_epilogue),
# emulated with the hardware's operations: a 24 x 24 -> 32-bit unsigned multiply of a byte, and 32-bit wrapping adds.

M32 = (1 << 32) - 1


def packed_add_sum(r, y, m, n, rnd):
    """r * m + y * n + rnd as the kernel forms it: u * |m| + v * |n| + c modulo 2^32, read as int32; u is the byte of
    r ^ 0x80 (m >= 0) or r ^ 0x7F (m < 0), likewise v for y."""
    def term(x, mult):
        u = (x & 0xFF) ^ (0x80 if mult >= 0 else 0x7F)
        assert 0 <= u <= 255 and abs(mult) < 1 << 24
        return (u * abs(mult)) & M32, ((-128 * mult) if mult >= 0 else (127 * mult)) & M32
    tr, cr = term(r, m)
    ty, cy = term(y, n)
    s = (tr + ty + ((rnd + cr + cy) & M32)) & M32
    return s - (1 << 32) if s >= 1 << 31 else s


@pytest.mark.parametrize("m,n", [(0, 0), (1, 1), (300, -200), (11157253, 4299753), (-12000000, 4000000),
                                 (16000000, -700000), (-8388608, -8000000), ((1 << 24) - 1, 0), (-(1 << 24) + 1, 0),
                                 (1 << 23, -(1 << 23)), (-1, 1)])
def test_packed_add_is_the_add_inside_int32(m, n):
    """Every pair of int8 operands: the byte-multiply form equals r m + y n + rnd whenever that lies inside int32 (the
    add's proof); planted: the 127 correction of a negative multiplier replaced by 128 fails."""
    r = np.arange(-128, 128, dtype=np.int64)[:, None]
    y = np.arange(-128, 128, dtype=np.int64)[None, :]
    rnd = 1 << 23
    want = r * m + y * n + rnd
    inside = (want >= -(1 << 31)) & (want < 1 << 31)
    got = np.vectorize(lambda a, b: packed_add_sum(int(a), int(b), m, n, rnd))(r, y)
    assert np.array_equal(got[inside], want[inside])
    if m < 0:   # a plausible slip: the same correction for both signs
        bad = np.vectorize(lambda a, b: (((a & 0xFF) ^ 0x7F) * -m - 128 * m + b * n + rnd))(r, y)
        assert not np.array_equal(bad[inside], want[inside])


def wide_lut_index(x, s):
    """(x + 2^31) >> s, unsigned, with x + 2^31 formed modulo 2^32 (the kernel adds 2^31 through the rounding
    constant)."""
    return ((x + (1 << 31)) & M32) >> s


@pytest.mark.parametrize("s", [1, 2, 12, 16, 17, 18, 24, 30, 31])
def test_wide_lut_index_is_the_shift_plus_an_offset(s):
    """For every int32 x, (x + 2^31) >> s (unsigned) equals floor(x / 2^s) + 2^(31 - s), in [0, 2^(32 - s)): the
    widened table's entry u = lut[clamp(u - 2^(31 - s), -128, 127) + 128] is then the clamped requant's LUT value."""
    rng = np.random.default_rng(s)
    x = np.concatenate([np.arange(-(1 << 31), -(1 << 31) + 4096), np.arange(-4096, 4096),
                        np.arange((1 << 31) - 4096, 1 << 31), rng.integers(-(1 << 31), 1 << 31, 100000)])
    x = x.astype(np.int64)
    u = wide_lut_index(x, s)
    assert np.array_equal(u, (x >> s) + (1 << (31 - s)))
    assert u.min() >= 0 and u.max() < 1 << (32 - s)
    lut = np.random.default_rng(1).integers(-128, 128, 256)
    table = lut[np.clip(np.arange(1 << (32 - s)) - (1 << (31 - s)), -128, 127) + 128] if s >= 12 else None
    if table is not None:
        assert np.array_equal(table[u], lut[np.clip(x >> s, -128, 127) + 128])


def rsqrt_index_closed(ss, n):
    """The fused rmsnorm epilogue's (idx, k) (csrc/gemm.hip norm_chunk): with b and c the bit lengths of ss and n,
    k = k0 or k0 + 1, k0 = max(0, floor((b - c + 1) / 2)), whichever first brings ss >> 2k below n."""
    b = int(ss).bit_length()
    c = int(n).bit_length()
    k0 = max(0, (b - c + 1) >> 1)
    k = k0 + (1 if (ss >> (2 * k0)) >= n else 0)
    return ss >> (2 * k), k


@pytest.mark.parametrize("n", [1, 2, 3, 5, 255, 256, 257, 1000, 1023, 1024, 1025, 4096, 12345])
def test_rsqrt_index_closed_form(n):
    """The closed form equals the reference loop (shift right by 2 until below n) for sums of squares across the
    int32 range: every value up to 2^16, powers of two and their neighbours, and random draws."""
    from oracle import semantics as sem
    rng = np.random.default_rng(n)
    ss = np.unique(np.concatenate([np.arange(1 << 16), [(1 << p) + d for p in range(31) for d in (-1, 0, 1)],
                                   rng.integers(0, (1 << 31) - 1, 20000)]))
    ss = ss[(ss >= 0) & (ss < 1 << 31)]
    idx, k = sem.rsqrt_index(ss, n)
    got = np.array([rsqrt_index_closed(int(v), n) for v in ss])
    assert np.array_equal(got[:, 0], idx) and np.array_equal(got[:, 1], k)


# ---------------------------------------------------------------------------------------------------------------
# embed_quantize_vec4 (csrc/eltwise.hip): rint(x / scale) taken as rint(fl(x fl(1 / scale))) unless that product lies
# within 2^-50 of its magnitude of a half-integer, or 1 / scale is not a normal double; then the quotient itself.
# Every operation is an IEEE double operation, the same on the host as on the GPU.

def embed_rint(x, s):
    inv = 1.0 / s
    use = np.isfinite(inv) and abs(inv) >= np.finfo(np.float64).tiny
    with np.errstate(invalid="ignore", over="ignore"):
        q = x * inv
        v = np.rint(q)
        exact = ~(use & (np.abs(q - np.floor(q) - 0.5) > 2.0 ** -50 * np.abs(q)))
        v[exact] = np.rint(x[exact] / s)
    return v, exact


def near_ties(s, rng):
    """Products of s with every half-integer in [-300.5, 300.5], each with its two neighbours either side, and
    random multiples of s."""
    base = (np.arange(-300, 301) + 0.5) * s
    up, down = np.nextafter(base, np.inf), np.nextafter(base, -np.inf)
    return np.concatenate([base, up, down, np.nextafter(up, np.inf), np.nextafter(down, -np.inf),
                           rng.standard_normal(500) * s * 100])


def test_embed_rint_equals_the_quotient_rint():
    """On inputs crowded at the half-integers (where rint changes value) and at random, over scales from 1e-7 to 20,
    the guarded product rounds as the correctly rounded quotient does; planted: without the guard it does not."""
    rng = np.random.default_rng(5)
    unguarded = 0
    for _ in range(60):
        s = float(10.0 ** rng.uniform(-7, 1)) * rng.uniform(1, 2)
        x = near_ties(s, rng)
        want = np.rint(x / s)
        got, _ = embed_rint(x, s)
        assert np.array_equal(got, want), s
        unguarded += int((np.rint(x * (1.0 / s)) != want).sum())
    assert unguarded > 0


def test_embed_rint_takes_the_quotient_where_the_product_cannot_serve():
    """A subnormal scale (1 / scale infinite), infinite and NaN inputs, and ties at a power-of-two scale (exact product,
    ties to even on both paths)."""
    x = np.array([0.0, 1e-300, -2.5e-300, np.inf, -np.inf, np.nan, 3.0])
    got, exact = embed_rint(x, 5e-310)
    assert exact.all()
    with np.errstate(over="ignore"):
        want = np.rint(x / 5e-310)
    assert np.array_equal(got, want, equal_nan=True)
    got, exact = embed_rint(np.array([np.inf, np.nan, 1.0]), 0.25)
    assert exact[:2].all() and got[2] == 4.0
    s = 2.0 ** -12
    x = (np.arange(-20, 21) + 0.5) * s
    got, _ = embed_rint(x, s)
    assert np.array_equal(got, np.rint(x / s)) and np.array_equal(got % 2, np.zeros_like(got))
