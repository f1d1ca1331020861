"""GPU parity per op: each C-ABI entry point against the oracle on the same seeded inputs, bit-exact.

Config 2 (the standalone int8 linear + requant sweep: M in {256, 4096, 16384}, K = N in {768, 3072}, uniform
int8 in [-127, 127]) runs at its full sizes; the edge cases cover odd shapes (the byte-load path), i16 results,
LUT epilogues, negative multipliers, head-batched strided operands and the device-side int32 contract flags.
"""
import re

import numpy as np
import pytest

from anvil_mi355x import quantize as Q
from anvil_mi355x import runtime as rt
from oracle import semantics as sem

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return rt.device(0)


def up(dev, arr, dt):
    return dev.upload(np.ascontiguousarray(np.asarray(arr)).astype(rt.NP_DTYPE[dt]))


def run_gemm(dev, a, w, m, s, lut=None, dtype="i8"):
    """qlinear on the device: a (M, K) @ w (K, N), w uploaded transposed (N, K)."""
    M, K = a.shape
    N = w.shape[1]
    A, Bt = up(dev, a, "i8"), up(dev, w.T, "i8")
    Cb = dev.alloc(M * N * rt.ITEMSIZE[dtype])
    L = None if lut is None else up(dev, lut, "i8")
    dev.gemm_i8(A, Bt, Cb, 1, 1, M, N, K, [0, 0, K, 0, 0, K, 0, 0, N], m, s, L, dtype)
    dev.sync()
    return Cb.download((M, N), rt.NP_DTYPE[dtype]).astype(np.int64)


CONFIG2 = [(M, K) for M in (256, 4096, 16384) for K in (768, 3072)]


@pytest.mark.parametrize("M,K", CONFIG2)
def test_gemm_config2_sweep(dev, M, K):
    rng = np.random.default_rng([2, M, K])
    a = rng.integers(-127, 128, (M, K))
    w = rng.integers(-127, 128, (K, K))
    acc = sem.matmul_i8(a, w, fast=True)
    (m,), s = Q.choose_shift([127 / (1.5 * int(np.abs(acc).max()))], [128 * int(np.abs(w).sum(axis=0).max())])
    want = sem.requant(acc, m, s)
    got = run_gemm(dev, a, w, m, s)
    assert np.array_equal(got, want), (M, K, int((got != want).sum()))
    assert 50 < np.abs(want).max() <= 127          # the requant scale keeps the outputs spread, not saturated


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (7, 5, 3), (33, 17, 65), (130, 48, 257), (255, 100, 129),
                                   (64, 16, 64), (200, 1000, 40)])
@pytest.mark.parametrize("dtype", ["i8", "i16"])
def test_gemm_odd_shapes(dev, M, K, N, dtype):
    rng = np.random.default_rng([3, M, K, N])
    a = rng.integers(-128, 128, (M, K))
    w = rng.integers(-128, 128, (K, N))
    m = int(rng.integers(1, 3000)) * (-1 if N % 2 else 1)
    s = int(rng.integers(8, 20))
    want = sem.qmatmul(a, w, m, s, dtype=dtype)
    assert np.array_equal(run_gemm(dev, a, w, m, s, dtype=dtype), want)


def test_gemm_lut_epilogue(dev):
    rng = np.random.default_rng(4)
    a, w = rng.integers(-128, 128, (300, 96)), rng.integers(-128, 128, (96, 200))
    lut = rng.integers(-128, 128, 256)
    want = sem.qmatmul(a, w, 555, 17, lut)
    assert np.array_equal(run_gemm(dev, a, w, 555, 17, lut), want)


@pytest.mark.parametrize("B,H,T,d", [(2, 3, 40, 16), (3, 2, 130, 32), (1, 4, 64, 64)])
def test_gemm_head_batched_strided(dev, B, H, T, d):
    """scores = qh @ kT read in place from q, k (B, T, H*d): batch strides (T*C, d), row stride C."""
    rng = np.random.default_rng([5, B, H, T, d])
    C = H * d
    q, k = rng.integers(-128, 128, (B, T, C)), rng.integers(-128, 128, (B, T, C))
    qh = q.reshape(B, T, H, d).transpose(0, 2, 1, 3)
    kT = k.reshape(B, T, H, d).transpose(0, 2, 3, 1)
    want = sem.qmatmul(qh, kT, 700, 14)
    Q_, K_ = up(dev, q, "i8"), up(dev, k, "i8")
    out = dev.alloc(B * H * T * T)
    dev.gemm_i8(Q_, K_, out, B, H, T, T, d, [T * C, d, C, T * C, d, C, H * T * T, T * T, T], 700, 14, None, "i8")
    dev.sync()
    assert np.array_equal(out.download((B, H, T, T), np.int8).astype(np.int64), want)


def test_gemm_overflow_flag(dev):
    """acc * M past int32 raises OverflowError, as the reference's checked requant does."""
    a = np.full((4, 8), -128)
    w = np.full((8, 16), 127)
    acc = 128 * 8 * 127
    m_ok = ((1 << 31) - 1 - (1 << 9)) // acc
    assert np.array_equal(run_gemm(dev, a, w, m_ok, 10), sem.qmatmul(a, w, m_ok, 10))
    with pytest.raises(OverflowError):
        sem.qmatmul(a, w, m_ok + 1, 10)
    with pytest.raises(OverflowError):
        run_gemm(dev, a, w, m_ok + 1, 10)
    assert np.array_equal(run_gemm(dev, a, w, m_ok, 10), sem.qmatmul(a, w, m_ok, 10))   # flags were cleared


def _rms(dev, x, xdt, w, lut, m, s, c=0, e=0, flags=0):
    rows, d = x.shape
    out = dev.alloc(rows * d)
    dev.rmsnorm_int(up(dev, x, xdt), xdt, up(dev, w, "i8"), up(dev, lut, "i32"), len(lut), m, s, c, e, rows, d, out,
                    flags)
    dev.sync()
    return out.download((rows, d), np.int8).astype(np.int64)


@pytest.mark.parametrize("flags", [0, rt.OP_UNCHECKED, rt.OP_UNCHECKED | rt.RMS_S24])
@pytest.mark.parametrize("d", [8, 16, 32, 64, 128, 256, 512, 768, 1000, 1024])
def test_rmsnorm_i8(dev, d, flags):
    """flags=UNCHECKED selects the dot4 kernel with four rows a wave where d is a multiple of 16 up to 1024 (the
    proof's bounds hold for m = 1 and these LUTs), RMS_S24 its 24-bit multiply-add (every |lut m| < 2^23 here), on
    16 lanes a row when d is 256, 512, 768 or 1024, 8 lanes a row when d is 128, and 1, 2 or 4 lanes a row with
    per-lane row values when d is 16, 32 or 64; results are the same bits either way."""
    rng = np.random.default_rng([6, d])
    w = rng.integers(-127, 128, d)
    lut, s = Q.rsqrt_table(0.03, 0.01, 0.02, int(np.abs(w).max()), d, 1e-5)
    x = np.concatenate([rng.integers(-128, 128, (200, d)), np.full((1, d), -128), np.zeros((1, d), int),
                        np.full((1, d), 127), np.rint(rng.standard_normal((50, d)) * 3).astype(int)])
    want = sem.rmsnorm_int(x, w, lut, 1, s)
    assert int(np.abs(lut).max()) < (1 << 23)
    assert np.array_equal(_rms(dev, x, "i8", w, lut, 1, s, flags=flags), want)


@pytest.mark.parametrize("flags,d", [(rt.OP_UNCHECKED, 64), (rt.OP_UNCHECKED | rt.RMS_S24, 64),
                                     (rt.OP_UNCHECKED | rt.RMS_S24, 32), (rt.OP_UNCHECKED | rt.RMS_S24, 128),
                                     (rt.OP_UNCHECKED | rt.RMS_S24, 768)])
def test_rmsnorm_fast_walks_many_row_groups(dev, flags, d):
    """More row groups of four than the grid has waves (a cap of eight workgroups of four waves per CU): each wave
    walks several groups through both of its row buffers (three each on MI355X's 256 CUs), and the last group is
    ragged (rows % 4 == 3)."""
    rows = 8 * 4 * 256 * 4 * 3 + 3
    rng = np.random.default_rng([61, rows])
    w = rng.integers(-127, 128, d)
    lut, s = Q.rsqrt_table(0.03, 0.01, 0.02, int(np.abs(w).max()), d, 1e-5)
    x = rng.integers(-128, 128, (rows, d))
    want = sem.rmsnorm_int(x, w, lut, 1, s)
    assert np.array_equal(_rms(dev, x, "i8", w, lut, 1, s, flags=flags), want)


@pytest.mark.parametrize("d", [32, 64, 128, 768])
def test_rmsnorm_shift_reaching_int32_bounds(dev, d):
    """Requant shifts s + k from 20 up to 27: at 24 and above the pre-shift clamp bounds saturate to the int32 limits
    (rows with a large sum of squares take k up to 7 with a 1024-entry LUT)."""
    rng = np.random.default_rng([62, d])
    w = rng.integers(-127, 128, d)
    lut = rng.integers(1, 1 << 14, 1024)
    x = np.concatenate([rng.integers(-128, 128, (61, d)), rng.integers(-3, 4, (60, d)), np.full((2, d), -128)])
    want = sem.rmsnorm_int(x, w, lut, 1, 20)
    got = _rms(dev, x, "i8", w, lut, 1, 20, flags=rt.OP_UNCHECKED | rt.RMS_S24)
    assert np.array_equal(got, want)
    assert np.abs(want).max() > 0


@pytest.mark.parametrize("n", [5, 1000, 1024, 1025, 3000])
@pytest.mark.parametrize("d", [128, 256, 768])
def test_rmsnorm_i8_table_lengths(dev, d, n):
    """rsqrt tables of n entries: up to 1024 the 16- and 8-lane kernels stage the table in LDS (words past n read as
    zeros and are never indexed), longer ones take the four-rows-a-wave kernel. Short tables drive k, and with it
    the requant shift, up to 27."""
    rng = np.random.default_rng([64, d, n])
    w = rng.integers(-127, 128, d)
    lut = rng.integers(1, 1 << 14, n)
    x = np.concatenate([rng.integers(-128, 128, (90, d)), rng.integers(-2, 3, (40, d)), np.full((2, d), -128),
                        np.zeros((1, d), int)])
    want = sem.rmsnorm_int(x, w, lut, 1, 16)
    got = _rms(dev, x, "i8", w, lut, 1, 16, flags=rt.OP_UNCHECKED | rt.RMS_S24)
    assert np.array_equal(got, want)
    assert np.abs(want).max() > 0


def _wide_case(d, rows, seed):
    """A proven wide rmsnorm (table, s, c, e from the quantizer for |x| <= 2^15) and rows over the full int16 range:
    random rows, the extreme constant rows, a zero row and quiet rows (small sums: low table indexes, k = 0)."""
    rng = np.random.default_rng([8, d, seed])
    w = rng.integers(-127, 128, d)
    lut, s, c, e = Q.wide_rsqrt_table(4e-4, 0.01, 0.02, int(np.abs(w).max()), d, 1e-6, 1 << 15)
    x = np.concatenate([rng.integers(-(1 << 15), 1 << 15, (rows, d)), np.full((1, d), -(1 << 15)),
                        np.full((1, d), (1 << 15) - 1), np.zeros((1, d), int), rng.integers(-40, 41, (rows // 4, d))])
    return x, w, lut, s, c, e


@pytest.mark.parametrize("flags", [0, rt.OP_UNCHECKED, rt.OP_UNCHECKED | rt.RMS_S24])
@pytest.mark.parametrize("d", [8, 16, 24, 32, 40, 128, 504, 512, 520, 768, 1536, 2048])
def test_rmsnorm_i16_wide(dev, d, flags):
    """int16 rows with square shift c and sum offset e. UNCHECKED selects the wide kernel: L lanes a row (the power
    of two >= d / 8, at most 64; lanes past the row idle when d / 8 is not one), up to four 16-byte chunks a lane
    for d > 512; with RMS_S24 (asserted to hold) the 24-bit multiply-add, without it the 32-bit wrapping product."""
    x, w, lut, s, c, e = _wide_case(d, 300, 0)
    if flags & rt.RMS_S24:
        assert int(np.abs(lut).max()) < (1 << 23)
    want = sem.rmsnorm_wide(x, w, lut, 1, s, c, e, "i16")
    assert c > 0 or d == 1
    assert np.array_equal(_rms(dev, x, "i16", w, lut, 1, s, c, e, flags=flags), want)


@pytest.mark.parametrize("d", [8, 32, 768])
def test_rmsnorm_i16_wide_walks_many_row_groups(dev, d):
    """More row groups than the grid has waves (eight workgroups of four waves per CU, 64 / L rows a group): each
    wave walks three or more groups through both row buffers, and the last group is ragged."""
    lanes = min(64, 1 << max(0, (d // 8 - 1).bit_length()))
    rows = 8 * 4 * 256 * (64 // lanes) * 3 + 5
    rng = np.random.default_rng([63, d])
    w = rng.integers(-127, 128, d)
    lut, s, c, e = Q.wide_rsqrt_table(4e-4, 0.01, 0.02, int(np.abs(w).max()), d, 1e-6, 1 << 15)
    x = rng.integers(-(1 << 15), 1 << 15, (rows, d))
    want = sem.rmsnorm_wide(x, w, lut, 1, s, c, e, "i16")
    flags = rt.OP_UNCHECKED | (rt.RMS_S24 if int(np.abs(lut).max()) < (1 << 23) else 0)
    assert np.array_equal(_rms(dev, x, "i16", w, lut, 1, s, c, e, flags=flags), want)


def test_rmsnorm_i16_wide_multiplier(dev):
    """A multiplier M != 1 with the table scaled down by the same factor, so every product stays proven: the wide
    kernel forms lut[i] M per row (wrapping in 32 bits without RMS_S24), and the checked kernel agrees."""
    d = 64
    x, w, lut, s, c, e = _wide_case(d, 200, 1)
    m = 5
    lut = lut // m
    want = sem.rmsnorm_wide(x, w, lut, m, s, c, e, "i16")
    for flags in (0, rt.OP_UNCHECKED):
        assert np.array_equal(_rms(dev, x, "i16", w, lut, m, s, c, e, flags=flags), want)


def _softmax(dev, x, lut, one, causal, dtype="i8", flags=0):
    *lead, t1, t2 = x.shape
    batch = int(np.prod(lead)) if lead else 1
    out = dev.alloc(x.size * rt.ITEMSIZE[dtype])
    dev.softmax_lut(up(dev, x, "i8"), up(dev, lut, "i32"), one, causal, batch, t1, t2, out, dtype, flags)
    dev.sync()
    return out.download(x.shape, rt.NP_DTYPE[dtype]).astype(np.int64)


SOFTMAX_SHAPES = [(2, 3, 4, 4), (5, 7, 3), (2, 1, 100, 100), (1, 2, 64, 1024), (3, 33, 65), (1, 17, 16),
                  (2, 40, 1040), (1, 9, 2048), (1, 5, 4096), (3, 70, 48)]


@pytest.mark.parametrize("flags", [0, rt.OP_UNCHECKED])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", SOFTMAX_SHAPES)
def test_softmax(dev, causal, shape, flags):
    """flags=UNCHECKED (exp_lut keeps every intermediate in int32, entries >= 0, lut[255] = 2^E) selects the
    per-row quotient-table kernel where t2 is a multiple of 16 up to 4096; results are the same bits either way."""
    rng = np.random.default_rng([9, *shape])
    x = rng.integers(-128, 128, shape)
    x[..., 0, :] = -128                          # a row of the minimum value
    x[..., -1, :] = 127                          # and one of the maximum
    lut = Q.exp_table(0.05, shape[-1])
    want = sem.softmax_lut(x, lut, 127, causal)
    assert np.array_equal(_softmax(dev, x, lut, 127, causal, flags=flags), want)


@pytest.mark.parametrize("flags", [0, rt.OP_UNCHECKED])
def test_softmax_i32_result(dev, flags):
    rng = np.random.default_rng(10)
    for shape in ((4, 6, 9), (2, 5, 32)):
        x = rng.integers(-128, 128, shape)
        lut = np.round((1 << 14) * np.exp((np.arange(256) - 255) / 24.0)).astype(np.int64)
        for one in (1, 1000, 4095):
            for causal in (False, True):
                want = sem.softmax_lut(x, lut, one, causal)
                assert np.array_equal(_softmax(dev, x, lut, one, causal, "i32", flags), want)


DT_PAIRS = [("i8", "i8", "i8"), ("i16", "i8", "i16"), ("i8", "i16", "i16"), ("i16", "i16", "i8"), ("i16", "i16", "i16")]


@pytest.mark.parametrize("da,db,do", DT_PAIRS)
def test_add_requant(dev, da, db, do):
    rng = np.random.default_rng([11, len(da), len(db), DT_PAIRS.index((da, db, do))])
    n = 10007
    lim = {"i8": 128, "i16": 1 << 15}
    a, b = rng.integers(-lim[da], lim[da], n), rng.integers(-lim[db], lim[db], n)
    ma, mb, s = (300, 500, 10) if da == db == "i8" else (1 << 14, 1 << 13, 14 + (do == "i8") * 6)
    want = sem.add_requant(a, b, ma, mb, s, do)
    out = dev.alloc(n * rt.ITEMSIZE[do])
    dev.add_requant(up(dev, a, da), da, up(dev, b, db), db, ma, mb, s, n, out, do)
    dev.sync()
    assert np.array_equal(out.download((n,), rt.NP_DTYPE[do]).astype(np.int64), want)


def test_add_requant_known_answer(dev):
    """Reference tests/frontend/test_quantize.py:109-112: i16 operands with an i8 result saturate at int8."""
    a, b = np.array([30000, -30000, 200, -129, 5]), np.zeros(5, int)
    out = dev.alloc(5)
    dev.add_requant(up(dev, a, "i16"), "i16", up(dev, b, "i8"), "i8", 1, 1, 0, 5, out, "i8")
    dev.sync()
    assert list(out.download((5,), np.int8)) == [127, -128, 127, -128, 5]


def test_lut_and_lut_mul(dev):
    rng = np.random.default_rng(12)
    n = 70001
    x, y, t = rng.integers(-128, 128, n), rng.integers(-128, 128, n), rng.integers(-128, 128, 256)
    out = dev.alloc(n)
    dev.lut_i8(up(dev, x, "i8"), up(dev, t, "i8"), n, out)
    dev.sync()
    assert np.array_equal(out.download((n,), np.int8).astype(np.int64), sem.lut_i8(x, t))
    dev.lut_mul(up(dev, x, "i8"), up(dev, y, "i8"), up(dev, t, "i8"), 300, 12, n, out)
    dev.sync()
    assert np.array_equal(out.download((n,), np.int8).astype(np.int64), sem.swiglu_lut(x, y, t, 300, 12))


@pytest.mark.parametrize("da,db,do", DT_PAIRS)
@pytest.mark.parametrize("wide_m", [False, True])
def test_add_requant_unchecked_vector_and_tail(dev, da, db, do, wide_m):
    """ANVIL_OP_UNCHECKED (a proven graph): 32-bit arithmetic, 24-bit multiplies when |Ma|, |Mb| < 2^23 and 32-bit
    ones otherwise, 16 elements a lane over aligned operands plus the n % 16 tail, and operands offset off the 16-byte
    grid (one-element kernel) -- all equal to the reference's checked formula (anvil/semantics.py:106-115)."""
    rng = np.random.default_rng([23, DT_PAIRS.index((da, db, do)), int(wide_m)])
    lim = {"i8": 128, "i16": 1 << 15}
    # multipliers whose worst case a Ma + b Mb + rnd stays inside int32 at these operand ranges: with wide_m, Ma is
    # past 24 bits (32-bit multiplies) and a's values stay within int8 whatever its dtype
    alim = 128 if wide_m else lim[da]
    ma = (1 << 23) + 5 if wide_m else 3000
    mb = -(((1 << 30) - (1 << 21)) // lim[db])
    s = 24 if do == "i8" else 16
    for n, off in ((16 * 4099 + 11, 0), (4096, 0), (999, 1), (15, 0)):
        a, b = rng.integers(-alim, alim, n), rng.integers(-lim[db], lim[db], n)
        want = sem.add_requant(a, b, ma, mb, s, do)
        A = dev.alloc((n + 16) * rt.ITEMSIZE[da])
        B = dev.alloc((n + 16) * rt.ITEMSIZE[db])
        A.upload(a.astype(rt.NP_DTYPE[da]), off * rt.ITEMSIZE[da])
        B.upload(b.astype(rt.NP_DTYPE[db]), off * rt.ITEMSIZE[db])
        out = dev.alloc((n + 16) * rt.ITEMSIZE[do])
        dev.add_requant(A.ptr + off * rt.ITEMSIZE[da], da, B.ptr + off * rt.ITEMSIZE[db], db, ma, mb, s, n,
                        out.ptr + off * rt.ITEMSIZE[do], do, rt.OP_UNCHECKED)
        dev.sync()
        got = out.download((n,), rt.NP_DTYPE[do], offset=off * rt.ITEMSIZE[do]).astype(np.int64)
        assert np.array_equal(got, want), (n, off, int((got != want).sum()))


def test_add_requant_checked_vector_flags_overflow(dev):
    """Checked add over aligned operands (the 16-element kernel): an int32 overflow in one element of the middle of
    the array raises OverflowError at the next sync, as the interpreter raises for the same op."""
    n = 16 * 1000
    a, b = np.zeros(n, int), np.zeros(n, int)
    a[8007] = 100                                         # 100 * 2^25 leaves int32
    out = dev.alloc(n)
    dev.add_requant(up(dev, a, "i8"), "i8", up(dev, b, "i8"), "i8", 1 << 25, 1, 0, n, out, "i8")
    with pytest.raises(OverflowError):
        dev.sync()
    dev.sync()


@pytest.mark.parametrize("mult", [300, (1 << 23) + 3])
def test_lut_and_lut_mul_unchecked_and_unaligned(dev, mult):
    """lut over 16-byte chunks and its tail, and lut_mul with ANVIL_OP_UNCHECKED (24-bit and 32-bit multiply), on
    aligned operands and on operands offset by 3 bytes (one-element kernel), against the oracle."""
    rng = np.random.default_rng([24, mult])
    # with a 32-bit multiplier the table's entries stay in [-1, 1], so table * y * mult + rnd fits int32
    t = rng.integers(-128, 128, 256) if mult < (1 << 23) else rng.integers(-1, 2, 256)
    s = 12 if mult < (1 << 23) else 30
    for n, off in ((16 * 7001 + 5, 0), (5003, 3)):
        x, y = rng.integers(-128, 128, n), rng.integers(-128, 128, n)
        X, Y, O = dev.alloc(n + 16), dev.alloc(n + 16), dev.alloc(n + 16)
        X.upload(x.astype(np.int8), off)
        Y.upload(y.astype(np.int8), off)
        T = up(dev, t, "i8")
        dev.lut_i8(X.ptr + off, T, n, O.ptr + off)
        dev.sync()
        assert np.array_equal(O.download((n,), np.int8, offset=off).astype(np.int64), sem.lut_i8(x, t))
        dev.lut_mul(X.ptr + off, Y.ptr + off, T, mult, s, n, O.ptr + off, rt.OP_UNCHECKED)
        dev.sync()
        assert np.array_equal(O.download((n,), np.int8, offset=off).astype(np.int64),
                              sem.swiglu_lut(x, y, t, mult, s))


@pytest.mark.parametrize("dt", ["i8", "i16", "i32"])
def test_copy_strided(dev, dt):
    rng = np.random.default_rng(13)
    src = rng.integers(-100, 100, (3, 4, 5, 6))
    perm = [2, 0, 3, 1]
    want = np.transpose(src, perm)
    st = [int(np.prod(src.shape[i + 1:])) for i in range(4)]
    out = dev.alloc(src.size * rt.ITEMSIZE[dt])
    dev.copy_strided(up(dev, src, dt), out, rt.ITEMSIZE[dt], want.shape, [st[p] for p in perm])
    dev.sync()
    assert np.array_equal(out.download(want.shape, rt.NP_DTYPE[dt]).astype(np.int64), want)


@pytest.mark.parametrize("f64", [False, True])
def test_quantize_input(dev, f64):
    """round half to even at float64, saturating (reference anvil/driver.py:233-241)."""
    rng = np.random.default_rng(14)
    x = np.concatenate([rng.standard_normal(5000) * 3, [0.5, 1.5, 2.5, -0.5, -2.5, 1e9, -1e9]])
    x = x.astype(np.float64 if f64 else np.float32)
    scale = 0.025
    want = np.clip(np.rint(np.asarray(x, dtype=np.float64) / scale), -128, 127).astype(np.int64)
    xd = dev.upload(np.ascontiguousarray(x))
    out = dev.alloc(x.size)
    dev.quantize(xd, f64, scale, x.size, out, "i8")
    dev.sync()
    assert np.array_equal(out.download((x.size,), np.int8).astype(np.int64), want)
    # i16 results, and an input offset off the 16-byte grid (one-element kernel throughout)
    want16 = np.clip(np.rint(np.asarray(x, dtype=np.float64) / (scale / 300)), -32768, 32767).astype(np.int64)
    out16 = dev.alloc(2 * x.size)
    dev.quantize(xd, f64, scale / 300, x.size, out16, "i16")
    dev.sync()
    assert np.array_equal(out16.download((x.size,), np.int16).astype(np.int64), want16)
    isz = x.itemsize
    dev.quantize(xd.ptr + isz, f64, scale, x.size - 1, out.ptr + 1, "i8")
    dev.sync()
    assert np.array_equal(out.download((x.size - 1,), np.int8, offset=1).astype(np.int64), want[1:])


@pytest.mark.parametrize("f64", [False, True])
def test_quantize_flags_nonfinite_input(dev, f64):
    """A NaN or infinite element (refused by the reference, anvil/driver.py:265-266) makes the next sync raise
    ValueError and is stored as 0; every finite element is quantized as usual, and the flag is cleared."""
    rng = np.random.default_rng(15)
    x = (rng.standard_normal(3000) * 3).astype(np.float64 if f64 else np.float32)
    bad = [7, 1500, 2999]
    x[bad] = [np.nan, np.inf, -np.inf]
    xd, out = dev.upload(np.ascontiguousarray(x)), dev.alloc(x.size)
    dev.quantize(xd, f64, 0.025, x.size, out, "i8")
    with pytest.raises(ValueError, match="NaN or infinite"):
        dev.sync()
    dev.sync()                                            # cleared
    got = out.download((x.size,), np.int8).astype(np.int64)
    fin = np.isfinite(x)
    want = np.clip(np.rint(np.asarray(x[fin], dtype=np.float64) / 0.025), -128, 127)
    assert np.array_equal(got[fin], want) and not got[bad].any()


def _attention_case(B, H, T, D, causal, seed, ms_sign=1, lut_kind="exp", one=127):
    """Random q, k, v (B, T, H D) i8 with scores and output requants that spread over int8, the reference chain
    qmatmul -> softmax_lut -> qmatmul evaluated by the oracle, and the head-split views the fused kernel reads.
    lut_kind: "exp" (the quantizer's table), "steep" (an exp table with a run of zeros at the low end), "random"
    (positive and not monotone, so no threshold shortcut applies), "self" (every key equal to its own query and the
    self score near the clamp: each row peaks on the diagonal, and from T = 64 most 32 x 32 tiles hold p = 0 only,
    beside live ones in the same wave) or "shift25" (score shift 25: the int32 pre-shift range reaches scores in
    [-64, 63] only, so the lowest score, which masked keys of the diagonal tile take, is -64 rather than -128;
    q, k in [-40, 40] keep acc M_s inside int32 as a proven graph's would be)."""
    rng = np.random.default_rng([21, B, H, T, D, int(causal), seed])
    C = H * D
    q, k, v = (rng.integers(-128, 128, (B, T, C)) for _ in range(3))
    if lut_kind == "shift25":
        q, k = rng.integers(-40, 41, (B, T, C)), rng.integers(-40, 41, (B, T, C))
    if seed == 1:
        q[0, :, :D] = 0                                      # a head of all-zero scores: uniform rows
        q[-1, :, -D:], k[-1, :, -D:] = 127, -128             # a head of scores clamped to -128: max = -128
    ms = ms_sign * max(1, round(40 / (74.0 ** 2 * np.sqrt(D)) * (1 << 16)))
    ss, mo, so = 16, 1, 7
    if lut_kind == "random":
        lut = rng.integers(1, 1 << 20, 256)
    elif lut_kind == "shift25":
        ms, ss = ((1 << 31) - (1 << 25)) // (D * 40 * 40), 25    # |acc M_s| + 2^24 < 2^31 for any q, k in range
        lut = Q.exp_table(0.05, T, one)
    elif lut_kind == "self":
        k[:] = q
        ms = round(1.2 * 127 / (D * 5461) * (1 << 16))      # E[q^2] = 5461: the self score just past 127
        lut = Q.exp_table(0.3, T, one)
    else:
        lut = Q.exp_table(0.5 if lut_kind == "steep" else 0.05, T, one)
    split = lambda a: a.reshape(B, T, H, D).transpose(0, 2, 1, 3)       # noqa: E731
    scores = sem.qmatmul(split(q), np.swapaxes(split(k), -1, -2), ms, ss, fast=True)
    p = sem.softmax_lut(scores, lut, one, causal)
    o = sem.qmatmul(p, split(v), mo, so, fast=True)          # (B, H, T, D)
    return q, k, v, (ms, ss, mo, so), lut, o.transpose(0, 2, 1, 3).reshape(B, T, C)


@pytest.mark.parametrize("B,H,T,D", [(1, 2, 32, 16), (2, 3, 64, 32), (1, 2, 96, 64), (2, 2, 128, 32),
                                     (1, 3, 256, 64), (1, 2, 160, 128), (1, 2, 1024, 64), (2, 1, 512, 16),
                                     (1, 1, 1024, 128), (1, 2, 1024, 32), (1, 2, 992, 64), (5, 2, 16, 16),
                                     (3, 3, 16, 32), (300, 2, 16, 16)])
@pytest.mark.parametrize("causal", [True, False])
def test_fused_attention_matches_the_three_ops(dev, B, H, T, D, causal):
    """anvil_attention_i8 over q, k (B, T, H D), v^T (B, H D, T) and o (B, T, H D), as the planner lays them out,
    bit-exact with the oracle's scores -> softmax -> P.V chain, for the quantizer's exp table, a table with a zero run,
    a non-monotone one and rows peaked on the diagonal (tiles whose p are all zero are skipped), and one = 127 or
    100. T = 16 runs the one-lane-a-row kernel (four heads a wave; 300 x 2 heads leave the last wave part empty)."""
    for seed, sign, kind, one in ((0, 1, "exp", 127), (1, -1, "exp", 127), (2, 1, "random", 127), (3, 1, "steep", 100),
                                  (4, 1, "self", 127), (5, 1, "shift25", 127)):
        q, k, v, (ms, ss, mo, so), lut, want = _attention_case(B, H, T, D, causal, seed, sign, kind, one)
        if kind == "steep":
            assert (lut == 0).any() and np.all(np.diff(lut) >= 0)
        if kind == "random":
            assert np.any(np.diff(lut) < 0)
        C = H * D
        vt = np.ascontiguousarray(np.swapaxes(v, 1, 2))      # (B, C, T)
        out = dev.alloc(B * T * C)
        strides = [T * C, D, C, T * C, D, C, C * T, D * T, T, T * C, D, C]
        dev.attention_i8(up(dev, q, "i8"), up(dev, k, "i8"), up(dev, vt, "i8"), out, B, H, T, D, strides, ms, ss,
                         up(dev, lut, "i32"), one, causal, mo, so, rt.OP_UNCHECKED)
        dev.sync()
        got = out.download((B, T, C), np.int8).astype(np.int64)
        assert np.array_equal(got, want), (seed, kind, np.argwhere(got != want)[:5])
        if T == 16:                                         # V's own rows (ATTN_V_ROWS) in place of V^T
            out2 = dev.alloc(B * T * C)
            strides_v = strides[:6] + [T * C, D, C] + strides[9:]
            dev.attention_i8(up(dev, q, "i8"), up(dev, k, "i8"), up(dev, v, "i8"), out2, B, H, T, D, strides_v, ms, ss,
                             up(dev, lut, "i32"), one, causal, mo, so, rt.OP_UNCHECKED | rt.ATTN_V_ROWS)
            dev.sync()
            assert np.array_equal(out2.download((B, T, C), np.int8).astype(np.int64), want), (seed, kind, "V rows")


@pytest.mark.parametrize("B,H,T,D,pad", [(1, 2, 32, 16, 0), (2, 3, 64, 32, 16), (1, 3, 256, 64, 0),
                                         (1, 2, 160, 128, 32), (1, 2, 1024, 64, 0), (2, 1, 512, 16, 0),
                                         (1, 2, 992, 64, 16), (7, 2, 16, 16, 0), (3, 3, 16, 32, 16)])
@pytest.mark.parametrize("causal", [True, False])
def test_fused_attention_keep_stores_scores_and_probabilities(dev, B, H, T, D, pad, causal):
    """anvil_attention_i8_keep: the output as anvil_attention_i8's, and every score (the whole T x T product, past
    the causal diagonal too) and every probability (0 for masked keys and for tiles skipped as all-zero) stored,
    bit-exact with the oracle's scores -> softmax -> P.V chain. S and P start filled with another byte, so an
    element the kernel leaves unwritten fails; pad > 0 gives their rows a stride of T + pad."""
    for seed, sign, kind, one in ((0, 1, "exp", 127), (2, 1, "random", 127), (3, 1, "steep", 100), (4, 1, "self", 127),
                                  (5, 1, "shift25", 127)):
        q, k, v, (ms, ss, mo, so), lut, want = _attention_case(B, H, T, D, causal, seed, sign, kind, one)
        split = lambda a: a.reshape(B, T, H, D).transpose(0, 2, 1, 3)       # noqa: E731
        scores = sem.qmatmul(split(q), np.swapaxes(split(k), -1, -2), ms, ss, fast=True)
        p = sem.softmax_lut(scores, lut, one, causal)
        C, ld = H * D, T + pad
        vt = np.ascontiguousarray(np.swapaxes(v, 1, 2))      # (B, C, T)
        out = dev.alloc(B * T * C)
        sb, pb = dev.alloc(B * H * T * ld), dev.alloc(B * H * T * ld)
        for b in (sb, pb):
            b.upload(np.full(B * H * T * ld, 0x5A, np.uint8))
        strides = [T * C, D, C, T * C, D, C, C * T, D * T, T, T * C, D, C, H * T * ld, T * ld, ld, H * T * ld, T * ld,
                   ld]
        dev.attention_i8_keep(up(dev, q, "i8"), up(dev, k, "i8"), up(dev, vt, "i8"), out, sb, pb, B, H, T, D, strides,
                              ms, ss, up(dev, lut, "i32"), one, causal, mo, so, rt.OP_UNCHECKED)
        dev.sync()
        got = out.download((B, T, C), np.int8).astype(np.int64)
        assert np.array_equal(got, want), (seed, kind, np.argwhere(got != want)[:5])
        gs = sb.download((B, H, T, ld), np.int8).astype(np.int64)
        gp = pb.download((B, H, T, ld), np.int8).astype(np.int64)
        assert np.array_equal(gs[..., :T], scores), (seed, kind, np.argwhere(gs[..., :T] != scores)[:5])
        assert np.array_equal(gp[..., :T], p), (seed, kind, np.argwhere(gp[..., :T] != p)[:5])
        assert np.all(gs[..., T:] == 0x5A) and np.all(gp[..., T:] == 0x5A)      # the row padding is untouched


def test_fused_attention_keep_checks_its_strides(dev):
    """The kept form refuses S / P strides that are not multiples of 16 or rows shorter than T, before any launch."""
    B, H, T, D = 1, 1, 64, 32
    bufs = [dev.alloc(4096) for _ in range(6)]
    lut = up(dev, Q.exp_table(0.05, T, 127), "i32")
    base = [T * D, T * D, D, T * D, T * D, D, D * T, D * T, T, T * D, T * D, D]
    for tail, msg in (([T * T, T * T, T, T * T, T * T, T + 8], "multiple of 16"),
                      ([T * T, T * T, 48, T * T, T * T, T], "out of range")):
        with pytest.raises(ValueError, match=msg):
            dev.attention_i8_keep(*bufs, B, H, T, D, base + tail, 1, 16, lut, 127, True, 1, 7, rt.OP_UNCHECKED)


# add_requant multipliers: a negative one, config 5's two adds (Ma above 2^23, 128 (Ma + Mb) close to 2^31), and
# Ma = Mb = 1 with no shift
# multipliers of every sign, at and above 2^23 (the 24-bit byte-multiply form covers magnitudes below 2^24; the
# worst-case sum still inside int32)
ADD_MULTS = [(300, -200, 9), (11157253, 4299753, 24), (7873258, 3110671, 23), (1, 1, 0), (-12000000, 4000000, 24),
             (16000000, -700000, 24), (-8388608, -8000000, 24)]


@pytest.mark.parametrize("M,K,N", [(256, 768, 768), (300, 64, 200), (33, 48, 72), (1024, 256, 384)])
@pytest.mark.parametrize("store_y", [True, False])
@pytest.mark.parametrize("ma,mb,s2", ADD_MULTS)
def test_gemm_with_fused_residual_add(dev, M, K, N, store_y, ma, mb, s2):
    """anvil_gemm_i8_add: y = qlinear(a, w) [LUT] and D = add_requant(r, y) in one launch, bit-exact with the two ops;
    N not a multiple of 16 takes the per-byte epilogue."""
    rng = np.random.default_rng([31, M, K, N, int(store_y)])
    a, w, r = rng.integers(-128, 128, (M, K)), rng.integers(-128, 128, (K, N)), rng.integers(-128, 128, (M, N))
    m, s = 3, 16
    lut = rng.integers(-128, 128, 256) if N == 200 else None
    y = sem.qmatmul(a, w, m, s, lut)
    want = sem.add_requant(r, y, ma, mb, s2)
    c = dev.alloc(M * N) if store_y else None
    d = dev.alloc(M * N)
    wt = np.ascontiguousarray(w.T)
    flags = rt.GEMM_UNCHECKED | rt.GEMM_MUL24
    dev.gemm_i8_add(up(dev, a, "i8"), up(dev, wt, "i8"), c, 1, 1, M, N, K, [0, 0, K, 0, 0, K, 0, 0, N], m, s,
                    None if lut is None else up(dev, lut, "i8"), up(dev, r, "i8"), ma, mb, s2, d,
                    [0, 0, N, 0, 0, N], flags)
    dev.sync()
    assert np.array_equal(d.download((M, N), np.int8).astype(np.int64), want)
    if store_y:
        assert np.array_equal(c.download((M, N), np.int8).astype(np.int64), y)


@pytest.mark.parametrize("M,K,N", [(256, 768, 768), (300, 64, 200), (33, 48, 72), (1024, 256, 384), (4096 + 37, 32, 32),
                                   (32768, 768, 3072)])
@pytest.mark.parametrize("store_y", [True, False])
def test_gemm_with_fused_i16_residual_add(dev, M, K, N, store_y):
    """anvil_gemm_i8_add_ex on the wide residual stream (ADR-004): y = qlinear(a, w) as int16, D = add_requant(R, y)
    with R and D int16, in one launch, bit-exact with the two ops. Interior tiles, ragged edges (N not a multiple of
    8 takes the per-element epilogue), rows of 32 entries (the frozen v2 model's width) and a wide product that the
    persistent kernels would otherwise take."""
    rng = np.random.default_rng([32, M, K, N, int(store_y)])
    a, w = rng.integers(-128, 128, (M, K), dtype=np.int8), rng.integers(-128, 128, (K, N), dtype=np.int8)
    r = rng.integers(-32768, 32768, (M, N), dtype=np.int16)
    # the oracle on every row of the small shapes, on the first and last 256 rows and 512 others of the large one
    rows = (np.arange(M) if M * N <= 1 << 22 else
            np.unique(np.concatenate([np.arange(256), np.arange(M - 256, M), rng.integers(0, M, 512)])))
    a64, w64 = a.astype(np.int64), w.astype(np.int64)
    acc = sem.matmul_i8(a64[rows], w64, fast=True)
    (m,), s = Q.choose_shift([20000 / (1.5 * max(1, int(np.abs(acc).max())))], [128 * int(np.abs(w64).sum(axis=0).max())])
    ma, mb, s2 = 16000, -15000, 15
    y = sem.qmatmul(a64[rows], w64, m, s, None, "i16", fast=True)
    want = sem.add_requant(r[rows].astype(np.int64), y, ma, mb, s2, "i16")
    c = dev.alloc(2 * M * N) if store_y else None
    d = dev.alloc(2 * M * N)
    flags = rt.GEMM_UNCHECKED | (rt.GEMM_MUL24 if K * 128 * 128 < (1 << 23) and m < (1 << 23) else 0)  # static bound
    dev.gemm_i8_add(up(dev, a, "i8"), up(dev, np.ascontiguousarray(w.T), "i8"), c, 1, 1, M, N, K,
                    [0, 0, K, 0, 0, K, 0, 0, N], m, s, None, up(dev, r, "i16"), ma, mb, s2, d, [0, 0, N, 0, 0, N],
                    flags, "i16")
    dev.sync()
    got = d.download((M, N), np.int16)[rows].astype(np.int64)
    assert np.array_equal(got, want), np.argwhere(got != want)[:5]
    if store_y:
        assert np.array_equal(c.download((M, N), np.int16)[rows].astype(np.int64), y)


def _add_norm_case(M, N, K, seed, wide_shift=False):
    """Operands of a fused qlinear + add_requant + rmsnorm_int and the oracle's three results (y, D, H)."""
    rng = np.random.default_rng([33, M, N, K, seed])
    a, w = rng.integers(-128, 128, (M, K)), rng.integers(-128, 128, (K, N))
    r = rng.integers(-128, 128, (M, N))
    acc = sem.matmul_i8(a[:256], w, fast=True)
    (m,), s = Q.choose_shift([127 / (1.5 * max(1, int(np.abs(acc).max())))], [128 * int(np.abs(w).sum(axis=0).max())])
    ma, mb, s2 = [(7873258, 3110671, 23), (-12000000, 4000000, 24), (300, -200, 9)][seed % 3]
    nw = rng.integers(-127, 128, N)
    if wide_shift:       # shifts s + k from 20 up past 24 (the clamp bounds at the int32 limits)
        nlut, ns = rng.integers(1, 1 << 14, 1024), 20
    else:
        nlut, ns = Q.rsqrt_table(0.03, 0.01, 0.02, int(np.abs(nw).max()), N, 1e-5)
    y = sem.qmatmul(a, w, m, s, None, fast=True)
    d = sem.add_requant(r, y, ma, mb, s2)
    h = sem.rmsnorm_int(d, nw, nlut, 1, ns)
    return a, w, r, m, s, ma, mb, s2, nw, nlut, ns, y, d, h


@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (1024, 128, 128), (16384, 128, 512), (256, 256, 256),
                                   (16384, 256, 256), (384, 256, 1024)])
@pytest.mark.parametrize("store_y,kb", [(True, False), (False, True), (False, False)])
def test_gemm_add_norm(dev, M, N, K, store_y, kb):
    """anvil_gemm_i8_add_norm: y = qlinear(a, w), D = add_requant(r, y) and H = rmsnorm_int(D) in one launch, each
    128 x N tile spanning its rows (the blocks' C = 128 and 256): D, H (row-major or K-blocked) and y bit-exact
    against the three ops, with add multipliers of both signs and at 2^23."""
    a, w, r, m, s, ma, mb, s2, nw, nlut, ns, y, d, h = _add_norm_case(M, N, K, M + K + int(store_y) + 2 * int(kb))
    C_ = dev.alloc(M * N) if store_y else None
    D_, H_ = dev.alloc(M * N), dev.alloc(M * N)
    flags = rt.GEMM_UNCHECKED | rt.GEMM_NORM_S24 | (rt.GEMM_MUL24 if K * 128 * 128 < (1 << 23) and m < (1 << 23) else 0)
    dev.gemm_i8_add_norm(up(dev, a, "i8"), up(dev, np.ascontiguousarray(w.T), "i8"), C_, M, N, K,
                         [0, 0, K, 0, 0, K, 0, 0, N], m, s, None, up(dev, r, "i8"), ma, mb, s2, D_, [0, 0, N, 0, 0, N],
                         up(dev, nw, "i8"), up(dev, nlut, "i32"), len(nlut), 1, ns, H_, 64 if kb else N,
                         M * 64 if kb else 0, flags)
    dev.sync()
    assert np.array_equal(D_.download((M, N), np.int8).astype(np.int64), d)
    got_h = H_.download((M * N,), np.int8).astype(np.int64)
    got_h = got_h.reshape(N // 64, M, 64).transpose(1, 0, 2).reshape(M, N) if kb else got_h.reshape(M, N)
    assert np.array_equal(got_h, h), np.argwhere(got_h != h)[:5]
    if store_y:
        assert np.array_equal(C_.download((M, N), np.int8).astype(np.int64), y)


@pytest.mark.parametrize("N", [128, 256])
def test_gemm_add_norm_shifts_reaching_int32_bounds(dev, N):
    """The fused rmsnorm with a 1024-entry table and s = 20: rows with large sums take k up to 7, so s + k passes
    24, where the pre-shift clamp bounds saturate to the int32 limits (as in the stand-alone kernel's test)."""
    M, K = 1024, 256
    a, w, r, m, s, ma, mb, s2, nw, nlut, ns, y, d, h = _add_norm_case(M, N, K, 5, wide_shift=True)
    D_, H_ = dev.alloc(M * N), dev.alloc(M * N)
    dev.gemm_i8_add_norm(up(dev, a, "i8"), up(dev, np.ascontiguousarray(w.T), "i8"), None, M, N, K,
                         [0, 0, K, 0, 0, K, 0, 0, N], m, s, None, up(dev, r, "i8"), ma, mb, s2, D_, [0, 0, N, 0, 0, N],
                         up(dev, nw, "i8"), up(dev, nlut, "i32"), len(nlut), 1, ns, H_, N, 0,
                         rt.GEMM_UNCHECKED | rt.GEMM_NORM_S24)
    dev.sync()
    assert np.array_equal(H_.download((M, N), np.int8).astype(np.int64), h)
    assert np.abs(h).max() > 0


@pytest.mark.parametrize("M,N,ma,flags,what", [(200, 128, 300, None, "multiple of 128"), (128, 192, 300, None, "128 or 256"),
                                               (128, 128, 1 << 24, None, "below 2^24"),
                                               (128, 128, 300, rt.GEMM_UNCHECKED, "NORM_S24")])
def test_gemm_add_norm_rejects(dev, M, N, ma, flags, what):
    """The fused entry point's preconditions, each refused with a ValueError before any launch."""
    K = 64
    flags = rt.GEMM_UNCHECKED | rt.GEMM_NORM_S24 if flags is None else flags
    buf = dev.alloc(max(M, 256) * max(N, 256) * 4)
    with pytest.raises(ValueError, match=re.escape(what)):
        dev.gemm_i8_add_norm(buf, buf, None, M, N, K, [0, 0, K, 0, 0, K, 0, 0, N], 1, 8, None, buf, ma, 1, 8, buf,
                             [0, 0, N, 0, 0, N], buf, buf, 1024, 1, 8, buf, N, 0, flags)


@pytest.mark.parametrize("M,N,K,dtype,lut,add", [(32768, 3072, 768, "i8", True, False),
                                                 (49115, 2080, 768, "i16", False, False),
                                                 (32768, 3072, 3072, "i8", False, False),
                                                 (32768, 3072, 768, "i8", False, True)])
def test_gemm_wide_products_take_the_persistent_kernel(dev, M, N, K, dtype, lut, add):
    """Products with N >= 2048 and at least six 256 x 256 tiles per CU run on the persistent kernel (register epilogue,
    permuted B rows). Checked on sampled rows, the first and last 256 among them (edge rows and columns included)."""
    _check_sampled_gemm(dev, M, N, K, dtype, lut, add, 41)


@pytest.mark.parametrize("M,N,K,dtype,lut,add", [(16384 + 37, 3072, 3072, "i8", True, False),
                                                 (20000, 2080, 2048, "i16", False, False),
                                                 (16384, 3072, 3072, "i8", False, True),
                                                 (8192 + 5, 2048 + 48, 2304, "i8", False, False)])
def test_gemm_wide_long_k_two_stages(dev, M, N, K, dtype, lut, add):
    """N and K >= 2048 (config 2's 16384 x 3072 x 3072) run on the persistent 256 x 256 kernel with 128-byte K blocks in
    two LDS stages: ragged rows and columns, a LUT, an i16 result and the fused residual add."""
    _check_sampled_gemm(dev, M, N, K, dtype, lut, add, 47)


@pytest.mark.parametrize("M,N,K,dtype,lut,add", [(32768 + 37, 768, 3072, "i8", False, False),
                                                 (32768, 1536, 2048, "i8", True, False),
                                                 (33000, 768, 2048, "i16", False, False),
                                                 (32768, 768, 3072, "i8", False, True)])
def test_gemm_long_k_narrow_n(dev, M, N, K, dtype, lut, add):
    """K >= 2048 with N below 2048 (the block's proj shape). K a multiple of 384 (24 K blocks of 128) runs on the
    persistent kernel with 256 x 128 tiles and 128-byte K blocks, the fused residual add included; K 2048 (16 blocks)
    with N a multiple of 192 runs on 256 x 192 tiles, whose staged epilogue has 12 16-byte chunks a row (a thread's
    chunks change column between store passes). Ragged M exercises the partial-tile epilogues; an i16 result and a
    LUT are included."""
    _check_sampled_gemm(dev, M, N, K, dtype, lut, add, 43)


@pytest.mark.parametrize("M,N,K", [(32768, 768, 768), (32768 + 37, 768, 3072), (32768, 3072, 768)])
@pytest.mark.parametrize("ma,mb,s2", ADD_MULTS[1:3])
def test_gemm_fused_add_block_multipliers(dev, M, N, K, ma, mb, s2):
    """The block's add multipliers on the kernels that take the block's shapes: 256 x 128 tiles (y), the persistent
    kernel with 128-byte K blocks (proj, ragged rows) and the 256 x 256 persistent kernel."""
    _check_sampled_gemm(dev, M, N, K, "i8", False, True, 45, (ma, mb, s2))


@pytest.mark.parametrize("M,N,K,s", [(32768, 3072, 768, 12), (32768, 3072, 768, 16), (32768, 3072, 768, 17),
                                     (32768, 3072, 768, 27), (32768 + 37, 3072 + 40, 768, 18),
                                     (32768, 768, 3072, 17), (32768, 768, 3072, 18)])
def test_gemm_persistent_lut_table_forms(dev, M, N, K, s):
    """The persistent kernels' LUT epilogue at shifts on both sides of the widened table's limit: a table of
    2^(32 - s) entries that fits beside the LDS stages (32 KiB for the 256 x 256 kernel, s >= 17; 16 KiB for the
    256 x 128 one with 128-byte K blocks, s >= 18) is indexed by (x + 2^31) >> s with the clamp folded into its entries, otherwise the
    rotated 256-entry table follows a clamp. The multiplier spreads the accumulators over the whole int32 range, so
    both clamp ends and every table region are hit; ragged edges take the per-element path."""
    _check_sampled_gemm(dev, M, N, K, "i8", True, False, 49, s=s)


def _check_sampled_gemm(dev, M, N, K, dtype, lut, add, seed, mults=(300, -200, 9), s=20):
    rng = np.random.default_rng([seed, M, N, K])
    a, w = rng.integers(-128, 128, (M, K), dtype=np.int8), rng.integers(-128, 128, (K, N), dtype=np.int8)
    rows = np.unique(np.concatenate([np.arange(256), np.arange(M - 256, M), rng.integers(0, M, 512)]))
    acc = sem.matmul_i8(a[rows].astype(np.int64), w.astype(np.int64), fast=True)   # float64 BLAS, exact here
    m = int(min(((1 << 31) - 1 - (1 << (s - 1))) // int(np.abs(acc).max() * 2), (1 << 23) - 1))
    L = rng.integers(-128, 128, 256) if lut else None
    flags = rt.GEMM_UNCHECKED | rt.GEMM_MUL24
    wt = np.ascontiguousarray(w.T)
    c = dev.alloc(M * N * rt.ITEMSIZE[dtype])
    st = [0, 0, K, 0, 0, K, 0, 0, N]
    y = sem.qmatmul(a[rows].astype(np.int64), w.astype(np.int64), m, s, L, dtype=dtype, fast=True)
    if add:
        r = rng.integers(-128, 128, (M, N), dtype=np.int8)
        d = dev.alloc(M * N)
        dev.gemm_i8_add(up(dev, a, "i8"), up(dev, wt, "i8"), c, 1, 1, M, N, K, st, m, s, None, up(dev, r, "i8"),
                        *mults, d, [0, 0, N, 0, 0, N], flags)
    else:
        dev.gemm_i8(up(dev, a, "i8"), up(dev, wt, "i8"), c, 1, 1, M, N, K, st, m, s,
                    None if L is None else up(dev, L, "i8"), dtype, flags)
    dev.sync()
    got = c.download((M, N), rt.NP_DTYPE[dtype])[rows].astype(np.int64)
    assert np.array_equal(got, y), np.argwhere(got != y)[:5]
    if add:
        want = sem.add_requant(r[rows].astype(np.int64), y, *mults)
        assert np.array_equal(d.download((M, N), np.int8)[rows].astype(np.int64), want)


@pytest.mark.parametrize("M,N,K", [(262144, 32, 32), (4096 + 37, 64, 32), (20000 + 5, 32, 64), (8192, 64, 64)])
@pytest.mark.parametrize("dtype,lut,add", [("i8", False, False), ("i8", True, False), ("i16", False, False),
                                           ("i8", False, True)])
def test_narrow_products_take_the_skinny_kernel(dev, M, N, K, dtype, lut, add):
    """K and N each 32 or 64 with at least 4096 rows (the frozen models' layers): one wave per 32-row block, weight
    fragments in registers; ragged row counts, the LUT epilogue, i16 results and the fused i8 residual add, checked
    on sampled rows (the first and last 256 among them)."""
    _check_sampled_gemm(dev, M, N, K, dtype, lut, add, 43)


@pytest.mark.parametrize("N,K,n", [(32, 32, 3), (64, 32, 2), (32, 64, 4)])
def test_narrow_group_shares_its_left_operand(dev, N, K, n):
    """anvil_gemm_i8_group of narrow products reading one left operand (q, k and v of one input; gate and up): one
    pass of the skinny kernel, every member bit-exact with the oracle, each with its own requant and one with a LUT."""
    M = 16384 * 16 + 7
    rng = np.random.default_rng([44, N, K, n])
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    rows = np.unique(np.concatenate([np.arange(256), np.arange(M - 256, M), rng.integers(0, M, 512)]))
    A = up(dev, a, "i8")
    calls, wants, outs = [], [], []
    for j in range(n):
        w = rng.integers(-128, 128, (K, N), dtype=np.int8)
        acc = sem.matmul_i8(a[rows].astype(np.int64), w.astype(np.int64), fast=True)
        s = 18 + j
        m = int(min(((1 << 31) - 1 - (1 << (s - 1))) // int(np.abs(acc).max() * 2), (1 << 23) - 1))
        L = rng.integers(-128, 128, 256) if j == 1 else None
        wants.append(sem.qmatmul(a[rows].astype(np.int64), w.astype(np.int64), m, s, L, fast=True))
        c = dev.alloc(M * N)
        outs.append(c)
        calls.append((A, up(dev, np.ascontiguousarray(w.T), "i8"), c, 1, 1, M, N, K, [0, 0, K, 0, 0, K, 0, 0, N], m, s,
                      None if L is None else up(dev, L, "i8"), "i8", rt.GEMM_UNCHECKED | rt.GEMM_MUL24))
    dev.gemm_i8_group(calls)
    dev.sync()
    for j in range(n):
        got = outs[j].download((M, N), np.int8)[rows].astype(np.int64)
        assert np.array_equal(got, wants[j]), (j, np.argwhere(got != wants[j])[:5])


# members (M, N, K, batch, A shared by the batch entries, LUT): q / k / v of the block (v computed transposed, per
# sequence, with the weight as the shared left operand), ragged rows and columns, tile counts that are not multiples
# of 8 (padding workgroups between members), and a group whose members take different kernels (one launch each)
GROUP_CASES = {
    "qkv": [(24576, 768, 768, 1, False, False), (24576, 768, 768, 1, False, True), (768, 1024, 768, 24, True, False)],
    "ragged": [(24576 + 300, 768, 768, 1, False, False), (768, 1000, 768, 24, True, True),
               (20000 + 37, 840 + 5, 512 + 16, 1, False, False), (4096, 640, 256, 7, False, False)],
    "mixed": [(24576, 768, 768, 1, False, False), (300, 200, 64, 1, False, True), (16384, 3072, 768, 1, False, False)],
}


@pytest.mark.parametrize("dtype", ["i8", "i16"])
@pytest.mark.parametrize("case", sorted(GROUP_CASES))
def test_gemm_group_matches_separate_launches(dev, case, dtype):
    """anvil_gemm_i8_group: every member's result equals anvil_gemm_i8_ex's for the same arguments (the whole
    result, device against device), and the oracle's on sampled rows of each batch entry."""
    members = GROUP_CASES[case]
    if dtype == "i16":
        members = [mb[:5] + (False,) for mb in members]
    rng = np.random.default_rng([47, len(case), dtype == "i8"])
    s, flags = 20, rt.GEMM_UNCHECKED | rt.GEMM_MUL24
    calls, sep, checks = [], [], []
    for M, N, K, nb, shared, lut in members:
        a = rng.integers(-128, 128, (1 if shared else nb, M, K), dtype=np.int8)
        bt = rng.integers(-128, 128, (nb, N, K), dtype=np.int8)
        L = rng.integers(-128, 128, 256) if lut else None
        rows = np.unique(np.concatenate([np.arange(min(M, 64)), np.arange(max(M - 64, 0), M), rng.integers(0, M, 64)]))
        accs = [sem.matmul_i8(a[0 if shared else b][rows].astype(np.int64), bt[b].T.astype(np.int64), fast=True)
                for b in range(nb)]
        m = int(min(((1 << 31) - 1 - (1 << (s - 1))) // int(2 * max(np.abs(x).max() for x in accs)), (1 << 23) - 1))
        st = [0, 0 if shared else M * K, K, 0, N * K, K, 0, M * N, N]
        A, Bt = up(dev, a, "i8"), up(dev, bt, "i8")
        Ld = None if L is None else up(dev, L, "i8")
        c1, c2 = dev.alloc(nb * M * N * rt.ITEMSIZE[dtype]), dev.alloc(nb * M * N * rt.ITEMSIZE[dtype])
        calls.append((A, Bt, c1, 1, nb, M, N, K, st, m, s, Ld, dtype, flags))
        sep.append((A, Bt, c2, 1, nb, M, N, K, st, m, s, Ld, dtype, flags))
        want = [sem.requant_dtype(x, m, s, dtype) for x in accs]
        checks.append((c1, c2, (nb, M, N), rows, [w if L is None else sem.lut_i8(w, L) for w in want], (A, Bt, Ld)))
    dev.gemm_i8_group(calls)
    for c in sep:
        dev.gemm_i8(*c)
    dev.sync()
    for i, (c1, c2, shape, rows, want, _) in enumerate(checks):
        got = c1.download(shape, rt.NP_DTYPE[dtype])
        assert np.array_equal(got, c2.download(shape, rt.NP_DTYPE[dtype])), (case, i)
        for b, w in enumerate(want):
            assert np.array_equal(got[b][rows].astype(np.int64), w), (case, i, b)


@pytest.mark.parametrize("dtype", ["i8", "i16"])
@pytest.mark.parametrize("C", [48, 772, 30])
def test_embed_quantize(dev, dtype, C):
    """anvil_embed_quantize: clamp(rint((wte[id] + wpe[t]) / scale)) in float64, as the host computes it. C a multiple
    of 4 takes the four-columns-a-lane kernel (772: more float4 columns than a wave has lanes), C = 30 the
    one-element kernel."""
    rng = np.random.default_rng([51, dtype == "i8", C])
    vocab, T, B = 300, 40, 3
    wte = rng.normal(0, 0.02, (vocab, C)).astype(np.float32)
    wpe = rng.normal(0, 0.02, (T + 5, C)).astype(np.float32)
    ids = rng.integers(0, vocab, (B, T))
    scale = 0.0004 if dtype == "i8" else 1e-6
    x = wte.astype(np.float64)[ids] + wpe.astype(np.float64)[None, :T]
    lo, hi = (-128, 127) if dtype == "i8" else (-32768, 32767)
    want = np.clip(np.rint(x / scale), lo, hi).astype(np.int64)
    out = dev.alloc(B * T * C * rt.ITEMSIZE[dtype])
    dev.embed_quantize(dev.upload(ids.astype(np.int64)), B * T, T, C, dev.upload(wte), vocab, dev.upload(wpe), scale,
                       out, dtype)
    dev.sync()
    assert np.array_equal(out.download((B, T, C), rt.NP_DTYPE[dtype]).astype(np.int64), want)
    assert (want == lo).any() and (want == hi).any()           # saturation on both sides is exercised


@pytest.mark.parametrize("k", [0, 3, 41, 126, -128])
def test_embed_quantize_at_half_integers(dev, k):
    """The four-columns-a-lane kernel rounds x / scale through a multiply by 1 / scale away from the half-integers
    and takes the quotient near them: scales that put x0 / scale at or next to +-(k + 1/2) for some of the table's
    sums x0 (each such element takes the quotient), and a power-of-two scale (an exact product), all against the
    host's float64 quotient."""
    rng = np.random.default_rng([52, k + 200])
    vocab, T, C = 64, 8, 64
    wte = rng.normal(0, 0.05, (vocab, C)).astype(np.float32)
    wpe = np.zeros((T, C), np.float32)
    wpe[1:] = rng.normal(0, 0.05, (T - 1, C)).astype(np.float32)
    ids = rng.integers(0, vocab, (4, T))
    x = wte.astype(np.float64)[ids] + wpe.astype(np.float64)[None, :T]
    x0 = x[np.abs(x) > 1e-3].ravel()[:6]
    scales = [float(v) / (k + 0.5) for v in x0]
    scales += [np.nextafter(s, np.inf) for s in scales[:2]] + [2.0 ** -10]
    for scale in scales:
        scale = abs(scale)
        want = np.clip(np.rint(x / scale), -128, 127).astype(np.int64)
        out = dev.alloc(ids.size * C)
        dev.embed_quantize(dev.upload(ids.astype(np.int64)), ids.size, T, C, dev.upload(wte), vocab, dev.upload(wpe),
                           scale, out, "i8")
        dev.sync()
        assert np.array_equal(out.download((4, T, C), np.int8).astype(np.int64), want), scale


def test_page_locked_download_round_trip(dev):
    """anvil_host_alloc memory as a download target: every byte of a device buffer arrives, a second download into
    the same host buffer replaces the first, and an oversized request is refused before the copy."""
    rng = np.random.default_rng(77)
    a = rng.integers(-128, 128, (3, 1000), dtype=np.int8)
    b = rng.integers(-2 ** 15, 2 ** 15, (1500,), dtype=np.int16)
    da, db = dev.upload(a), dev.upload(b)
    host = dev.host_alloc(3000)
    got = da.download((3, 1000), np.int8, into=host)
    assert np.array_equal(got, a)
    got = db.download((1500,), np.int16, into=host)
    assert np.array_equal(got, b) and np.array_equal(host.array(np.int16, 1500), b)
    with pytest.raises(ValueError):
        da.download((3001,), np.int8, into=host)
    host.free()
