"""K-blocked GEMM operands and results (ANVIL_GEMM_A_KBLOCK / B_KBLOCK / C_KBLOCK): row r's 64-element block j at
r * 64 + j * stride.
Every fast kernel family reads them (256 x 128 and 128 x 128 tiles, 256 x 192, the three persistent forms, split-K, the
fused residual add, batched and grouped products), with a last K block that is partial and padding rows between
blocks; the results equal the oracle's (reference op: anvil/semantics.py:95-103) on sampled rows."""
import numpy as np
import pytest

from anvil_mi355x import runtime as rt
from oracle import semantics as sem

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return rt.device(0)


def up(dev, arr, dt="i8"):
    return dev.upload(np.ascontiguousarray(np.asarray(arr)).astype(rt.NP_DTYPE[dt]))


def kblock(x, pad_rows, rng):
    """(R, K) -> (ceil(K / 64), R + pad_rows, 64): block j of row r at [j, r]; the pad rows hold noise, K past its end
    zeros. Returns the array and its block stride in bytes."""
    R, K = x.shape
    nb = -(-K // 64)
    out = rng.integers(-128, 128, (nb, R + pad_rows, 64), dtype=np.int8)
    xp = np.zeros((R, nb * 64), np.int8)
    xp[:, :K] = x
    out[:, :R, :] = xp.reshape(R, nb, 64).transpose(1, 0, 2)
    return out, (R + pad_rows) * 64


def _operands(dev, a, wt, mode, rng):
    """Device A and Bt in the mode's layouts and the strides[2] / strides[5] and flags that describe them."""
    M, K = a.shape
    flags = 0
    if "A" in mode:
        ak, lda = kblock(a, 3, rng)
        A, flags = up(dev, ak), flags | rt.GEMM_A_KBLOCK
    else:
        A, lda = up(dev, a), K
    if "B" in mode:
        bk, ldb = kblock(wt, 5, rng)
        B, flags = up(dev, bk), flags | rt.GEMM_B_KBLOCK
    else:
        B, ldb = up(dev, wt), K
    return A, B, lda, ldb, flags


def _result(dev, M, N, dtype, mode):
    """The result buffer (K-blocked with two pad rows when "C" is in the mode), strides[8], its flag, and a reader."""
    if "C" not in mode:
        c = dev.alloc(M * N * rt.ITEMSIZE[dtype])
        return c, N, 0, lambda: c.download((M, N), rt.NP_DTYPE[dtype])
    nb, rows = -(-N // 64), M + 2
    c = dev.alloc(nb * rows * 64 * rt.ITEMSIZE[dtype])
    read = lambda: c.download((nb, rows, 64), rt.NP_DTYPE[dtype])[:, :M].transpose(1, 0, 2).reshape(M, -1)[:, :N]  # noqa
    return c, rows * 64, rt.GEMM_C_KBLOCK, read


def _check(dev, M, N, K, mode, seed, lut=False, dtype="i8", add=False):
    rng = np.random.default_rng([71, M, N, K, seed])
    a, w = rng.integers(-128, 128, (M, K), dtype=np.int8), rng.integers(-128, 128, (K, N), dtype=np.int8)
    rows = np.unique(np.concatenate([np.arange(min(M, 256)), np.arange(max(0, M - 256), M), rng.integers(0, M, 256)]))
    acc = sem.matmul_i8(a[rows].astype(np.int64), w.astype(np.int64), fast=True)
    s = 20
    m = int(min(((1 << 31) - 1 - (1 << (s - 1))) // int(np.abs(acc).max() * 2 + 1), (1 << 23) - 1))
    L = rng.integers(-128, 128, 256) if lut else None
    A, B, lda, ldb, flags = _operands(dev, a, np.ascontiguousarray(w.T), mode, rng)
    c, ldc, cflag, read = _result(dev, M, N, dtype, mode)
    flags |= rt.GEMM_UNCHECKED | rt.GEMM_MUL24 | cflag
    st = [0, 0, lda, 0, 0, ldb, 0, 0, ldc]
    y = sem.qmatmul(a[rows].astype(np.int64), w.astype(np.int64), m, s, L, dtype=dtype, fast=True)
    if add:
        r = rng.integers(-128, 128, (M, N), dtype=np.int8)
        d = dev.alloc(M * N)
        dev.gemm_i8_add(A, B, c, 1, 1, M, N, K, st, m, s, None, up(dev, r), 300, -200, 9, d, [0, 0, N, 0, 0, N], flags)
    else:
        dev.gemm_i8(A, B, c, 1, 1, M, N, K, st, m, s, None if L is None else up(dev, L), dtype, flags)
    dev.sync()
    got = read()[rows].astype(np.int64)
    assert np.array_equal(got, y), (mode, np.argwhere(got != y)[:5])
    if add:
        want = sem.add_requant(r[rows].astype(np.int64), y, 300, -200, 9)
        assert np.array_equal(d.download((M, N), np.int8)[rows].astype(np.int64), want)


# (M, N, K) per kernel family: 128 x 128 tiles with a partial last K block, 256 x 128 (the block's q), the persistent
# 256 x 256 x 64 (fc), 256 x 128 x 128 (proj, ragged rows), 256 x 256 x 128 (config 2), 256 x 192, and split-K
SHAPES = [(300, 200, 80), (32768, 768, 768), (32768, 3072, 768), (32768 + 37, 768, 3072), (16384, 3072, 3072),
          (32768, 1536, 2048), (256, 3072, 3072)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("mode", ["A", "B", "AB", "C", "ABC"])
def test_kblocked_operands_match_the_oracle(dev, M, N, K, mode):
    _check(dev, M, N, K, mode, 0)


@pytest.mark.parametrize("M,N,K", [(32768, 768, 768), (32768 + 37, 768, 3072)])
def test_kblocked_operands_with_the_fused_add(dev, M, N, K):
    """The block's y and proj shapes with their residual add in the epilogue, both operands K-blocked."""
    _check(dev, M, N, K, "AB", 1, add=True)
    _check(dev, M, N, K, "ABC", 4, add=True)          # y stored K-blocked beside the row-major sum


def test_kblocked_operands_lut_and_i16(dev):
    _check(dev, 4096 + 9, 640, 1024 + 16, "AB", 2, lut=True)
    _check(dev, 4096 + 9, 640, 1024 + 16, "AB", 3, dtype="i16")
    _check(dev, 4096 + 9, 640 + 16, 1024 + 16, "ABC", 5, lut=True)
    _check(dev, 4096 + 9, 640 + 16, 1024 + 16, "ABC", 6, dtype="i16")


def test_kblocked_batched_and_grouped(dev):
    """Batch entries each with their own K-blocked A (batch stride past the blocks), and a group call whose members mix
    K-blocked and row-major operands."""
    rng = np.random.default_rng(72)
    nb, M, N, K = 3, 1000, 384, 320
    a = rng.integers(-128, 128, (nb, M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (K, N), dtype=np.int8)
    blocks = [kblock(a[i], 2, rng) for i in range(nb)]
    per, lda = blocks[0][0].size, blocks[0][1]
    A = up(dev, np.concatenate([b.ravel() for b, _ in blocks]))
    bk, ldb = kblock(np.ascontiguousarray(w.T), 0, rng)
    c = dev.alloc(nb * M * N)
    m, s = 3, 16
    dev.gemm_i8(A, up(dev, bk), c, 1, nb, M, N, K, [0, per, lda, 0, 0, ldb, 0, M * N, N], m, s, None, "i8",
                rt.GEMM_UNCHECKED | rt.GEMM_A_KBLOCK | rt.GEMM_B_KBLOCK)
    dev.sync()
    want = sem.qmatmul(a.astype(np.int64), w.astype(np.int64), m, s, fast=True)
    assert np.array_equal(c.download((nb, M, N), np.int8).astype(np.int64), want)

    # a group: K-blocked A with row-major Bt, and row-major A with K-blocked Bt, one launch
    M2 = 24576
    x = rng.integers(-128, 128, (M2, 768), dtype=np.int8)
    ws = [rng.integers(-128, 128, (768, 768), dtype=np.int8) for _ in range(2)]
    xk, ldx = kblock(x, 0, rng)
    X, XK = up(dev, x), up(dev, xk)
    w0 = up(dev, np.ascontiguousarray(ws[0].T))
    w1k, ldw1 = kblock(np.ascontiguousarray(ws[1].T), 0, rng)
    outs = [dev.alloc(M2 * 768) for _ in range(2)]
    f = rt.GEMM_UNCHECKED
    calls = [(XK, w0, outs[0], 1, 1, M2, 768, 768, [0, 0, ldx, 0, 0, 768, 0, 0, 768], 5, 18, None, "i8",
              f | rt.GEMM_A_KBLOCK),
             (X, up(dev, w1k), outs[1], 1, 1, M2, 768, 768, [0, 0, 768, 0, 0, ldw1, 0, 0, 768], 5, 18, None, "i8",
              f | rt.GEMM_B_KBLOCK)]
    dev.gemm_i8_group(calls)
    dev.sync()
    rows = rng.integers(0, M2, 300)
    for o, wi in zip(outs, ws):
        want = sem.qmatmul(x[rows].astype(np.int64), wi.astype(np.int64), 5, 18, fast=True)
        assert np.array_equal(o.download((M2, 768), np.int8)[rows].astype(np.int64), want)


@pytest.mark.parametrize("xdt,d,flags", [("i8", 768, rt.OP_UNCHECKED | rt.RMS_S24), ("i8", 256, rt.OP_UNCHECKED | rt.RMS_S24),
                                         ("i8", 128, rt.OP_UNCHECKED | rt.RMS_S24), ("i8", 64, rt.OP_UNCHECKED | rt.RMS_S24),
                                         ("i8", 320, rt.OP_UNCHECKED | rt.RMS_S24), ("i8", 768, rt.OP_UNCHECKED),
                                         ("i8", 192, 0), ("i16", 64, rt.OP_UNCHECKED), ("i16", 768, rt.OP_UNCHECKED),
                                         ("i16", 128, 0)])
@pytest.mark.parametrize("rows", [203, 8 * 4 * 256 * 4 * 2 + 3])
def test_rmsnorm_kblocked_result(dev, xdt, d, flags, rows):
    """ANVIL_RMS_OUT_KBLOCK on every rmsnorm kernel (16, 8 or 4 lanes a row, four rows a wave, the wide int16 form and
    the checked one): the result K-blocked, block stride rows * 64, equal to the oracle's rows; ragged row counts, and
    more row groups than the grid has waves."""
    from anvil_mi355x import quantize as Q
    rng = np.random.default_rng([73, d, rows, flags])
    w = rng.integers(-127, 128, d)
    if xdt == "i8":
        lut, s = Q.rsqrt_table(0.03, 0.01, 0.02, int(np.abs(w).max()), d, 1e-5)
        c = e = 0
        x = rng.integers(-128, 128, (rows, d))
        want = sem.rmsnorm_int(x, w, lut, 1, s)
    else:
        lut, s, c, e = Q.wide_rsqrt_table(4e-4, 0.01, 0.02, int(np.abs(w).max()), d, 1e-6, 1 << 15)
        x = rng.integers(-(1 << 15), 1 << 15, (rows, d))
        want = sem.rmsnorm_wide(x, w, lut, 1, s, c, e, "i16")
    out = dev.alloc(rows * d)
    dev.rmsnorm_int(up(dev, x, xdt), xdt, up(dev, w), up(dev, lut, "i32"), len(lut), 1, s, c, e, rows, d, out,
                    flags | rt.RMS_OUT_KBLOCK)
    dev.sync()
    got = out.download((d // 64, rows, 64), np.int8).transpose(1, 0, 2).reshape(rows, d).astype(np.int64)
    assert np.array_equal(got, want)
