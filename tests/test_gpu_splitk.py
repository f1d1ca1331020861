"""Split-K GEMMs (ANVIL_GEMM_SPLITK, and the library's own choice for few-tile products) against the oracle and the
one-pass kernels: same bits, on ragged shapes, i16 results, LUT epilogues and the 24-bit requant, run repeatedly so
that a workspace left dirty by one call would show up in the next (reference op: anvil/semantics.py:95-103)."""
import numpy as np
import pytest

from anvil_mi355x import quantize as Q
from anvil_mi355x import runtime as rt
from oracle import semantics as sem

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return rt.device(0)


def _case(M, K, N, seed, dtype="i8", lut=False):
    rng = np.random.default_rng([41, M, K, N, seed])
    a = rng.integers(-128, 128, (M, K))
    w = rng.integers(-128, 128, (K, N))
    acc = sem.matmul_i8(a, w, fast=True)
    target = 127 if dtype == "i8" else 20000
    (m,), s = Q.choose_shift([target / (1.5 * max(1, int(np.abs(acc).max())))],
                             [128 * int(np.abs(w).sum(axis=0).max())])
    table = rng.integers(-128, 128, 256) if lut else None
    want = sem.qmatmul(a, w, m, s, table, dtype, fast=True)
    return a, w, m, s, table, want, int(np.abs(acc).max())


def _run(dev, a, w, m, s, table, dtype, flags):
    M, K = a.shape
    N = w.shape[1]
    up = lambda x, dt: dev.upload(np.ascontiguousarray(x).astype(rt.NP_DTYPE[dt]))   # noqa: E731
    A, Bt = up(a, "i8"), up(w.T, "i8")
    L = None if table is None else up(table, "i8")
    Cb = dev.alloc(M * N * rt.ITEMSIZE[dtype])
    dev.gemm_i8(A, Bt, Cb, 1, 1, M, N, K, [0, 0, K, 0, 0, K, 0, 0, N], m, s, L, dtype, flags)
    dev.sync()
    return Cb.download((M, N), rt.NP_DTYPE[dtype]).astype(np.int64)


SHAPES = [(256, 768, 768), (256, 3072, 3072), (300, 1024, 200), (33, 48, 72), (1000, 4096, 130), (128, 3072, 2048),
          (1, 512, 16), (129, 640, 129)]


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("dtype,lut", [("i8", False), ("i8", True), ("i16", False)])
def test_forced_split_k_matches_oracle_and_one_pass(dev, M, K, N, dtype, lut):
    for seed in range(2):                                     # a second call on a workspace the first one used
        a, w, m, s, table, want, amax = _case(M, K, N, seed, dtype, lut)
        flags = rt.GEMM_UNCHECKED | rt.GEMM_SPLITK
        if amax < (1 << 23) and m < (1 << 23):
            flags |= rt.GEMM_MUL24
        got = _run(dev, a, w, m, s, table, dtype, flags)
        assert np.array_equal(got, want), (M, K, N, dtype, lut, seed, int((got != want).sum()))
        one = _run(dev, a, w, m, s, table, dtype, flags & ~rt.GEMM_SPLITK)
        assert np.array_equal(one, got)


def test_few_tile_products_repeat_exactly(dev):
    """The config-2 shape 256 x 3072 x 3072 takes split-K by itself (256 x 768 x 768 does not); ten calls in a row
    give the same bits."""
    for K in (768, 3072):
        a, w, m, s, table, want, _ = _case(256, K, K, 7)
        for _ in range(10):
            assert np.array_equal(_run(dev, a, w, m, s, None, "i8", rt.GEMM_UNCHECKED), want)
