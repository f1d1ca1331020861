"""anvil_gemm_i8_noalloc: the allocation-free variant of anvil_gemm_i8_ex (its split-K partial sums live in the
library's static per-device scratch instead of a workspace the context allocates). Called through the C ABI and
compared with anvil_gemm_i8_ex on the same inputs, bit for bit, on two calls in a row, the second one smaller."""
import ctypes as C

import numpy as np
import pytest

from anvil_mi355x import quantize as Q
from anvil_mi355x import runtime as rt
from oracle import semantics as sem

pytestmark = pytest.mark.gpu

@pytest.fixture(scope="module")
def dev():
    return rt.device(0)


def _inputs(M, K, N, seed):
    rng = np.random.default_rng([53, M, K, N, seed])
    a = rng.integers(-128, 128, (M, K))
    w = rng.integers(-128, 128, (K, N))
    acc = sem.matmul_i8(a, w, fast=True)
    (m,), s = Q.choose_shift([127 / (1.5 * max(1, int(np.abs(acc).max())))], [128 * int(np.abs(w).sum(axis=0).max())])
    return a, w, m, s


def _both(dev, a, w, m, s, flags):
    """(anvil_gemm_i8_ex result, anvil_gemm_i8_noalloc result) of one product."""
    M, K = a.shape
    N = w.shape[1]
    A = dev.upload(np.ascontiguousarray(a).astype(np.int8))
    Bt = dev.upload(np.ascontiguousarray(w.T).astype(np.int8))
    C1, C2 = dev.alloc(M * N), dev.alloc(M * N)
    strides = [0, 0, K, 0, 0, K, 0, 0, N]
    dev.gemm_i8(A, Bt, C1, 1, 1, M, N, K, strides, m, s, None, "i8", flags)
    st = (C.c_int64 * 9)(*strides)
    dev.lib.call("anvil_gemm_i8_noalloc", dev.ctx, C.c_void_p(A.ptr), C.c_void_p(Bt.ptr), C.c_void_p(C2.ptr), 1, 1,
                 M, N, K, st, int(m), s, None, rt.I8, flags)
    dev.sync()
    return C1.download((M, N), np.int8), C2.download((M, N), np.int8)


def _workspace_sums(d) -> int:
    out = C.c_longlong(-1)
    d.lib.call("anvil_workspace_sums", d.ctx, C.byref(out))
    return int(out.value)


def test_noalloc_split_allocates_no_workspace_and_keeps_the_scratch_to_one_context():
    """A fresh context that has never split K runs a split-K product through anvil_gemm_i8_noalloc: its workspace
    stays empty (nothing allocated), while anvil_gemm_i8_ex on the same product then allocates one. Until that
    context is destroyed, a second context's split into the device's scratch is refused rather than racing. (First
    in this file: the shared context of the tests below claims the scratch for the rest of the process.)"""
    first = rt.Device(0)
    second = rt.Device(0)
    try:
        a, w, m, s = _inputs(256, 3072, 3072, 2)
        M, K = a.shape
        N = w.shape[1]
        A = first.upload(np.ascontiguousarray(a).astype(np.int8))
        Bt = first.upload(np.ascontiguousarray(w.T).astype(np.int8))
        C1, C2 = first.alloc(M * N), first.alloc(M * N)
        strides = [0, 0, K, 0, 0, K, 0, 0, N]
        flags = rt.GEMM_UNCHECKED | rt.GEMM_SPLITK
        assert _workspace_sums(first) == 0
        first.gemm_i8_noalloc(A, Bt, C2, 1, 1, M, N, K, strides, m, s, None, "i8", flags)
        first.sync()
        assert _workspace_sums(first) == 0
        with pytest.raises(RuntimeError, match="belongs to another context"):
            second.gemm_i8_noalloc(A, Bt, C1, 1, 1, M, N, K, strides, m, s, None, "i8", flags)
        first.gemm_i8(A, Bt, C1, 1, 1, M, N, K, strides, m, s, None, "i8", flags)
        first.sync()
        assert _workspace_sums(first) > 0
        assert np.array_equal(C1.download((M, N), np.int8), C2.download((M, N), np.int8))
        for buf in (A, Bt, C1, C2):
            buf.free()
        first.close()
        # the scratch is free again once its holder is destroyed
        A = second.upload(np.ascontiguousarray(a).astype(np.int8))
        Bt = second.upload(np.ascontiguousarray(w.T).astype(np.int8))
        C3 = second.alloc(M * N)
        second.gemm_i8_noalloc(A, Bt, C3, 1, 1, M, N, K, strides, m, s, None, "i8", flags)
        second.sync()
        assert np.array_equal(C3.download((M, N), np.int8).astype(np.int64), sem.qmatmul(a, w, m, s, fast=True))
        for buf in (A, Bt, C3):
            buf.free()
    finally:
        first.close()
        second.close()


CASES = [  # (first shape, second smaller shape, flags): split-K by the library's choice, forced, and one-pass
    ((256, 3072, 3072), (256, 768, 768), rt.GEMM_UNCHECKED),
    ((640, 2048, 1024), (100, 512, 48), rt.GEMM_UNCHECKED | rt.GEMM_SPLITK),
    ((4096, 768, 768), (1000, 256, 300), rt.GEMM_UNCHECKED),
]


@pytest.mark.parametrize("first,second,flags", CASES)
def test_noalloc_matches_the_allocating_entry_point(dev, first, second, flags):
    for shape, seed in ((first, 0), (second, 1)):
        a, w, m, s = _inputs(*shape, seed)
        want = sem.qmatmul(a, w, m, s, fast=True)
        got_ex, got_static = _both(dev, a, w, m, s, flags)
        assert np.array_equal(got_static, got_ex), (shape, flags)
        assert np.array_equal(got_static.astype(np.int64), want), (shape, flags)


def test_noalloc_rejects_a_split_beyond_the_static_scratch(dev):
    """256 tiles of 128 x 128 in two K chunks = 2^23 partial sums > the 2^22 the static scratch holds: a clear
    ValueError before any launch."""
    M = N = 2048
    st = (C.c_int64 * 9)(0, 0, 512, 0, 0, 512, 0, 0, N)
    A, Bt, Cb = dev.alloc(M * 512), dev.alloc(N * 512), dev.alloc(M * N)
    with pytest.raises(ValueError, match="exceeds the static scratch"):
        dev.lib.call("anvil_gemm_i8_noalloc", dev.ctx, C.c_void_p(A.ptr), C.c_void_p(Bt.ptr), C.c_void_p(Cb.ptr),
                     1, 1, M, N, 512, st, 1, 20, None, rt.I8, rt.GEMM_UNCHECKED | rt.GEMM_SPLITK)
    dev.sync()
