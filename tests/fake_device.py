"""A CPU stand-in for anvil_mi355x.runtime.Device, for testing the driver's host logic without a GPU.

Test infrastructure only: it emulates each C-ABI call (same arguments: pointers, sizes, element strides) over a
host byte heap, computing with oracle.semantics, so the planner's buffers, views, strides and batch folding are
checked on the CPU exactly as the kernels would read them. The product never uses it.
"""
from __future__ import annotations

import threading

import numpy as np

from anvil_mi355x import runtime as rt
from oracle import semantics as sem

NP = {"i8": np.int8, "i16": np.int16, "i32": np.int32}
SIZE = {"i8": 1, "i16": 2, "i32": 4}
BASE = 1 << 20


class FakeBuffer:
    def __init__(self, dev, nbytes):
        self.dev, self.nbytes = dev, int(nbytes)
        self.ptr = dev._bump(max(1, self.nbytes))
        dev.buffers.append((self.ptr, self.ptr + self.nbytes))

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        raw = arr.view(np.uint8).reshape(-1)
        o = self.ptr - BASE + offset
        self.dev.heap[o:o + raw.size] = raw

    def download(self, shape, dtype, offset=0, into=None):
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        o = self.ptr - BASE + offset
        if into is None:
            return self.dev.heap[o:o + n].copy().view(dtype).reshape(shape)
        out = into.array(dtype, n // np.dtype(dtype).itemsize).reshape(shape)
        out.view(np.uint8).reshape(-1)[:] = self.dev.heap[o:o + n]
        return out


class FakeGraph:
    def __init__(self, fn, args):
        self.fn, self.args, self.launches = fn, args, 0

    def launch(self):
        self.launches += 1
        self.fn(*self.args)


class FakeHostBuffer:
    """Host memory standing in for a page-locked buffer: downloads write into it and views of it are reused."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.mem = np.zeros(max(1, self.nbytes), dtype=np.uint8)

    def array(self, dtype, count):
        return self.mem[:int(count) * np.dtype(dtype).itemsize].view(dtype)

    def free(self):
        pass


class FakeDevice:
    def __init__(self, heap_bytes=1 << 28, fast=False):
        self.fast = fast             # matmuls in float64 BLAS (exact for int8 operands), for large graphs
        self.heap = np.zeros(heap_bytes, dtype=np.uint8)
        self.top = 0
        self.lock = threading.Lock()
        self.calls = []
        self.flags = 0
        self.buffers = []            # (start, end) of every allocation, for the operand-range checks

    def _bump(self, n):
        p = BASE + self.top
        self.top += (n + 255) // 256 * 256
        if self.top > self.heap.size:
            raise MemoryError("fake heap exhausted")
        return p

    def alloc(self, nbytes):
        return FakeBuffer(self, nbytes)

    def capture(self, fn, *args):
        """A stand-in graph: nothing runs at capture, every launch() makes the recorded calls again."""
        self.captures = getattr(self, "captures", 0) + 1
        return FakeGraph(fn, args)

    def host_alloc(self, nbytes):
        self.host_allocs = getattr(self, "host_allocs", 0) + 1
        return FakeHostBuffer(nbytes)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        b = FakeBuffer(self, arr.nbytes)
        b.upload(arr)
        return b

    def view(self, ptr, dtype, dims, strides):
        ptr = ptr.ptr if hasattr(ptr, "ptr") else int(ptr)
        it = SIZE[dtype]
        base = self.heap[ptr - BASE:].view(np.uint8)
        arr = base[: (len(base) // it) * it].view(NP[dtype])
        return np.lib.stride_tricks.as_strided(arr, shape=tuple(dims), strides=tuple(s * it for s in strides))

    def store(self, ptr, dtype, dims, strides, values):
        self.view(ptr, dtype, dims, strides)[...] = np.asarray(values).astype(NP[dtype])

    def sync(self):
        f, self.flags = self.flags, 0
        if f:
            raise f

    def record(self, slot):
        pass

    def timed(self, slot0, slot1, fn, *args):
        self.record(slot0)
        fn(*args)
        self.record(slot1)

    def elapsed_ms(self, a, b):
        return 0.0

    def _guard(self, fn):
        try:
            return fn()
        except (OverflowError, ValueError, ZeroDivisionError) as e:
            self.flags = type(e)
            return None

    # ---------------------------------------------------------------------------------------------- ops
    def _in_one_buffer(self, ptr, nbytes, what):
        """The kernels' buffer resource of a GEMM operand spans [ptr, ptr + nbytes): from the first row's base to the
        last row's K-th byte (row-major) or the last K block's last row (K-blocked). Loads anywhere inside it must
        stay inside the allocation the operand lives in, as the kernels read stages past K within that range."""
        ptr = ptr.ptr if hasattr(ptr, "ptr") else int(ptr)
        assert any(s <= ptr and ptr + nbytes <= e for s, e in self.buffers), \
            f"{what}: operand range [{ptr:#x}, {ptr + nbytes:#x}) leaves its allocation"

    def _check_operands(self, A, Bt, b0, b1, M, N, K, strides, flags):
        self._in_one_buffer(A, 1 + self._operand_end((b0, b1, M), strides[0:3], flags & rt.GEMM_A_KBLOCK, K), "A")
        self._in_one_buffer(Bt, 1 + self._operand_end((b0, b1, N), strides[3:6], flags & rt.GEMM_B_KBLOCK, K), "Bt")

    def gemm_i8(self, A, Bt, Cp, b0, b1, M, N, K, strides, mult, shift, lut, out_dtype, flags=0):
        """Every output is computed, also under the causal flags (a superset of what the kernel writes)."""
        self.calls.append(("gemm", b0, b1, M, N, K, tuple(strides), flags))
        self._check_operands(A, Bt, b0, b1, M, N, K, strides, flags)
        sa0, sa1, lda, sb0, sb1, ldb, sc0, sc1, ldc = strides
        a = self._operand(A, b0, b1, M, K, sa0, sa1, lda, flags & rt.GEMM_A_KBLOCK)
        bt = self._operand(Bt, b0, b1, N, K, sb0, sb1, ldb, flags & rt.GEMM_B_KBLOCK)
        lt = None if lut is None else self.view(lut, "i8", (256,), (1,)).astype(np.int64)
        out = self._guard(lambda: sem.qmatmul(a, np.swapaxes(bt, -1, -2), mult, shift, lt, out_dtype,
                                                      fast=self.fast))
        if out is not None:
            self._store_result(Cp, out_dtype, b0, b1, M, N, (sc0, sc1, ldc), flags & rt.GEMM_C_KBLOCK, out)

    def _operand(self, ptr, b0, b1, rows, K, s0, s1, ld, kblocked):
        """A GEMM operand (b0, b1, rows, K): row-major rows of stride ld, or K-blocked (row r's 64-byte K block j at
        r 64 + j ld, as ANVIL_GEMM_A_KBLOCK / B_KBLOCK describe)."""
        if not kblocked:
            return self.view(ptr, "i8", (b0, b1, rows, K), (s0, s1, ld, 1)).astype(np.int64)
        nb = -(-K // 64)
        v = self.view(ptr, "i8", (b0, b1, rows, nb, 64), (s0, s1, 64, ld, 1)).astype(np.int64)
        return v.reshape(b0, b1, rows, nb * 64)[..., :K]

    def _store_result(self, ptr, dtype, b0, b1, M, N, strides, kblocked, values):
        """A GEMM result (b0, b1, M, N): row-major, or K-blocked (ANVIL_GEMM_C_KBLOCK: (m, n) at m 64 + (n // 64) ld +
        n % 64; N a multiple of 64 here)."""
        s0, s1, ld = strides
        if not kblocked:
            self.store(ptr, dtype, (b0, b1, M, N), (s0, s1, ld, 1), values)
            return
        assert N % 64 == 0
        self.store(ptr, dtype, (b0, b1, M, N // 64, 64), (s0, s1, 64, ld, 1),
                   np.asarray(values).reshape(b0, b1, M, N // 64, 64))

    @staticmethod
    def _operand_end(dims, strides, kblocked, K):
        """Offset of the last byte an operand (b0, b1, rows, K) covers."""
        b0, b1, rows = dims
        s0, s1, ld = strides
        if not kblocked:
            return (b0 - 1) * s0 + (b1 - 1) * s1 + (rows - 1) * ld + K - 1
        return (b0 - 1) * s0 + (b1 - 1) * s1 + (rows - 1) * 64 + (-(-K // 64) - 1) * ld + 63

    def gemm_i8_group(self, calls):
        """Members run one after another; none may write bytes another member reads or writes."""
        self.calls.append(("gemm_group", len(calls)))
        assert 1 <= len(calls) <= 4

        def span(ptr, dtype, dims, strides):
            p = ptr.ptr if hasattr(ptr, "ptr") else int(ptr)
            last = sum((d - 1) * s for d, s in zip(dims, strides))
            return p, p + (last + 1) * SIZE[dtype]

        reads, writes = [], []
        for A, Bt, Cp, b0, b1, M, N, K, st, _, _, lut, dt, fl in calls:
            pa, pb = (x.ptr if hasattr(x, "ptr") else int(x) for x in (A, Bt))
            r = [(pa, pa + 1 + self._operand_end((b0, b1, M), st[0:3], fl & rt.GEMM_A_KBLOCK, K)),
                 (pb, pb + 1 + self._operand_end((b0, b1, N), st[3:6], fl & rt.GEMM_B_KBLOCK, K))]
            if lut is not None:
                r.append(span(lut, "i8", (256,), (1,)))
            reads.append(r)
            pc = Cp.ptr if hasattr(Cp, "ptr") else int(Cp)
            end = self._operand_end((b0, b1, M), st[6:9], fl & rt.GEMM_C_KBLOCK, N)
            writes.append((pc, pc + (end + 1) * SIZE[dt]))
        hit = lambda x, y: x[0] < y[1] and y[0] < x[1]                       # noqa: E731
        for i, w in enumerate(writes):
            for j in range(len(calls)):
                if j != i:
                    assert not hit(w, writes[j]) and not any(hit(w, r) for r in reads[j]), (i, j)
        for c in calls:
            self.gemm_i8(*c)

    def gemm_i8_add(self, A, Bt, Cp, b0, b1, M, N, K, strides, mult, shift, lut, R, ma, mb, shift2, D, rstrides,
                    flags, out_dtype="i8"):
        """y = qmatmul epilogue, D = add_requant of the residual R (times ma) and y (times mb); y, R, D out_dtype."""
        dt = out_dtype
        self.calls.append(("gemm_add", b0, b1, M, N, K, tuple(strides), flags, Cp is not None, dt))
        self._check_operands(A, Bt, b0, b1, M, N, K, strides, flags)
        sa0, sa1, lda, sb0, sb1, ldb, sc0, sc1, ldc = strides
        sr0, sr1, ldr, sd0, sd1, ldd = rstrides
        a = self._operand(A, b0, b1, M, K, sa0, sa1, lda, flags & rt.GEMM_A_KBLOCK)
        bt = self._operand(Bt, b0, b1, N, K, sb0, sb1, ldb, flags & rt.GEMM_B_KBLOCK)
        lt = None if lut is None else self.view(lut, "i8", (256,), (1,)).astype(np.int64)
        r = self.view(R, dt, (b0, b1, M, N), (sr0, sr1, ldr, 1)).astype(np.int64)

        def both():
            y = sem.qmatmul(a, np.swapaxes(bt, -1, -2), mult, shift, lt, dt, fast=self.fast)
            return y, sem.add_requant(r, y, ma, mb, shift2, dt)
        out = self._guard(both)
        if out is not None:
            if Cp is not None:
                self._store_result(Cp, dt, b0, b1, M, N, (sc0, sc1, ldc), flags & rt.GEMM_C_KBLOCK, out[0])
            self.store(D, dt, (b0, b1, M, N), (sd0, sd1, ldd, 1), out[1])

    def gemm_i8_add_norm(self, A, Bt, Cp, M, N, K, strides, mult, shift, lut, R, ma, mb, shift2, D, rstrides, nw, nlut,
                         nlut_len, nmult, nshift, H, ld, kb, flags):
        """gemm_i8_add (batch 1, int8), then H = rmsnorm_int(D): the preconditions of the fused entry point, then the
        three ops."""
        self.calls.append(("gemm_add_norm", M, N, K, tuple(strides), flags, Cp is not None, ld, kb))
        assert N in (128, 256) and M % 128 == 0 and flags & rt.GEMM_NORM_S24 and flags & rt.GEMM_UNCHECKED
        assert max(abs(ma), abs(mb)) < 1 << 24 and (ld == 64 if kb else ld >= N)
        self.gemm_i8_add(A, Bt, Cp, 1, 1, M, N, K, strides, mult, shift, lut, R, ma, mb, shift2, D, rstrides,
                         flags & ~rt.GEMM_NORM_S24)
        d = self.view(D, "i8", (M, N), (rstrides[5], 1)).astype(np.int64)
        w = self.view(nw, "i8", (N,), (1,)).astype(np.int64)
        lt = self.view(nlut, "i32", (nlut_len,), (1,)).astype(np.int64)
        assert int(np.abs(lt).max()) * abs(nmult) < 1 << 23
        h = self._guard(lambda: sem.rmsnorm_int(d, w, lt, nmult, nshift))
        if h is not None:
            self._store_result(H, "i8", 1, 1, M, N, (0, 0, kb if kb else ld), bool(kb), h.reshape(1, 1, M, N))

    def _vt(self, Vt, b0, b1, T, D, st, flags):
        """The attention's V^T operand: given as V^T rows, or (ATTN_V_ROWS, T = 16 only) as V's own rows."""
        if flags & rt.ATTN_V_ROWS:
            assert T == 16, "V rows are for the T = 16 kernel"
            v = self.view(Vt, "i8", (b0, b1, T, D), (st[6], st[7], st[8], 1)).astype(np.int64)
            return np.swapaxes(v, -1, -2)
        return self.view(Vt, "i8", (b0, b1, D, T), (st[6], st[7], st[8], 1)).astype(np.int64)

    def attention_i8(self, Q, K, Vt, O, b0, b1, T, D, strides, ms, ss, lut, one, causal, mo, so, flags):
        """The three ops the fused kernel replaces, over the same strided operands."""
        self.calls.append(("attention", b0, b1, T, D, tuple(strides), flags))
        st = strides
        q = self.view(Q, "i8", (b0, b1, T, D), (st[0], st[1], st[2], 1)).astype(np.int64)
        k = self.view(K, "i8", (b0, b1, T, D), (st[3], st[4], st[5], 1)).astype(np.int64)
        vt = self._vt(Vt, b0, b1, T, D, st, flags)
        lv = self.view(lut, "i32", (256,), (1,)).astype(np.int64)

        def chain():
            scores = sem.qmatmul(q, np.swapaxes(k, -1, -2), ms, ss, fast=self.fast)
            p = sem.softmax_lut(scores, lv, one, causal)
            return sem.qmatmul(p, np.swapaxes(vt, -1, -2), mo, so, fast=self.fast)
        r = self._guard(chain)
        if r is not None:
            self.store(O, "i8", (b0, b1, T, D), (st[9], st[10], st[11], 1), r)

    def attention_i8_keep(self, Q, K, Vt, O, S, P, b0, b1, T, D, strides, ms, ss, lut, one, causal, mo, so, flags):
        """attention_i8 that also stores the scores and the probabilities (strides 12..17)."""
        self.calls.append(("attention_keep", b0, b1, T, D, tuple(strides), flags))
        st = strides
        q = self.view(Q, "i8", (b0, b1, T, D), (st[0], st[1], st[2], 1)).astype(np.int64)
        k = self.view(K, "i8", (b0, b1, T, D), (st[3], st[4], st[5], 1)).astype(np.int64)
        vt = self._vt(Vt, b0, b1, T, D, st, flags)
        lv = self.view(lut, "i32", (256,), (1,)).astype(np.int64)

        def chain():
            scores = sem.qmatmul(q, np.swapaxes(k, -1, -2), ms, ss, fast=self.fast)
            p = sem.softmax_lut(scores, lv, one, causal)
            return scores, p, sem.qmatmul(p, np.swapaxes(vt, -1, -2), mo, so, fast=self.fast)
        r = self._guard(chain)
        if r is not None:
            self.store(S, "i8", (b0, b1, T, T), (st[12], st[13], st[14], 1), r[0])
            self.store(P, "i8", (b0, b1, T, T), (st[15], st[16], st[17], 1), r[1])
            self.store(O, "i8", (b0, b1, T, D), (st[9], st[10], st[11], 1), r[2])

    def rmsnorm_int(self, x, x_dtype, w, lut, lut_len, mult, shift, ss_shift, ss_init, rows, cols, out, flags=0):
        self.calls.append(("rmsnorm", rows, cols, flags))
        xv = self.view(x, x_dtype, (rows, cols), (cols, 1)).astype(np.int64)
        wv = self.view(w, "i8", (cols,), (1,)).astype(np.int64)
        lv = self.view(lut, "i32", (lut_len,), (1,)).astype(np.int64)
        r = self._guard(lambda: sem.rmsnorm_wide(xv, wv, lv, mult, shift, ss_shift, ss_init, x_dtype))
        if r is not None and flags & rt.RMS_OUT_KBLOCK:        # K-blocked: [cols // 64][rows][64]
            self.store(out, "i8", (rows, cols // 64, 64), (64, rows * 64, 1), r.reshape(rows, cols // 64, 64))
        elif r is not None:
            self.store(out, "i8", (rows, cols), (cols, 1), r)

    def softmax_lut(self, x, lut, one, causal, batch, t1, t2, out, out_dtype, flags=0):
        self.calls.append(("softmax", batch, t1, t2, flags))
        xv = self.view(x, "i8", (batch, t1, t2), (t1 * t2, t2, 1)).astype(np.int64)
        lv = self.view(lut, "i32", (256,), (1,)).astype(np.int64)
        r = self._guard(lambda: sem.softmax_lut(xv, lv, one, causal))
        if r is not None:
            self.store(out, out_dtype, (batch, t1, t2), (t1 * t2, t2, 1), r)

    def add_requant(self, a, a_dtype, b, b_dtype, ma, mb, shift, n, out, out_dtype, flags=0):
        self.calls.append(("add", n, flags))
        av = self.view(a, a_dtype, (n,), (1,)).astype(np.int64)
        bv = self.view(b, b_dtype, (n,), (1,)).astype(np.int64)
        r = self._guard(lambda: sem.add_requant(av, bv, ma, mb, shift, out_dtype))
        if r is not None:
            self.store(out, out_dtype, (n,), (1,), r)

    def lut_i8(self, x, table, n, out):
        self.calls.append(("lut", n))
        r = sem.lut_i8(self.view(x, "i8", (n,), (1,)).astype(np.int64), self.view(table, "i8", (256,), (1,)))
        self.store(out, "i8", (n,), (1,), r)

    def lut_mul(self, x, y, table, mult, shift, n, out, flags=0):
        self.calls.append(("lut_mul", n, flags))
        xv = self.view(x, "i8", (n,), (1,)).astype(np.int64)
        yv = self.view(y, "i8", (n,), (1,)).astype(np.int64)
        tv = self.view(table, "i8", (256,), (1,)).astype(np.int64)
        r = self._guard(lambda: sem.swiglu_lut(xv, yv, tv, mult, shift))
        if r is not None:
            self.store(out, "i8", (n,), (1,), r)

    def copy_strided(self, src, dst, elem_size, dims, src_strides):
        self.calls.append(("copy", tuple(dims)))
        dt = {1: "i8", 2: "i16", 4: "i32"}[elem_size]
        v = self.view(src, dt, dims, src_strides).copy()
        self.store(dst, dt, dims, [int(np.prod(dims[i + 1:])) for i in range(len(dims))], v)

    def _raw(self, ptr, dtype, n):
        ptr = ptr.ptr if hasattr(ptr, "ptr") else int(ptr)
        return self.heap[ptr - BASE:ptr - BASE + n * np.dtype(dtype).itemsize].view(dtype)

    def quantize(self, x, x_is_f64, scale, n, out, out_dtype):
        """clamp(rint(float64(x) / scale)), as the host's quantize_input."""
        self.calls.append(("quantize", n, bool(x_is_f64)))
        v = self._raw(x, np.float64 if x_is_f64 else np.float32, n).astype(np.float64)
        lo, hi = {"i8": (-128, 127), "i16": (-32768, 32767)}[out_dtype]
        fin = np.isfinite(v)
        if not fin.all():                                # the kernel's flag: the next sync raises
            self.flags = self.flags or ValueError("a float input holds NaN or infinite values")
        self.store(out, out_dtype, (n,), (1,), np.where(fin, np.clip(np.rint(np.where(fin, v, 0) / scale), lo, hi), 0))

    def embed_quantize(self, ids, rows, T, Cdim, wte, vocab, wpe, scale, out, out_dtype):
        self.calls.append(("embed", rows, T, Cdim))
        idv = self._raw(ids, np.int64, rows)
        if idv.size and (idv.min() < 0 or idv.max() >= vocab):
            self.flags = ValueError
            return
        te = self._raw(wte, np.float32, vocab * Cdim).reshape(vocab, Cdim).astype(np.float64)
        pe = self._raw(wpe, np.float32, T * Cdim).reshape(T, Cdim).astype(np.float64)
        x = te[idv] + pe[np.arange(rows) % T]
        lo, hi = {"i8": (-128, 127), "i16": (-32768, 32767)}[out_dtype]
        self.store(out, out_dtype, (rows * Cdim,), (1,), np.clip(np.rint(x / scale), lo, hi).reshape(-1))
