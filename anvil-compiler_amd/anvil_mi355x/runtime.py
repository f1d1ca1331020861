"""ctypes binding of libanvil_mi355x.so (the C ABI in include/anvil_mi355x.h) and device-memory handles.

    lib = runtime.library()                   # loads the in-tree .so; raises if it is missing or stale
    dev = runtime.Device(0)                   # anvil_init: a context with its own stream on device 0
    buf = dev.alloc(nbytes); buf.upload(arr); buf.download(shape, np.int8)
    dev.sync()                                # raises OverflowError / ValueError / ZeroDivisionError found on device

Status codes map to the exceptions the reference interpreter raises for the same condition
(anvil/semantics.py: OverflowError for int32 overflow, ValueError for range / shift errors, ZeroDivisionError for a
softmax row summing to zero). There is no CPU fallback: without the library every device call raises.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import threading
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libanvil_mi355x.so"

I8, I16, I32 = 1, 2, 4
DTYPE_CODE = {"i8": I8, "i16": I16, "i32": I32}
NP_DTYPE = {"i8": np.int8, "i16": np.int16, "i32": np.int32}
ITEMSIZE = {"i8": 1, "i16": 2, "i32": 4}

_ERRORS = {1: ValueError, 2: OverflowError, 3: ZeroDivisionError, 4: RuntimeError}

# anvil_gemm_i8_ex flags (include/anvil_mi355x.h)
GEMM_UNCHECKED, GEMM_CAUSAL_SKIP, GEMM_CAUSAL_K, GEMM_MUL24, GEMM_SPLITK = 1, 2, 4, 8, 16
GEMM_A_KBLOCK, GEMM_B_KBLOCK, GEMM_C_KBLOCK = 32, 64, 128
GEMM_NORM_S24 = 256                          # anvil_gemm_i8_add_norm: |rsqrt table entry x mult| < 2^23
# anvil_rmsnorm_int_ex / anvil_softmax_lut_ex / anvil_attention_i8 flags
OP_UNCHECKED, ATTN_S24, RMS_S24, RMS_OUT_KBLOCK, ATTN_V_ROWS = 1, 2, 2, 4, 4

_p, _i, _i64, _i32, _sz, _f64 = C.c_void_p, C.c_int, C.c_int64, C.c_int32, C.c_size_t, C.c_double
# symbol -> argtypes (restype int for all but anvil_last_error), in include/anvil_mi355x.h order
SIGNATURES = {
    "anvil_last_error": None,
    "anvil_version": [],
    "anvil_init": [_i, C.POINTER(_p)],
    "anvil_destroy": [_p],
    "anvil_sync": [_p],
    "anvil_alloc": [_p, _sz, C.POINTER(_p)],
    "anvil_free": [_p, _p],
    "anvil_host_alloc": [_p, _sz, C.POINTER(_p)],
    "anvil_host_free": [_p, _p],
    "anvil_upload": [_p, _p, _p, _sz],
    "anvil_download": [_p, _p, _p, _sz],
    "anvil_zero": [_p, _p, _sz],
    "anvil_graph_begin": [_p],
    "anvil_graph_end": [_p, C.POINTER(_p)],
    "anvil_graph_launch": [_p, _p],
    "anvil_graph_destroy": [_p, _p],
    "anvil_event_record": [_p, _i],
    "anvil_event_elapsed": [_p, _i, _i, C.POINTER(C.c_float)],
    "anvil_time_kernels": [_p, _i, _i],
    "anvil_gemm_i8": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i32, _i, _p, _i],
    "anvil_gemm_i8_ex": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i32, _i, _p, _i, _i],
    "anvil_gemm_i8_noalloc": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i32, _i, _p, _i, _i],
    "anvil_workspace_sums": [_p, C.POINTER(C.c_longlong)],
    "anvil_gemm_i8_group": [_p, _p, _i],
    "anvil_gemm_i8_add": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i32, _i, _p, _p, _i32, _i32, _i, _p, _p, _i],
    "anvil_gemm_i8_add_ex": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i32, _i, _p, _i, _p, _i32, _i32, _i, _p, _p,
                             _i],
    "anvil_gemm_i8_add_norm": [_p, _p, _p, _p, _i, _i, _i, _p, _i32, _i, _p, _p, _i32, _i32, _i, _p, _p, _p, _i],
    "anvil_rmsnorm_int": [_p, _p, _i, _p, _p, _i, _i32, _i, _i, _i32, _i64, _i, _p],
    "anvil_rmsnorm_int_ex": [_p, _p, _i, _p, _p, _i, _i32, _i, _i, _i32, _i64, _i, _p, _i],
    "anvil_softmax_lut": [_p, _p, _p, _i32, _i, _i64, _i, _i, _p, _i],
    "anvil_softmax_lut_ex": [_p, _p, _p, _i32, _i, _i64, _i, _i, _p, _i, _i],
    "anvil_attention_i8": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p, _i32, _i, _p, _i32, _i, _i32, _i, _i],
    "anvil_attention_i8_keep": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p, _i32, _i, _p, _i32, _i, _i32, _i, _i],
    "anvil_add_requant": [_p, _p, _i, _p, _i, _i32, _i32, _i, _i64, _p, _i],
    "anvil_add_requant_ex": [_p, _p, _i, _p, _i, _i32, _i32, _i, _i64, _p, _i, _i],
    "anvil_lut_i8": [_p, _p, _p, _i64, _p],
    "anvil_lut_mul": [_p, _p, _p, _p, _i32, _i, _i64, _p],
    "anvil_lut_mul_ex": [_p, _p, _p, _p, _i32, _i, _i64, _p, _i],
    "anvil_copy_strided": [_p, _p, _p, _i, _i, _p, _p],
    "anvil_quantize": [_p, _p, _i, _f64, _i64, _p, _i],
    "anvil_embed_quantize": [_p, _p, _i64, _i, _i, _p, _i, _p, _f64, _p, _i],
}



class GemmDesc(C.Structure):
    """anvil_gemm_desc: the arguments of one anvil_gemm_i8_ex call."""
    _fields_ = [("A", _p), ("Bt", _p), ("C", _p), ("lut", _p), ("strides", _i64 * 9), ("batch0", _i32),
                ("batch1", _i32), ("M", _i32), ("N", _i32), ("K", _i32), ("mult", _i32), ("shift", _i32),
                ("out_dtype", _i32), ("flags", _i32)]


class NormEpilogue(C.Structure):
    """anvil_norm_epilogue: the rmsnorm fused after anvil_gemm_i8_add_norm's add."""
    _fields_ = [("w", _p), ("lut", _p), ("lut_len", _i32), ("mult", _i32), ("shift", _i32), ("out", _p),
                ("ld", _i64), ("kb", _i64)]


GEMM_GROUP_MAX = 4
_lib = None
_lock = threading.Lock()


class Library:
    def __init__(self, path: Path):
        if not path.exists():
            raise RuntimeError(f"{path} is missing: build it first (python -m anvil_mi355x.build, or "
                               "__graft_entry__.build())")
        self.path = path
        self.cdll = C.CDLL(str(path))
        for name, args in SIGNATURES.items():
            fn = getattr(self.cdll, name)
            if args is None:
                fn.restype, fn.argtypes = C.c_char_p, []
            else:
                fn.restype, fn.argtypes = C.c_int, args
        self.last_error = self.cdll.anvil_last_error

    def call(self, name, *args):
        rc = getattr(self.cdll, name)(*args)
        if rc:
            msg = self.last_error().decode(errors="replace")
            raise _ERRORS.get(rc, RuntimeError)(f"{name}: {msg}")
        return rc


def library() -> Library:
    """The process-wide handle on the in-tree libanvil_mi355x.so (ANVIL_MI355X_LIB overrides the path)."""
    global _lib
    with _lock:
        if _lib is None:
            _lib = Library(Path(os.environ.get("ANVIL_MI355X_LIB", LIB_PATH)))
        return _lib


def _ptr(x) -> int:
    return x.ptr if isinstance(x, DeviceBuffer) else int(x)


class DeviceBuffer:
    """A device allocation owned by a Device; freed when collected."""

    def __init__(self, dev: "Device", nbytes: int):
        self.dev, self.nbytes = dev, int(nbytes)
        out = C.c_void_p()
        dev.lib.call("anvil_alloc", dev.ctx, C.c_size_t(max(1, self.nbytes)), C.byref(out))
        self.ptr = int(out.value)

    def upload(self, arr: np.ndarray, offset: int = 0):
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError(f"upload of {arr.nbytes} bytes at {offset} overruns a {self.nbytes}-byte buffer")
        self.dev.lib.call("anvil_upload", self.dev.ctx, C.c_void_p(self.ptr + offset), arr.ctypes.data_as(C.c_void_p),
                          C.c_size_t(arr.nbytes))

    def download(self, shape, dtype, offset: int = 0, into: "HostBuffer | None" = None) -> np.ndarray:
        """The buffer's bytes from `offset` as an array of `shape` and `dtype`: a new array, or with `into` a view of
        that page-locked buffer (valid until its next use)."""
        count = math.prod(shape) if isinstance(shape, tuple) else int(shape)
        nbytes = count * np.dtype(dtype).itemsize
        if offset + nbytes > self.nbytes:
            raise ValueError(f"download of {nbytes} bytes at {offset} overruns a {self.nbytes}-byte buffer")
        out = np.empty(shape, dtype=dtype) if into is None else into.array(dtype, count).reshape(shape)
        self.dev.lib.call("anvil_download", self.dev.ctx, out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset),
                          C.c_size_t(nbytes))
        return out

    def free(self):
        if self.ptr and self.dev.ctx:
            self.dev.lib.call("anvil_free", self.dev.ctx, C.c_void_p(self.ptr))
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HostBuffer:
    """Page-locked host memory of a Device (anvil_host_alloc), freed when collected: the target of downloads that
    the DMA engine writes directly, with no pageable staging."""

    def __init__(self, dev: "Device", nbytes: int):
        self.dev, self.nbytes = dev, int(nbytes)
        out = C.c_void_p()
        dev.lib.call("anvil_host_alloc", dev.ctx, C.c_size_t(max(1, self.nbytes)), C.byref(out))
        self.ptr = int(out.value)

    def array(self, dtype, count: int) -> np.ndarray:
        """The first `count` elements as a numpy array over this memory (no copy; it must not outlive the buffer)."""
        nbytes = int(count) * np.dtype(dtype).itemsize
        if nbytes > self.nbytes:
            raise ValueError(f"{nbytes} bytes asked of a {self.nbytes}-byte host buffer")
        return np.frombuffer((C.c_char * max(1, nbytes)).from_address(self.ptr), dtype=dtype, count=int(count))

    def free(self):
        if self.ptr and self.dev.ctx:
            self.dev.lib.call("anvil_host_free", self.dev.ctx, C.c_void_p(self.ptr))
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipGraph:
    """An executable HIP graph of a Device's stream (anvil_graph_end), replayed by launch(); freed when collected."""

    def __init__(self, dev: "Device", handle: int):
        self.dev, self.handle = dev, int(handle)

    def launch(self):
        self.dev.lib.call("anvil_graph_launch", self.dev.ctx, C.c_void_p(self.handle))

    def free(self):
        if self.handle and self.dev.ctx:
            self.dev.lib.call("anvil_graph_destroy", self.dev.ctx, C.c_void_p(self.handle))
        self.handle = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Device:
    """One anvil_ctx: a HIP device and the stream every op of this context runs on."""

    def __init__(self, device: int = 0):
        self.lib = library()
        self.index = int(device)
        ctx = C.c_void_p()
        self.lib.call("anvil_init", self.index, C.byref(ctx))
        self.ctx = ctx
        self.lock = threading.Lock()

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def host_alloc(self, nbytes: int) -> HostBuffer:
        return HostBuffer(self, nbytes)

    def capture(self, fn, *args) -> HipGraph:
        """fn(*args) recorded as a HIP graph of this context's stream instead of run (anvil_graph_begin / _end): the
        op calls it makes must need no first-use allocation and no synchronisation. The capture ends whatever fn
        raises."""
        self.lib.call("anvil_graph_begin", self.ctx)
        handle = C.c_void_p()
        try:
            fn(*args)
        except BaseException:
            try:
                self.lib.call("anvil_graph_end", self.ctx, C.byref(handle))
                HipGraph(self, handle.value or 0).free()
            except Exception:
                pass
            raise
        self.lib.call("anvil_graph_end", self.ctx, C.byref(handle))
        return HipGraph(self, handle.value)

    def upload(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        b = DeviceBuffer(self, arr.nbytes)
        b.upload(arr)
        return b

    def sync(self):
        self.lib.call("anvil_sync", self.ctx)

    def zero(self, ptr, nbytes: int):
        self.lib.call("anvil_zero", self.ctx, C.c_void_p(_ptr(ptr)), C.c_size_t(nbytes))

    def record(self, slot: int):
        self.lib.call("anvil_event_record", self.ctx, slot)

    def elapsed_ms(self, slot0: int, slot1: int) -> float:
        ms = C.c_float()
        self.lib.call("anvil_event_elapsed", self.ctx, slot0, slot1, C.byref(ms))
        return float(ms.value)

    def time_kernels(self, slot0: int, slot1: int):
        """Arm the kernel-bound timer (anvil_time_kernels): the kernels launched until disarm() carry the events
        of slot0 (first kernel's start) and slot1 (last kernel's end)."""
        self.lib.call("anvil_time_kernels", self.ctx, slot0, slot1)

    def disarm(self):
        self.lib.call("anvil_time_kernels", self.ctx, -1, -1)

    def timed(self, slot0: int, slot1: int, fn, *args):
        """fn(*args) with its kernels bound to the events of slot0 and slot1."""
        self.time_kernels(slot0, slot1)
        try:
            fn(*args)
        finally:
            self.disarm()

    def close(self):
        if self.ctx:
            self.lib.call("anvil_destroy", self.ctx)
            self.ctx = None

    # ------------------------------------------------------------------------------------------ op calls
    def gemm_i8(self, A, Bt, Cp, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, flags=0):
        st = (C.c_int64 * 9)(*[int(s) for s in strides])
        self.lib.call("anvil_gemm_i8_ex", self.ctx, C.c_void_p(_ptr(A)), C.c_void_p(_ptr(Bt)), C.c_void_p(_ptr(Cp)),
                      batch0, batch1, M, N, K, st, int(mult), shift, C.c_void_p(_ptr(lut) if lut is not None else 0),
                      DTYPE_CODE[out_dtype], int(flags))

    def gemm_i8_noalloc(self, A, Bt, Cp, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, flags=0):
        """anvil_gemm_i8_noalloc: gemm_i8 with split-K partials in the library's static scratch (allocates nothing)."""
        st = (C.c_int64 * 9)(*[int(s) for s in strides])
        self.lib.call("anvil_gemm_i8_noalloc", self.ctx, C.c_void_p(_ptr(A)), C.c_void_p(_ptr(Bt)),
                      C.c_void_p(_ptr(Cp)), batch0, batch1, M, N, K, st, int(mult), shift,
                      C.c_void_p(_ptr(lut) if lut is not None else 0), DTYPE_CODE[out_dtype], int(flags))

    def gemm_i8_group(self, calls):
        """Independent gemm_i8 calls (tuples of its arguments) in one anvil_gemm_i8_group call."""
        descs = (GemmDesc * len(calls))()
        for d, (A, Bt, Cp, b0, b1, M, N, K, strides, mult, shift, lut, out_dtype, flags) in zip(descs, calls):
            d.A, d.Bt, d.C = _ptr(A), _ptr(Bt), _ptr(Cp)
            d.lut = _ptr(lut) if lut is not None else None
            d.strides[:] = [int(s) for s in strides]
            d.batch0, d.batch1, d.M, d.N, d.K = b0, b1, M, N, K
            d.mult, d.shift, d.out_dtype, d.flags = int(mult), shift, DTYPE_CODE[out_dtype], int(flags)
        self.lib.call("anvil_gemm_i8_group", self.ctx, descs, len(calls))

    def gemm_i8_add(self, A, Bt, Cp, batch0, batch1, M, N, K, strides, mult, shift, lut, R, ma, mb, shift2, D,
                    rstrides, flags, out_dtype="i8"):
        """anvil_gemm_i8_add_ex: y = the product's requant, D = add_requant(R, y) in its epilogue; y, R and D are
        out_dtype."""
        st = (C.c_int64 * 9)(*[int(s) for s in strides])
        rs = (C.c_int64 * 6)(*[int(s) for s in rstrides])
        self.lib.call("anvil_gemm_i8_add_ex", self.ctx, C.c_void_p(_ptr(A)), C.c_void_p(_ptr(Bt)),
                      C.c_void_p(_ptr(Cp) if Cp is not None else 0), batch0, batch1, M, N, K, st, int(mult), shift,
                      C.c_void_p(_ptr(lut) if lut is not None else 0), DTYPE_CODE[out_dtype], C.c_void_p(_ptr(R)),
                      int(ma), int(mb), shift2, C.c_void_p(_ptr(D)), rs, int(flags))

    def gemm_i8_add_norm(self, A, Bt, Cp, M, N, K, strides, mult, shift, lut, R, ma, mb, shift2, D, rstrides,
                         nw, nlut, nlut_len, nmult, nshift, H, ld, kb, flags):
        """anvil_gemm_i8_add_norm: gemm_i8_add (batch 1, int8) whose sum D also feeds rmsnorm_int(D, nw, nlut, nmult,
        nshift) into H (row stride ld, or K-blocked with block stride kb and ld 64), all in one epilogue."""
        st = (C.c_int64 * 9)(*[int(s) for s in strides])
        rs = (C.c_int64 * 6)(*[int(s) for s in rstrides])
        norm = NormEpilogue(C.c_void_p(_ptr(nw)), C.c_void_p(_ptr(nlut)), int(nlut_len), int(nmult), int(nshift),
                            C.c_void_p(_ptr(H)), int(ld), int(kb))
        self.lib.call("anvil_gemm_i8_add_norm", self.ctx, C.c_void_p(_ptr(A)), C.c_void_p(_ptr(Bt)),
                      C.c_void_p(_ptr(Cp) if Cp is not None else 0), M, N, K, st, int(mult), shift,
                      C.c_void_p(_ptr(lut) if lut is not None else 0), C.c_void_p(_ptr(R)), int(ma), int(mb), shift2,
                      C.c_void_p(_ptr(D)), rs, C.byref(norm), int(flags))

    def rmsnorm_int(self, x, x_dtype, w, lut, lut_len, mult, shift, ss_shift, ss_init, rows, cols, out, flags=0):
        self.lib.call("anvil_rmsnorm_int_ex", self.ctx, C.c_void_p(_ptr(x)), DTYPE_CODE[x_dtype], C.c_void_p(_ptr(w)),
                      C.c_void_p(_ptr(lut)), lut_len, int(mult), shift, ss_shift, int(ss_init), rows, cols,
                      C.c_void_p(_ptr(out)), int(flags))

    def softmax_lut(self, x, lut, one, causal, batch, t1, t2, out, out_dtype, flags=0):
        self.lib.call("anvil_softmax_lut_ex", self.ctx, C.c_void_p(_ptr(x)), C.c_void_p(_ptr(lut)), int(one),
                      int(bool(causal)), batch, t1, t2, C.c_void_p(_ptr(out)), DTYPE_CODE[out_dtype], int(flags))

    def attention_i8(self, Q, K, Vt, O, b0, b1, T, D, strides, ms, ss, lut, one, causal, mo, so, flags):
        st = (C.c_int64 * 12)(*[int(s) for s in strides])
        self.lib.call("anvil_attention_i8", self.ctx, C.c_void_p(_ptr(Q)), C.c_void_p(_ptr(K)), C.c_void_p(_ptr(Vt)),
                      C.c_void_p(_ptr(O)), b0, b1, T, D, st, int(ms), ss, C.c_void_p(_ptr(lut)), int(one),
                      int(bool(causal)), int(mo), so, int(flags))

    def attention_i8_keep(self, Q, K, Vt, O, S, P, b0, b1, T, D, strides, ms, ss, lut, one, causal, mo, so, flags):
        """attention_i8 that also stores the scores into S and the probabilities into P (18 strides)."""
        st = (C.c_int64 * 18)(*[int(s) for s in strides])
        self.lib.call("anvil_attention_i8_keep", self.ctx, C.c_void_p(_ptr(Q)), C.c_void_p(_ptr(K)),
                      C.c_void_p(_ptr(Vt)), C.c_void_p(_ptr(O)), C.c_void_p(_ptr(S)), C.c_void_p(_ptr(P)), b0, b1, T, D,
                      st, int(ms), ss, C.c_void_p(_ptr(lut)), int(one), int(bool(causal)), int(mo), so, int(flags))

    def add_requant(self, a, a_dtype, b, b_dtype, ma, mb, shift, n, out, out_dtype, flags=0):
        self.lib.call("anvil_add_requant_ex", self.ctx, C.c_void_p(_ptr(a)), DTYPE_CODE[a_dtype], C.c_void_p(_ptr(b)),
                      DTYPE_CODE[b_dtype], int(ma), int(mb), shift, n, C.c_void_p(_ptr(out)), DTYPE_CODE[out_dtype],
                      int(flags))

    def lut_i8(self, x, table, n, out):
        self.lib.call("anvil_lut_i8", self.ctx, C.c_void_p(_ptr(x)), C.c_void_p(_ptr(table)), n,
                      C.c_void_p(_ptr(out)))

    def lut_mul(self, x, y, table, mult, shift, n, out, flags=0):
        self.lib.call("anvil_lut_mul_ex", self.ctx, C.c_void_p(_ptr(x)), C.c_void_p(_ptr(y)), C.c_void_p(_ptr(table)),
                      int(mult), shift, n, C.c_void_p(_ptr(out)), int(flags))

    def copy_strided(self, src, dst, elem_size, dims, src_strides):
        r = len(dims)
        d = (C.c_int64 * r)(*[int(v) for v in dims])
        s = (C.c_int64 * r)(*[int(v) for v in src_strides])
        self.lib.call("anvil_copy_strided", self.ctx, C.c_void_p(_ptr(src)), C.c_void_p(_ptr(dst)), elem_size, r, d, s)

    def quantize(self, x, x_is_f64, scale, n, out, out_dtype):
        self.lib.call("anvil_quantize", self.ctx, C.c_void_p(_ptr(x)), int(bool(x_is_f64)), float(scale), n,
                      C.c_void_p(_ptr(out)), DTYPE_CODE[out_dtype])

    def embed_quantize(self, ids, rows, T, Cdim, wte, vocab, wpe, scale, out, out_dtype):
        self.lib.call("anvil_embed_quantize", self.ctx, C.c_void_p(_ptr(ids)), int(rows), int(T), int(Cdim),
                      C.c_void_p(_ptr(wte)), int(vocab), C.c_void_p(_ptr(wpe)), float(scale), C.c_void_p(_ptr(out)),
                      DTYPE_CODE[out_dtype])


_devices = {}


def device(index: int = 0) -> Device:
    """The shared Device for a HIP device index (one context per process and device)."""
    with _lock:
        d = _devices.get(index)
    if d is None:
        d = Device(index)
        with _lock:
            d = _devices.setdefault(index, d)
    return d
