"""Host-side elementwise work of a run (the input's finiteness check, widening read-back values to int64, float64
dequantization) split into chunks over a thread pool. numpy releases the GIL inside these loops, so the chunks run
in parallel; each element goes through the same operation as in one whole-array call, so results are identical.
Arrays below PAR_MIN elements take the single call."""
import concurrent.futures
import os
import threading

import numpy as np

PAR_MIN = 1 << 20
_pool = None
_pool_lock = threading.Lock()


def _workers() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def pool():
    global _pool
    with _pool_lock:                  # runs from several host threads at once create one pool between them
        if _pool is None:
            _pool = concurrent.futures.ThreadPoolExecutor(max_workers=_workers(), thread_name_prefix="anvil-host")
        return _pool


def _after_fork():
    # a forked child has none of the parent's pool threads (and a lock possibly taken by one of them): it starts its
    # own pool when it needs one
    global _pool, _pool_lock
    _pool = None
    _pool_lock = threading.Lock()


os.register_at_fork(after_in_child=_after_fork)


def _ranges(n: int, parts: int):
    step = -(-n // parts)
    return [(i, min(n, i + step)) for i in range(0, n, step)]


def _split(a: np.ndarray):
    """(axis, ranges) to chunk a along, or None for the single call: the flat array when it is contiguous, else its
    first dim of at least two entries when every dim before it has one."""
    if a.size < PAR_MIN or _workers() == 1:
        return None
    if a.flags.c_contiguous:
        return -1, _ranges(a.size, 4 * _workers())
    for ax, d in enumerate(a.shape):
        if d >= 2:
            return ax, _ranges(d, min(d, 4 * _workers()))
        if d != 1:
            break
    return None


def _chunks(a: np.ndarray, axis: int, lo: int, hi: int):
    if axis < 0:
        return a.reshape(-1)[lo:hi]
    return a[(slice(None),) * axis + (slice(lo, hi),)]


def _run(fn, spans):
    list(pool().map(lambda lh: fn(*lh), spans))


def all_finite(a: np.ndarray) -> bool:
    """np.all(np.isfinite(a))."""
    sp = _split(a)
    if sp is None:
        return bool(np.all(np.isfinite(a)))
    axis, spans = sp
    return all(pool().map(lambda lh: bool(np.all(np.isfinite(_chunks(a, axis, *lh)))), spans))


def astype(a: np.ndarray, dtype) -> np.ndarray:
    """a.astype(dtype): a new C-contiguous array."""
    sp = _split(a)
    if sp is None:
        return a.astype(dtype, order="C")
    out = np.empty(a.shape, dtype)
    axis, spans = sp
    _run(lambda lo, hi: np.copyto(_chunks(out, axis, lo, hi), _chunks(a, axis, lo, hi), casting="unsafe"), spans)
    return out


def scaled_f64(a: np.ndarray, s: float) -> np.ndarray:
    """np.asarray(a, dtype=np.float64) * s."""
    a = np.asarray(a)
    sp = _split(a)
    if sp is None:
        return np.asarray(a, dtype=np.float64) * s
    out = np.empty(a.shape, np.float64)
    axis, spans = sp
    _run(lambda lo, hi: np.multiply(_chunks(a, axis, lo, hi), s, out=_chunks(out, axis, lo, hi),
                                    dtype=np.float64), spans)
    return out
