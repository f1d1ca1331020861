"""anvil_mi355x.hostpar: the chunked, threaded host loops of a run give the single numpy call's results bit for bit,
on contiguous, strided and broadcast (stride 0) arrays, for the read-back widening, the float64 dequantization and
the input's finiteness check."""
import numpy as np
import pytest

from anvil_mi355x import hostpar


@pytest.fixture(params=[1, 1 << 40], ids=["threaded", "single"])
def par_min(request, monkeypatch):
    monkeypatch.setattr(hostpar, "PAR_MIN", request.param)


def _arrays(rng):
    base = rng.integers(-128, 128, (6, 37, 40), dtype=np.int8)
    yield base                                                    # contiguous
    yield base[:, ::3, 1::2]                                      # strided
    yield base.transpose(2, 0, 1)                                 # permuted
    yield np.lib.stride_tricks.as_strided(base, shape=(5, 37, 40), strides=(0, 40, 1))   # broadcast first dim
    yield base[:1]                                                # leading dim of one
    yield rng.integers(-(1 << 15), 1 << 15, (7, 300), dtype=np.int16)


def test_astype_matches_numpy(par_min):
    rng = np.random.default_rng(1)
    for a in _arrays(rng):
        got = hostpar.astype(a, np.int64)
        assert got.dtype == np.int64 and got.flags.c_contiguous and np.array_equal(got, a.astype(np.int64))


@pytest.mark.parametrize("s", [1.0, 0.0123456789, 3.7e-5, -2.5])
def test_scaled_f64_matches_numpy_bit_for_bit(par_min, s):
    rng = np.random.default_rng(2)
    for a in _arrays(rng):
        ints = a.astype(np.int64)
        want = np.asarray(ints, dtype=np.float64) * s
        got = hostpar.scaled_f64(ints, s)
        assert got.dtype == np.float64 and np.array_equal(got.view(np.uint64), want.view(np.uint64))
        got = hostpar.scaled_f64(a, s)                             # straight from the narrow integer view
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_all_finite(par_min, bad):
    x = np.random.default_rng(3).standard_normal((9, 33, 17)).astype(np.float32)
    assert hostpar.all_finite(x) and hostpar.all_finite(x[:, ::2])
    x[-1, -1, -1] = bad                                           # in the last chunk
    assert not hostpar.all_finite(x)
    assert not hostpar.all_finite(x[:, ::2, :])                   # row 32 of 33 is kept by the stride


def test_one_pool_for_concurrent_callers(monkeypatch):
    """Host threads that start runs at the same moment share one pool, and their results are each the single call's."""
    import threading
    monkeypatch.setattr(hostpar, "PAR_MIN", 1)
    monkeypatch.setattr(hostpar, "_pool", None)
    a = np.arange(-5000, 5000, dtype=np.int16).reshape(100, 100)
    pools, outs, go = [], [None] * 8, threading.Barrier(8)

    def work(i):
        go.wait()
        pools.append(hostpar.pool())
        outs[i] = hostpar.astype(a[i % 3:], np.int64)

    ts = [threading.Thread(target=work, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert len({id(p) for p in pools}) == 1
    assert all(np.array_equal(o, a[i % 3:].astype(np.int64)) for i, o in enumerate(outs))
