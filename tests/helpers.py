"""Test helpers: seeded random transformer-style graphs, the scalar C oracle binding and a graph walker over it.

random_case(seed) restates the coverage of the reference's random graph generator (tests/vortexv/vv_graphs.py:49-123):
multi-head batched matmuls with a transposed or plain right operand, transposes of any perm, reshapes, odd row
lengths, LUT epilogues, i16 results feeding an i16 rmsnorm with ss_shift / ss_init, causal and non-causal softmax
with T1 != T2 and an i32 softmax output. A draw the oracle rejects (int32 overflow, zero softmax sum) is redrawn.
"""
from __future__ import annotations

import ctypes as C
import gzip
import json
import subprocess
from pathlib import Path

import numpy as np

from anvil_mi355x.ir import GraphBuilder
from oracle import interp

ROOT = Path(__file__).resolve().parents[1]


def _rsqrt_lut(n):
    return np.round((1 << 15) / np.sqrt(np.arange(n) + 1)).astype(np.int64)


def _exp_lut(tau=24.0):
    return np.round((1 << 14) * np.exp((np.arange(256) - 255) / tau)).astype(np.int64)


SD = 60.0


def _scaled(rng, prod_sd, target_sd, lo=10, hi=20):
    s = int(rng.integers(lo, hi + 1))
    m = max(1, int(round(target_sd / prod_sd * (1 << s) * rng.uniform(0.5, 2.0))))
    return min(m, (1 << 31) - 1), s


def _mm(rng, k, target_sd=40.0):
    return _scaled(rng, SD * SD * np.sqrt(k), target_sd)


def _draw(rng):
    T = int(rng.integers(2, 9))
    T2 = T if rng.random() < 0.6 else int(rng.integers(2, 9))
    H = int(rng.integers(1, 4))
    dh = int(rng.integers(2, 11))
    d = int(rng.integers(3, 22))
    ff = int(rng.integers(3, 26))
    wide = rng.random() < 0.5
    neg_m = rng.random() < 0.3
    g = GraphBuilder("rand")
    consts = {}

    def const(name, shape, dtype="i8", value=None):
        v = rng.integers(-128, 128, shape) if value is None else np.asarray(value)
        consts[name] = np.asarray(v, dtype=np.int64)
        return g.const(name, list(consts[name].shape), dtype)

    x = g.input("x", [T, d])
    xk = g.input("xk", [T2, d])
    nl = int(rng.choice([64, 256, 1024]))
    rs = const("rsqrt", [nl], "i32", _rsqrt_lut(nl))
    rms = lambda: _scaled(rng, SD * (1 << 15) / (SD * np.sqrt(d)), 40.0, 4, 14)   # noqa: E731
    h = g.rmsnorm_int("h", x, const("nw", [d]), rs, *rms())
    hk = g.rmsnorm_int("hk", xk, const("nwk", [d]), rs, *rms())
    q = g.qlinear("q", h, const("wq", [d, H * dh]), *_mm(rng, d))
    k = g.qlinear("k", hk, const("wk", [d, H * dh]), *_mm(rng, d))
    v = g.qlinear("v", hk, const("wv", [d, H * dh]), *_mm(rng, d))
    qh = g.transpose("qh", g.reshape("q3", q, [T, H, dh]), [1, 0, 2])
    k3 = g.reshape("k3", k, [T2, H, dh])
    if rng.random() < 0.5:
        kT = g.transpose("kT", k3, [1, 2, 0])
    else:
        kT = g.transpose("kT", g.transpose("kh", k3, [1, 0, 2]), [0, 2, 1])
    sc = g.qmatmul("scores", qh, kT, *_mm(rng, dh))
    causal = bool(rng.random() < 0.6)
    ex = const("exp", [256], "i32", _exp_lut(float(rng.uniform(8, 40))))
    p = g.softmax_lut("p", sc, ex, int(rng.integers(32, 128)), causal)
    vh = g.transpose("vh", g.reshape("v3", v, [T2, H, dh]), [1, 0, 2])
    om, os_ = _mm(rng, T2)
    o = g.qmatmul("o", p, vh, -om if neg_m else om, os_)
    o2 = g.reshape("o2", g.transpose("ot", o, [1, 0, 2]), [T, H * dh])
    y = g.qlinear("y", o2, const("wo", [H * dh, d]), *_mm(rng, H * dh))
    rdt = "i16" if wide else "i8"
    rt_ = 2000.0 if wide else 40.0
    ma, s1 = _scaled(rng, SD, rt_ / 2, 8, 16)
    r1 = g.add_requant("r1", x, y, ma, _scaled(rng, SD, rt_ / 2, s1, s1)[0], s1, dtype=rdt)
    if wide:
        h2 = g.rmsnorm_int("h2", r1, const("nw2", [d]), rs, 1, int(rng.integers(12, 20)),
                           ss_shift=int(rng.integers(4, 9)), ss_init=int(rng.integers(0, 64)))
    else:
        h2 = g.rmsnorm_int("h2", r1, const("nw2", [d]), rs, *rms())
    silu = const("silu", [256])
    gate = g.qlinear("gate", h2, const("wg", [d, ff]), *_mm(rng, d),
                     lut=const("glut", [256]) if rng.random() < 0.5 else None)
    up = g.qlinear("up", h2, const("wu", [d, ff]), *_mm(rng, d))
    act = g.lut_mul("act", gate, up, silu, *_scaled(rng, SD * SD, 40.0))
    act = g.lut("act2", act, const("lut2", [256]))
    dn = g.qlinear("down", act, const("wd", [ff, d]), *_mm(rng, ff, 2000.0 if wide else 40.0), dtype=rdt)
    rsd = 2000.0 if wide else SD
    ma, s2 = _scaled(rng, rsd, 20.0, 8, 18)
    out = g.add_requant("out", r1, dn, ma, _scaled(rng, rsd, 20.0, s2, s2)[0], s2)
    p32 = g.softmax_lut("p32", sc, ex, int(rng.integers(1, 1 << 12)), not causal, dtype="i32")
    g.output(out, p32)
    inputs = {"x": rng.integers(-128, 128, (T, d)), "xk": rng.integers(-128, 128, (T2, d))}
    return g.module(), consts, inputs


def random_case(seed, tries=50):
    """(module, consts, inputs, oracle GraphResult) for seed, redrawn until the oracle accepts the draw."""
    rng = np.random.default_rng([7, seed])
    for _ in range(tries):
        m, c, x = _draw(rng)
        try:
            return m, c, x, interp.run(m, x, c)
        except (OverflowError, ValueError, ZeroDivisionError):
            continue
    raise RuntimeError(f"seed {seed}: no in-contract draw in {tries} tries")


# ----------------------------------------------------------------------------------------- scalar C oracle

_SO = None
_ERR = {1: ValueError, 2: OverflowError, 3: ZeroDivisionError}


def scalar_oracle():
    """ctypes handle on oracle/build/libscalar_oracle.so (built by oracle/Makefile on first use)."""
    global _SO
    if _SO is None:
        lib = ROOT / "oracle" / "build" / "libscalar_oracle.so"
        src = ROOT / "oracle" / "scalar_oracle.c"
        if not lib.exists() or lib.stat().st_mtime < src.stat().st_mtime:
            subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
        _SO = C.CDLL(str(lib))
    return _SO


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _chk(rc):
    if rc:
        raise _ERR.get(rc, RuntimeError)(f"scalar oracle status {rc}")


def _i64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


DT_BITS = {"i8": 8, "i16": 16, "i32": 32}


def scalar_run(m, inputs, consts, batch=False):
    """Evaluate a graph with the scalar C ops (layout ops in numpy): an interpreter independent of
    oracle.semantics, for cross-checking it. Returns {sym: int64 array}."""
    so = scalar_oracle()
    L = C.c_int64
    env, vals, is_const = {}, {}, set()
    fn = [op for op in m.ops[0].ops]
    nb = len(next(iter(inputs.values()))) if batch else None
    for op in fn:
        n = op.name.split(".")[-1]
        if n == "output":
            continue
        r = op.results[0]
        t = r.type
        if n == "input":
            val = _i64(inputs[op.sym_str])
        elif n == "const":
            val = _i64(consts[op.sym_str] if op.value is None else op.value)
            is_const.add(r)
        elif n in ("qmatmul", "qlinear"):
            a, b = env[op.a], env[op.b]
            K, N = b.shape[-2], b.shape[-1]
            Mr = a.shape[-2]
            lead = a.shape[:-2]
            batch_n = int(np.prod(lead)) if lead else 1
            bb = b.ndim > 2
            if bb and b.shape[:-2] != lead:
                b = np.broadcast_to(b, lead + b.shape[-2:])
            a_c, b_c = _i64(a), _i64(b)
            out = np.empty(lead + (Mr, N), dtype=np.int64)
            lut = None if op.lut is None else _i64(env[op.lut])
            _chk(so.so_qmatmul(_p(a_c), _p(b_c), _p(out), L(batch_n), L(Mr), L(K), L(N), int(bb), L(int(op.M)),
                               int(op.s), None if lut is None else _p(lut), DT_BITS[t.dtype]))
            val = out
        elif n == "lut":
            x = _i64(env[op.x])
            val = np.empty_like(x)
            _chk(so.so_lut(_p(x), _p(_i64(env[op.table])), _p(val), L(x.size)))
        elif n == "lut_mul":
            x, y = _i64(env[op.x]), _i64(env[op.y])
            val = np.empty_like(x)
            _chk(so.so_lut_mul(_p(x), _p(y), _p(_i64(env[op.table])), _p(val), L(x.size), L(int(op.M)), int(op.s)))
        elif n == "add_requant":
            a, b = _i64(env[op.a]), _i64(env[op.b])
            val = np.empty_like(a)
            _chk(so.so_add_requant(_p(a), _p(b), _p(val), L(a.size), L(int(op.Ma)), L(int(op.Mb)), int(op.s),
                                   DT_BITS[t.dtype]))
        elif n == "rmsnorm_int":
            x = _i64(env[op.x])
            lut = _i64(env[op.lut])
            val = np.empty_like(x)
            _chk(so.so_rmsnorm(_p(x), _p(_i64(env[op.w])), _p(lut), L(lut.size), _p(val), L(x.size // x.shape[-1]),
                               L(x.shape[-1]), L(int(op.M)), int(op.s), op.ss_shift_int, L(op.ss_init_int),
                               DT_BITS[op.x.type.dtype]))
        elif n == "softmax_lut":
            x = _i64(env[op.x])
            val = np.empty_like(x)
            t1, t2 = x.shape[-2], x.shape[-1]
            _chk(so.so_softmax(_p(x), _p(_i64(env[op.lut])), _p(val), L(x.size // (t1 * t2)), L(t1), L(t2),
                               L(int(op.one)), int(bool(op.causal)), DT_BITS[t.dtype]))
        elif n == "transpose":
            k = 0 if op.x in is_const or nb is None else 1
            val = np.transpose(env[op.x], list(range(k)) + [p + k for p in op.perm_list])
        elif n == "reshape":
            lead = () if op.x in is_const or nb is None else (nb,)
            val = env[op.x].reshape(lead + tuple(t.dims))
        else:
            raise NotImplementedError(op.name)
        if n in ("transpose", "reshape") and op.x in is_const:
            is_const.add(r)
        env[r] = val
        if op.sym_str is not None:
            vals[op.sym_str] = val
    return vals


GOLDEN = Path(__file__).resolve().parent / "golden"


def reference_model(name):
    """(IR text, consts, held-out input or None) of the reference's frozen model file tests/golden/model_graph_<name>."""
    body = json.load(gzip.open(GOLDEN / f"model_graph_{name}.json.gz", "rt"))
    consts = {k: np.asarray(v, dtype=np.int64).reshape(body["shapes"][k]) for k, v in body["consts"].items()}
    x = np.asarray(body["x"], dtype=np.int64) if "x" in body else None
    return body["ir"], consts, x
