"""Test helpers: seeded random transformer-style graphs, the scalar C oracle binding and a graph walker over it.

random_case(seed) draws a graph with the op mix the reference's random graph tests cover (tests/vortexv/
vv_graphs.py): head-batched matmuls whose right operand is a transposed view reached by one or two transposes, a
cross-attention key length, causal and non-causal softmax (one output in i32), reshapes, LUT epilogues, lut_mul and
lut, negative multipliers, and a wide variant whose i16 residual stream feeds an rmsnorm with ss_shift / ss_init.
The generator evaluates each op on the sampled inputs as it adds it, and fits every requant multiplier to the spread
of the accumulator it scales, so values spread across their dtype instead of saturating. A draw the oracle rejects
(int32 overflow, zero softmax sum) is redrawn.
"""
from __future__ import annotations

import ctypes as C
import gzip
import json
import subprocess
from pathlib import Path

import numpy as np

from anvil_mi355x import quantize as Q
from anvil_mi355x.ir import GraphBuilder
from oracle import interp
from oracle import semantics as sem

ROOT = Path(__file__).resolve().parents[1]


class _Fuzz:
    """A GraphBuilder paired with the values of its ops on one sampled input."""

    def __init__(self, rng):
        self.rng = rng
        self.b = GraphBuilder("rand")
        self.consts, self.val = {}, {}

    def pick(self, *opts):
        return opts[int(self.rng.integers(len(opts)))]

    def input(self, name, shape, dtype="i8"):
        v = self.b.input(name, list(shape), dtype)
        self.val[v] = self.rng.integers(-128, 128, shape)
        return v

    def const(self, name, data, dtype="i8"):
        data = np.asarray(data, dtype=np.int64)
        self.consts[name] = data
        v = self.b.const(name, list(data.shape), dtype)
        self.val[v] = data
        return v

    def weight(self, name, shape):
        return self.const(name, self.rng.integers(-128, 128, shape))

    def fit(self, acc, spread, shifts, negative=False):
        """(M, s): s drawn from `shifts`, M scaling the accumulator's root mean square to about `spread`."""
        s = int(self.rng.integers(shifts[0], shifts[1] + 1))
        sd = max(float(np.sqrt(np.mean(np.square(acc, dtype=np.float64)))), 1.0)
        m = int(np.clip(round(spread / sd * (1 << s) * self.rng.uniform(0.6, 1.7)), 1, (1 << 31) - 1))
        return -m if negative else m, s

    def matmul(self, kind, name, a, b, spread=45.0, lut=None, dtype="i8", negative=False):
        acc = self.val[a] @ self.val[b]
        m, s = self.fit(acc, spread, (9, 19), negative)
        r = getattr(self.b, kind)(name, a, b, m, s, lut=lut, dtype=dtype)
        self.val[r] = sem.qmatmul(self.val[a], self.val[b], m, s, None if lut is None else self.val[lut], dtype)
        return r

    def view(self, kind, name, x, arg):
        r = getattr(self.b, kind)(name, x, list(arg))
        self.val[r] = np.transpose(self.val[x], arg) if kind == "transpose" else self.val[x].reshape(arg)
        return r

    def rmsnorm(self, name, x, table, wide=False):
        d = self.val[x].shape[-1]
        w = self.weight(name + ".w", [d])
        xv = self.val[x]
        c, e = (int(self.rng.integers(3, 9)), int(self.rng.integers(0, 80))) if wide else (0, 0)
        ss = ((xv * xv + (1 << c >> 1)) >> c).sum(-1) + e
        idx, k = sem.rsqrt_index(ss, len(self.val[table]))
        acc = xv * self.val[w] * self.val[table][idx][..., None] / (2.0 ** k)[..., None]
        if wide:           # the wide rows keep M = 1, as the quantizer builds them: the spread is set by s alone
            rms = max(float(np.sqrt(np.mean(np.square(acc)))), 1.0)
            m, s = 1, int(np.clip(round(np.log2(rms / 45.0) + self.rng.uniform(-0.7, 0.7)), 0, 31 - int(k.max())))
        else:
            m, s = self.fit(acc, 45.0, (12, 22))
        r = self.b.rmsnorm_int(name, x, w, table, m, s, ss_shift=c, ss_init=e)
        self.val[r] = sem.rmsnorm_wide(xv, self.val[w], self.val[table], m, s, c, e, "i16" if wide else "i8")
        return r

    def add(self, name, a, b_, dtype, spread):
        ma, s = self.fit(self.val[a], spread / 2, (8, 16))
        mb, _ = self.fit(self.val[b_], spread / 2, (s, s))
        r = self.b.add_requant(name, a, b_, ma, mb, s, dtype=dtype)
        self.val[r] = sem.add_requant(self.val[a], self.val[b_], ma, mb, s, dtype)
        return r

    def softmax(self, name, x, table, one, causal, dtype="i8"):
        r = self.b.softmax_lut(name, x, table, one, causal, dtype=dtype)
        self.val[r] = sem.softmax_lut(self.val[x], self.val[table], one, causal)
        return r

    def lut(self, name, x, table):
        r = self.b.lut(name, x, table)
        self.val[r] = sem.lut_i8(self.val[x], self.val[table])
        return r

    def lut_mul(self, name, x, y, table):
        prod = self.val[table][self.val[x] + 128] * self.val[y]
        m, s = self.fit(prod, 45.0, (9, 19))
        r = self.b.lut_mul(name, x, y, table, m, s)
        self.val[r] = sem.swiglu_lut(self.val[x], self.val[y], self.val[table], m, s)
        return r


def _draw(rng):
    """One random graph: rmsnorm -> multi-head (possibly cross) attention -> residual -> rmsnorm -> gated MLP ->
    residual, plus a second softmax of the scores as an i32 output."""
    f = _Fuzz(rng)
    tq = int(rng.integers(2, 10))
    tk = tq if rng.random() < 0.55 else int(rng.integers(2, 10))
    heads, hd = int(rng.integers(1, 4)), int(rng.integers(2, 12))
    d, ff = int(rng.integers(3, 23)), int(rng.integers(3, 27))
    wide = bool(rng.random() < 0.5)
    n_rs = int(f.pick(64, 256, 1024))
    rsqrt = f.const("rsqrt", np.round(32768.0 / np.sqrt(np.arange(n_rs) + 1.0)), "i32")
    x, xk = f.input("x", (tq, d)), f.input("xk", (tk, d))
    h, hk = f.rmsnorm("h", x, rsqrt), f.rmsnorm("hk", xk, rsqrt)
    q = f.matmul("qlinear", "q", h, f.weight("wq", [d, heads * hd]))
    k = f.matmul("qlinear", "k", hk, f.weight("wk", [d, heads * hd]))
    v = f.matmul("qlinear", "v", hk, f.weight("wv", [d, heads * hd]))
    qh = f.view("transpose", "qh", f.view("reshape", "q3", q, (tq, heads, hd)), (1, 0, 2))
    k3 = f.view("reshape", "k3", k, (tk, heads, hd))
    if rng.random() < 0.5:
        kt = f.view("transpose", "kT", k3, (1, 2, 0))
    else:
        kt = f.view("transpose", "kT", f.view("transpose", "kh", k3, (1, 0, 2)), (0, 2, 1))
    scores = f.matmul("qmatmul", "scores", qh, kt)
    temp = float(rng.uniform(8.0, 40.0))
    exp = f.const("exp", np.round(16384.0 * np.exp((np.arange(256) - 255.0) / temp)), "i32")
    causal = bool(rng.random() < 0.6)
    p = f.softmax("p", scores, exp, int(rng.integers(32, 128)), causal)
    vh = f.view("transpose", "vh", f.view("reshape", "v3", v, (tk, heads, hd)), (1, 0, 2))
    o = f.matmul("qmatmul", "o", p, vh, negative=bool(rng.random() < 0.3))
    om = f.view("reshape", "o2", f.view("transpose", "ot", o, (1, 0, 2)), (tq, heads * hd))
    y = f.matmul("qlinear", "y", om, f.weight("wo", [heads * hd, d]))
    res_dt, res_spread = ("i16", 2000.0) if wide else ("i8", 45.0)
    r1 = f.add("r1", x, y, res_dt, res_spread)
    h2 = f.rmsnorm("h2", r1, rsqrt, wide=wide)
    glut = f.weight("glut", [256]) if rng.random() < 0.5 else None
    gate = f.matmul("qlinear", "gate", h2, f.weight("wg", [d, ff]), lut=glut)
    up = f.matmul("qlinear", "up", h2, f.weight("wu", [d, ff]))
    act = f.lut("act2", f.lut_mul("act", gate, up, f.weight("silu", [256])), f.weight("lut2", [256]))
    down = f.matmul("qlinear", "down", act, f.weight("wd", [ff, d]), spread=res_spread, dtype=res_dt)
    out = f.add("out", r1, down, "i8", 20.0)
    p32 = f.softmax("p32", scores, exp, int(rng.integers(1, 1 << 12)), not causal, dtype="i32")
    f.b.output(out, p32)
    inputs = {"x": f.val[x], "xk": f.val[xk]}
    return f.b.module(), f.consts, inputs


def random_case(seed, tries=50):
    """(module, consts, inputs, oracle GraphResult) for seed, redrawn until the oracle accepts the draw."""
    rng = np.random.default_rng([11, seed])
    for _ in range(tries):
        try:
            m, c, x = _draw(rng)
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


def kblock_graph():
    """x (16, 128) -> rmsnorm h -> qlinear a, qlinear b; h also feeds an add (so h stays row-major); a feeds two
    qlinears (K-blocked); b is returned (row-major); c = qlinear(a) feeds a lut (row-major)."""
    rng = np.random.default_rng(31)
    bld = GraphBuilder("kb")
    x = bld.input("x", [16, 128])
    w = bld.const("w", [128], value=rng.integers(-100, 100, 128))
    lut, s = Q.rsqrt_table(0.03, 0.01, 0.02, 100, 128, 1e-5)
    h = bld.rmsnorm_int("h", x, w, bld.const("r", [len(lut)], dtype="i32", value=lut), 1, s)
    wt = lambda n, k: bld.const(n, [k, 128], value=rng.integers(-128, 128, (k, 128)))      # noqa: E731
    a = bld.qlinear("a", h, wt("wa", 128), 3, 16)
    b = bld.qlinear("b", h, wt("wb", 128), 3, 16)
    r = bld.add_requant("r1", h, x, 1, 1, 1)
    c = bld.qlinear("c", a, wt("wc", 128), 3, 16)
    d = bld.qlinear("d", a, wt("wd", 128), 3, 16)
    e = bld.lut("e", c, bld.const("t", [256], value=rng.integers(-128, 128, 256)))
    bld.output(b, r, d, e)
    return bld.module()
