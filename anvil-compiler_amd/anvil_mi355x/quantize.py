"""Integer constants of a quantized graph, and the int32 proof that guards them.

Everything here runs once on the host while a model is built. It decides three kinds of constants:

* requant multipliers and shifts (choose_shift): the widest shift whose worst-case numerator still fits int32;
* lookup tables: the rsqrt table of rmsnorm_int (rsqrt_table, wide_rsqrt_table), softmax_lut's exp table
  (exp_table) and int8 -> int8 activation tables (activation_table);
* the int32 proof over a finished graph (prove_no_overflow, int32_bounds).

The numbers these produce must equal the reference quantizer's (anvil/frontend/quantize.py:40-253, symmetric
per-tensor int8, xf's contract 8), because bit-exact outputs need bit-equal constants: every float expression that
feeds a rint() or a round() keeps the reference's operation order, and every bound the proof checks is the
reference's. The code is organised differently: a shift search over all candidate shifts, a WideRow model of the
reachable (index, step) states of a wide rmsnorm row, and a BoundWalker with one handler per op kind that serves
two policies (the reference's decision, and the sound bound the GPU kernels rely on).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import ir as g

INT32_MAX = (1 << 31) - 1
RSQRT_LEN = 1024            # entries of an rmsnorm rsqrt table
SOFTMAX_ONE = 127           # softmax_lut's `one`: probabilities land in [0, 127]
HEADROOM = 1.5              # activation scale = HEADROOM * max|activation| / 127
DTYPE_MAG = {"i8": 128, "i16": 1 << 15, "i32": 1 << 31}    # largest |value| of each dtype


def half(s: int) -> int:
    """The rounding term of an arithmetic right shift by s: 2^(s-1), or 0 for s = 0."""
    return 1 << (s - 1) if s > 0 else 0


# ------------------------------------------------------------------------------------------------ requant

def choose_shift(ratios, bounds, extra: int = 0, top: int = 31):
    """(multipliers, s) for real ratios m_i applied to integers of magnitude <= bound_i: the largest s in
    [0, top - extra] at which M_i = round(m_i 2^s) keeps sum_i bound_i M_i + 2^(s+extra-1) within int32 (`extra` is
    a shift the op adds at run time, as rmsnorm's normalisation steps do). Reference: anvil/frontend/quantize.py:40-56
    (its fixed_point). ValueError when a multiplier rounds to 0 at that shift, OverflowError when no shift fits."""
    ratios, bounds = list(ratios), list(bounds)
    if not ratios or len(ratios) != len(bounds):
        raise ValueError(f"choose_shift: {len(ratios)} ratios against {len(bounds)} bounds")
    if min(ratios) <= 0 or min(bounds) < 0:
        raise ValueError(f"choose_shift: ratios must be > 0 and bounds >= 0 (got {ratios}, {bounds})")

    def numerator(s):
        mults = [round(m * (1 << s)) for m in ratios]
        return mults, sum(int(b) * mm for b, mm in zip(bounds, mults)) + half(s + extra)

    fitting = [s for s in range(top - extra + 1) if numerator(s)[1] <= INT32_MAX]
    if not fitting:
        raise OverflowError(f"choose_shift: bounds {bounds} overflow int32 for ratios {ratios} at every shift")
    s = max(fitting)
    mults = numerator(s)[0]
    if min(mults) < 1:
        raise ValueError(f"choose_shift: ratios {ratios} round to a zero multiplier at shift {s}")
    return mults, s


def maxabs_scale(x) -> float:
    """Symmetric int8 scale of x: max|x| / 127."""
    return float(np.abs(np.asarray(x)).max()) / 127


def to_int8(x, scale):
    """Round half to even at `scale`, saturating at int8, as int64."""
    return np.clip(np.rint(np.asarray(x) / scale), -128, 127).astype(np.int64)


# ------------------------------------------------------------------------------------------------ rmsnorm

def rsqrt_steps(ss: int, n: int):
    """(index, k): the row sum ss divided by 4 (two bits shifted out) k times, until it indexes an n-entry table
    (reference anvil/codegen/lower.py:107-113)."""
    ss, k = int(ss), 0
    while ss >= n:
        ss, k = ss >> 2, k + 1
    return ss, k


def loudest_row_steps(d: int, n: int = RSQRT_LEN, mag: int = 128) -> int:
    """The k of a row of d entries all of magnitude mag: the largest k any such row reaches."""
    return rsqrt_steps(d * mag * mag, n)[1]


def rsqrt_table(sx, sw, sh, wmax, d, eps, n=RSQRT_LEN):
    """(table, s) of an int8 rmsnorm from input scale sx through weight scale sw (max |w| = wmax) to output scale sh:
    table[i] = rint(sx sw / sh / sqrt(sx^2 i / d + eps) 2^s) for i >= 1, table[0] = 0, with s the widest shift at
    which x * w * table[i] (+ rounding, after up to loudest_row_steps(d) extra shifts) fits int32 for |x| <= 128
    (reference anvil/frontend/quantize.py:72-80)."""
    idx = np.arange(1, n)
    real = np.r_[0, 1 / np.sqrt(sx ** 2 * idx / d + eps) * sx * sw / sh]
    (top,), s = choose_shift([real.max()], [128 * wmax], loudest_row_steps(d, n))
    table = np.rint(real * (1 << s)).astype(np.int64)
    if table.max() != top:
        raise AssertionError("rsqrt_table: the table's largest entry differs from its chosen multiplier")
    return table, s


def square_shift(d: int, mag: int) -> int:
    """Least c for which d squares of magnitude mag, each rounded and shifted right by c, sum within int32 (the
    wide rmsnorm's ss_shift; 0 for int8 rows). Reference anvil/frontend/quantize.py:85-91."""
    c = next((c for c in range(31) if d * ((mag * mag + half(c)) >> c) <= INT32_MAX), None)
    if c is None:
        raise OverflowError(f"square_shift: {d} squares of {mag} overflow int32 at every shift")
    return c


@dataclass
class WideRow:
    """The reachable states of an rmsnorm row of d entries (|x| <= mag) with square shift c and sum offset e:
    ss = e + sum((x^2 + 2^(c-1)) >> c) lands on table index i after k steps of rsqrt_steps. For each k it holds
    xmax[k][i], the largest |x| one entry of such a row can have; x * table[i] is largest at large k, not at the
    table's largest entry (reference anvil/frontend/quantize.py:99-119)."""
    d: int
    n: int
    c: int
    mag: int
    e: int = 0
    xmax: dict = field(init=False)

    def __post_init__(self):
        top = self.d * ((self.mag * self.mag + half(self.c)) >> self.c) + self.e     # the loudest row's ss
        self.xmax = {}
        for k in range(rsqrt_steps(top, self.n)[1] + 1):
            # the largest ss that still lands on index i after k steps, capped by the loudest row
            ss_hi = [min((i + 1) * 4 ** k - 1, top) for i in range(self.n)]
            col = np.array([self._largest_entry(v - self.e) if v >= self.e else 0 for v in ss_hi], dtype=np.int64)
            if k > 0:
                col[: self.n // 4] = 0         # a shifted sum is >= n/4: lower indices need k = 0
            self.xmax[k] = col

    def _largest_entry(self, budget: int) -> int:
        """Largest |x| <= mag whose shifted square (x^2 + 2^(c-1)) >> c is at most budget."""
        return min(self.mag, math.isqrt(max(0, ((budget + 1) << self.c) - half(self.c) - 1)))

    @property
    def kmax(self) -> int:
        return max(self.xmax)

    def numerators(self, table, wmax: int, mult: int, s: int) -> dict:
        """{k: worst x * w * table[i] * mult + 2^(s+k-1)} over the reachable (i, k)."""
        table = np.asarray(table, dtype=np.int64)
        return {k: int((col * wmax * table).max()) * mult + half(s + k) for k, col in self.xmax.items()}

    def worst_product(self, table, wmax: int) -> int:
        table = np.asarray(table, dtype=np.int64)
        return max(int((col * wmax * table).max()) for col in self.xmax.values())


def wide_rsqrt_table(sx, sw, sh, wmax, d, eps, mag, n=RSQRT_LEN):
    """(table, s, c, e) of an rmsnorm over wide (int16) rows. Squares are rounded and shifted by c = square_shift(d,
    mag); eps enters as the integer offset e = max(1, round(eps / unit)) of the sum, unit = sx^2 2^c / d being the
    mean square one count of ss stands for, so the table holds the eps-free rsqrt(unit i) sx sw / sh. s is the widest
    shift at which every reachable x * w * table[i] (+ rounding) fits int32 under WideRow's bound (reference
    anvil/frontend/quantize.py:122-144)."""
    c = square_shift(d, mag)
    unit = sx ** 2 * (1 << c) / d
    e = max(1, int(round(eps / unit)))
    if d * ((mag * mag + half(c)) >> c) + e > INT32_MAX:
        raise OverflowError(f"wide_rsqrt_table: the eps offset {e} pushes the row sum past int32 at scale {sx}")
    idx = np.arange(1, n)
    real = np.r_[0, 1 / np.sqrt(unit * idx) * sx * sw / sh]
    row = WideRow(d, n, c, mag, e)
    for s in range(31 - row.kmax, -1, -1):
        table = np.rint(real * (1 << s)).astype(np.int64)
        if max(row.numerators(table, wmax, 1, s).values()) > INT32_MAX:
            continue
        coarsest = int(table[n // 4:].min())
        if coarsest < 64:
            raise ValueError(f"wide_rsqrt_table: at shift {s} the table's smallest reachable entry is {coarsest} < 64")
        return table, s, c, e
    raise OverflowError("wide_rsqrt_table: no table shift keeps the wide rmsnorm within int32")


# ------------------------------------------------------------------------------------------------ softmax

def exp_shift(t: int, one: int = SOFTMAX_ONE) -> int:
    """Largest E for which a softmax row of t entries, each <= 2^E, keeps its sum (t 2^E) and its numerators
    ((one + t // 2) 2^E) within int32 (reference anvil/frontend/quantize.py:155-157)."""
    return max(e for e in range(31) if max(one + t // 2, t) << e <= INT32_MAX)


def exp_table(score_scale, t: int, one: int = SOFTMAX_ONE):
    """softmax_lut's 256-entry table: entry j holds rint(exp((j - 255) score_scale) 2^E), E = exp_shift(t, one)
    (reference anvil/frontend/quantize.py:160-162)."""
    return np.rint(np.exp(np.arange(-255, 1) * score_scale) * (1 << exp_shift(t, one))).astype(np.int64)


# ------------------------------------------------------------------------------------------------ activations

def silu(x):
    return x / (1 + np.exp(-x))


def activation_table(f, s_in, s_out):
    """int8 -> int8 table of an elementwise activation: entry j holds to_int8(f((j - 128) s_in), s_out), as the
    reference tabulates its SiLU node (anvil/frontend/quantize.py:446-452)."""
    return to_int8(f(np.arange(-128, 128) * s_in), s_out)


# ------------------------------------------------------------------------------------------------ int32 proof

@dataclass
class Bounds:
    """What the int32 analysis of one graph found."""
    worst: dict            # op sym -> largest |intermediate| of the op
    failures: list         # one message per intermediate that can leave int32
    acc: dict              # matmul result Value -> bound on |accumulator|

    @property
    def ok(self) -> bool:
        return not self.failures


class BoundWalker:
    """Magnitude propagation over a graph: each value gets a bound on its |elements| (inputs by dtype, consts by
    their values, op results by their dtype or LUT), and each op's int32 intermediates are bounded from its
    operands' magnitudes, as the reference's prove_no_overflow does (anvil/frontend/quantize.py:175-253).

    reference=True reproduces that function's decision exactly, including its two loose spots: multipliers enter
    with their sign (a negative M bounds nothing), and a const right operand with batch dims sums its first axis.
    reference=False is the sound policy the GPU kernels' unchecked paths rely on: |M|, and the column sums of each
    batch entry of a const right operand."""

    def __init__(self, consts=None, reference: bool = True):
        self.consts = consts or {}
        self.reference = reference
        self.mag, self.values, self.worst, self.failures, self.acc = {}, {}, {}, [], {}
        self.handlers = {
            g.InputOp: self._input, g.ConstOp: self._const, g.QMatmulOp: self._matmul, g.QLinearOp: self._matmul,
            g.LutOp: self._lut, g.LutMulOp: self._lut_mul, g.RmsNormIntOp: self._rmsnorm,
            g.SoftmaxLutOp: self._softmax, g.AddRequantOp: self._add, g.TransposeOp: self._view,
            g.ReshapeOp: self._view,
        }

    def _m(self, attr) -> int:
        v = int(attr)
        return v if self.reference else abs(v)

    def walk(self, module) -> Bounds:
        for op in g.func_of(module).ops:
            if isinstance(op, g.OutputOp):
                continue
            handler = self.handlers.get(type(op))
            if handler is None:
                raise NotImplementedError(f"int32 proof: no bound for {op.name}")
            mag, terms = handler(op)
            self.mag[op.results[0]] = mag
            if terms:
                label = op.sym_str or op.name
                self.worst[label] = max(v for _, v in terms)
                self.failures += [f"{label}: {what} can reach {v} > {INT32_MAX}" for what, v in terms if v > INT32_MAX]
        return Bounds(self.worst, self.failures, self.acc)

    # ---- one handler per op kind: (magnitude of the result, [(intermediate, bound)])
    def _input(self, op):
        return DTYPE_MAG.get(g.qt(op.result).dtype, 1 << 31), []

    def _const(self, op):
        t = g.qt(op.result)
        src = op.value if op.value is not None else self.consts[op.sym_str]
        v = np.asarray(src, dtype=np.int64).reshape(t.dims)
        self.values[op.result] = v
        return (int(np.abs(v).max()) if v.size else 0), []

    def _matmul(self, op):
        mult, s = self._m(op.M), int(op.s)
        if op.b in self.values:
            w = np.abs(self.values[op.b])
            colsum = w.sum(axis=0) if self.reference else w.sum(axis=-2)
            acc = self.mag[op.a] * int(colsum.max())
        else:
            acc = g.qt(op.a).dims[-1] * self.mag[op.a] * self.mag[op.b]
        self.acc[op.result] = acc
        out = self.mag[op.lut] if op.lut is not None else DTYPE_MAG[g.qt(op.result).dtype]
        return out, [("accumulator", acc), ("requant numerator", acc * mult + half(s))]

    def _lut(self, op):
        return self.mag[op.table], []

    def _lut_mul(self, op):
        prod = self.mag[op.table] * self.mag[op.y]
        return 128, [("table * y", prod), ("requant numerator", prod * self._m(op.M) + half(int(op.s)))]

    def _rmsnorm(self, op):
        mult, s = self._m(op.M), int(op.s)
        d, n = g.qt(op.x).dims[-1], g.qt(op.lut).dims[0]
        c, e = op.ss_shift_int, op.ss_init_int
        mx, mw = self.mag[op.x], self.mag[op.w]
        if g.qt(op.x).dtype == "i8" and c == 0 and e == 0:
            # int8 rows: every entry at its dtype bound and the table at its largest entry
            kmax = loudest_row_steps(d, n, mx)
            xwr = mx * mw * self.mag[op.lut]
            terms = [("sum of squares", d * mx * mx), ("x * w * table", xwr),
                     ("requant numerator", xwr * mult + half(s + kmax))]
        else:
            if op.lut not in self.values:
                raise ValueError(f"{op.sym_str or op.name}: a wide rmsnorm is bounded through its rsqrt table, "
                                 "which must be a const")
            row = WideRow(d, n, c, mx, e)
            kmax, table = row.kmax, self.values[op.lut]
            terms = [("rounded square", mx * mx + half(c)), ("sum of squares", d * ((mx * mx + half(c)) >> c) + e),
                     ("x * w", mx * mw), ("x * w * table", row.worst_product(table, mw)),
                     ("requant numerator", max(row.numerators(table, mw, mult, s).values()))]
        if s + kmax > 31:
            self.failures.append(f"{op.sym_str or op.name}: requant shift s + kmax = {s + kmax} exceeds 31")
        return 128, terms

    def _softmax(self, op):
        one, top, t = int(op.one), self.mag[op.lut], g.qt(op.x).dims[-1]
        return one, [("row sum", t * top), ("numerator", top * one + t * top // 2)]

    def _add(self, op):
        num = self.mag[op.a] * self._m(op.Ma) + self.mag[op.b] * self._m(op.Mb) + half(int(op.s))
        return DTYPE_MAG[g.qt(op.result).dtype], [("requant numerator", num)]

    def _view(self, op):
        """A const seen through a transpose or reshape. The reference policy keeps the operand's array as it was
        (anvil/frontend/quantize.py:242-245), so its column sums follow the original axes; the sound policy applies
        the view, so a later matmul sums |w| over the K axis the product really contracts."""
        if op.x in self.values:
            v = self.values[op.x]
            if not self.reference:
                v = (np.transpose(v, op.perm_list) if isinstance(op, g.TransposeOp)
                     else v.reshape(g.qt(op.result).dims))
            self.values[op.result] = v
        return self.mag[op.x], []


def int32_bounds(module, consts=None, *, reference: bool = False) -> Bounds:
    """The int32 analysis of a graph under one policy (BoundWalker); never raises for a bound."""
    return BoundWalker(consts, reference).walk(module)


def prove_no_overflow(module, consts=None) -> dict:
    """The reference's compile-time check (anvil/frontend/quantize.py:175-253, called by anvil/driver.py:119-132):
    {op sym: worst |intermediate|} when every bound holds under its rules, else OverflowError naming each op."""
    b = int32_bounds(module, consts, reference=True)
    if not b.ok:
        raise OverflowError("int32 overflow possible: " + "; ".join(b.failures))
    return b.worst
