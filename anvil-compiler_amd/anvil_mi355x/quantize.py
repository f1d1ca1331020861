"""Quantization recipe (host setup, run once per model): fixed-point multipliers, LUT builders, overflow proof.

Restates the reference's anvil/frontend/quantize.py:32-253 (contract 8, symmetric per-tensor int8):

    fixed_point(ms, bounds, k)    largest shift s with sum(bound_i * round(m_i 2^s)) + 2^(s+k-1) <= INT32_MAX
    rmsnorm_lut / rmsnorm_lut_wide  rsqrt LUTs for rmsnorm_int (i8 rows; i16 rows with ss_shift / ss_init)
    exp_bits / exp_lut            softmax_lut's exp table, exp_lut[d + 255] = round(exp(d s) 2^E)
    act_lut(f, s_in, s_out)       any int8 -> int8 activation (SiLU, GELU) as a 256-entry LUT
    prove_no_overflow(module)     propagate magnitude bounds and bound every int32 intermediate of every op

The MI355X kernels compute every requant numerator in 64 bits and flag, rather than wrap, a value outside int32;
prove_no_overflow is what makes such a flag impossible for the graphs compile() accepts.
"""
from __future__ import annotations

import math

import numpy as np

from . import ir as g

INT32_MAX = (1 << 31) - 1
RSQRT_LEN = 1024
SOFTMAX_ONE = 127
HEADROOM = 1.5
QMAX = {"i8": 127, "i16": (1 << 15) - 1}


def _rnd(s):
    return (1 << (s - 1)) if s else 0


def rsqrt_index(ss: int, n: int):
    """(idx, k) for one row sum: shift right by 2 until below n, counting steps (reference codegen/lower.py:107-113)."""
    ss, k = int(ss), 0
    while ss >= n:
        ss >>= 2
        k += 1
    return ss, k


def fixed_point(ms, bounds, k=0, *, max_shift=31):
    """(M_i, s): the largest s in [0, max_shift - k] with M_i = round(m_i 2^s) and
    sum(bound_i M_i) + 2^(s+k-1) <= INT32_MAX (reference quantize.py:40-56). ValueError if a multiplier vanishes
    at the chosen shift, OverflowError if no shift fits."""
    if len(ms) != len(bounds) or not ms:
        raise ValueError("fixed_point needs one bound per multiplier")
    if any(m <= 0 for m in ms) or any(b < 0 for b in bounds):
        raise ValueError(f"multipliers must be positive and bounds non-negative: {ms}, {bounds}")
    for s in range(max_shift - k, -1, -1):
        mi = [round(m * (1 << s)) for m in ms]
        if sum(int(b) * m for b, m in zip(bounds, mi)) + ((1 << (s + k - 1)) if s + k else 0) <= INT32_MAX:
            if min(mi) < 1:
                raise ValueError(f"multipliers {ms} vanish at shift {s}")
            return mi, s
    raise OverflowError(f"bounds {bounds} leave no room for multipliers {ms}")


def maxabs_scale(x) -> float:
    return float(np.abs(np.asarray(x)).max()) / 127


def quantize_array(x, scale):
    return np.clip(np.rint(np.asarray(x) / scale), -128, 127).astype(np.int64)


def rsqrt_kmax(d, n=RSQRT_LEN, mag=128):
    """Normalisation steps rmsnorm_int takes on the loudest row of d entries of magnitude mag."""
    return rsqrt_index(d * mag * mag, n)[1]


def rmsnorm_lut(sx, sw, sh, wmax, d, eps, n=RSQRT_LEN):
    """(rsqrt_lut, s) for an i8 row (reference quantize.py:72-80): lut[i] = round(rsqrt(sx^2 i / d + eps) sx sw / sh
    2^s), lut[0] = 0."""
    ss = np.arange(1, n)
    r = np.r_[0, 1 / np.sqrt(sx ** 2 * ss / d + eps) * sx * sw / sh]
    (rmax,), s = fixed_point([r.max()], [128 * wmax], rsqrt_kmax(d, n))
    lut = np.rint(r * (1 << s)).astype(np.int64)
    assert lut.max() == rmax
    return lut, s


def ss_shift_for(d, mag):
    """Least c with d ((mag^2 + 2^(c-1)) >> c) <= INT32_MAX (reference quantize.py:85-91)."""
    for c in range(31):
        if d * ((mag * mag + _rnd(c)) >> c) <= INT32_MAX:
            return c
    raise OverflowError(f"no square shift fits {d} entries of magnitude {mag}")


def _xmax(ss_max, c, mag):
    return min(mag, math.isqrt(max(0, (ss_max + 1) * (1 << c) - _rnd(c) - 1)))


def rms_xmax_table(d, n, c, mag, e=0):
    """{k: largest |x| a row with rsqrt_index(ss) = (i, k) can hold, per LUT index i} (reference
    quantize.py:99-113)."""
    ss_top = d * ((mag * mag + _rnd(c)) >> c) + e
    kmax = rsqrt_index(ss_top, n)[1]
    out = {}
    for k in range(kmax + 1):
        hi = np.minimum((np.arange(n, dtype=object) + 1) * (4 ** k) - 1, ss_top)
        xm = np.array([_xmax(int(v) - e, c, mag) if v >= e else 0 for v in hi], dtype=np.int64)
        if k:
            xm[: n // 4] = 0
        out[k] = xm
    return out


def rms_wide_bounds(lut, wmax, M, s, xm_table):
    lut = np.asarray(lut, dtype=np.int64)
    return {k: int((xm * wmax * lut).max()) * M + _rnd(s + k) for k, xm in xm_table.items()}


def rmsnorm_lut_wide(sx, sw, sh, wmax, d, eps, mag, n=RSQRT_LEN):
    """(rsqrt_lut, s, c, e) for an i16 row with eps folded into the sum (reference quantize.py:122-144)."""
    c = ss_shift_for(d, mag)
    unit = sx ** 2 * (1 << c) / d
    e = max(1, int(round(eps / unit)))
    if d * ((mag * mag + _rnd(c)) >> c) + e > INT32_MAX:
        raise OverflowError(f"eps folds to {e}: the rmsnorm sum of squares cannot stay in int32 at scale {sx}")
    ss = np.arange(1, n)
    r = np.r_[0, 1 / np.sqrt(unit * ss) * sx * sw / sh]
    xm = rms_xmax_table(d, n, c, mag, e)
    kmax = max(xm)
    for s in range(31 - kmax, -1, -1):
        lut = np.rint(r * (1 << s)).astype(np.int64)
        if max(rms_wide_bounds(lut, wmax, 1, s, xm).values()) <= INT32_MAX:
            if lut[n // 4:].min() < 64:
                raise ValueError(f"rsqrt LUT too coarse at shift {s} (min entry {lut[n // 4:].min()})")
            return lut, s, c, e
    raise OverflowError("no rsqrt LUT shift fits a wide rmsnorm")


def exp_bits(t, one=SOFTMAX_ONE):
    """Largest E with every softmax_lut intermediate in int32 for rows of t entries <= 2^E (reference
    quantize.py:155-157)."""
    return max(e for e in range(31) if (one + t // 2) << e <= INT32_MAX and t << e <= INT32_MAX)


def exp_lut(score_scale, t, one=SOFTMAX_ONE):
    """exp_lut[d + 255] = round(exp(d score_scale) 2^E), d in [-255, 0] (reference quantize.py:160-162)."""
    return np.rint(np.exp(np.arange(-255, 1) * score_scale) * (1 << exp_bits(t, one))).astype(np.int64)


def silu(x):
    return x / (1 + np.exp(-x))


def gelu(x):
    """GELU, erf form (torch.nn.GELU's default)."""
    from scipy.special import erf
    return 0.5 * x * (1 + erf(np.asarray(x, dtype=np.float64) / math.sqrt(2)))


def act_lut(f, s_in, s_out):
    """int8 activation LUT: quantize_array(f(i s_in), s_out) for i in [-128, 127], the reference's recipe for an
    unfused SiLU node (quantize.py:446-452), applied here to any elementwise activation."""
    return quantize_array(f(np.arange(-128, 128) * s_in), s_out)


def silu_lut(s_in):
    """(lut, scale): SiLU at its own max-abs scale (reference quantize.py:147-152)."""
    y = silu(np.arange(-128, 128) * s_in)
    s = maxabs_scale(y)
    return quantize_array(y, s), s


# ----------------------------------------------------------------------------------------- overflow proof

def prove_no_overflow(module, consts=None, acc_bounds: dict | None = None) -> dict:
    """Magnitude propagation over the graph (reference quantize.py:175-253): int8 inputs 128, i16 2^15, softmax
    outputs `one`, LUT outputs max|table|. Returns {op sym: worst |intermediate|}; raises OverflowError naming
    every op whose bound exceeds INT32_MAX. acc_bounds, when given, receives {matmul result value: bound on its
    |accumulator|} (what lets a kernel use a 24-bit requant multiply)."""
    consts = consts or {}
    mag, cval, worst, bad = {}, {}, {}, []
    for op in g.func_of(module).ops:
        if isinstance(op, g.OutputOp):
            continue
        r = op.results[0]
        name = op.sym_str or op.name
        checks = {}
        if isinstance(op, g.InputOp):
            m = {"i8": 128, "i16": 1 << 15}.get(g.qt(r).dtype, 1 << 31)
        elif isinstance(op, g.ConstOp):
            v = (np.asarray(op.value, dtype=np.int64).reshape(g.qt(r).dims) if op.value is not None
                 else np.asarray(consts[op.sym_str], dtype=np.int64))
            cval[r] = v
            m = int(np.abs(v).max()) if v.size else 0
        elif isinstance(op, (g.QMatmulOp, g.QLinearOp)):
            M, s = abs(int(op.M)), int(op.s)          # magnitudes: a negative multiplier flips no bound
            if op.b in cval:
                acc = mag[op.a] * int(np.abs(cval[op.b]).sum(axis=0).max())
            else:
                acc = g.qt(op.a).dims[-1] * mag[op.a] * mag[op.b]
            checks = {"acc": acc, "acc*M + round": acc * M + _rnd(s)}
            if acc_bounds is not None:
                acc_bounds[r] = acc
            m = mag[op.lut] if op.lut is not None else (128 if g.qt(r).dtype == "i8" else 1 << 15)
        elif isinstance(op, g.LutOp):
            m = mag[op.table]
        elif isinstance(op, g.LutMulOp):
            M, s = abs(int(op.M)), int(op.s)          # magnitudes: a negative multiplier flips no bound
            prod = mag[op.table] * mag[op.y]
            checks = {"lut*y": prod, "lut*y*M + round": prod * M + _rnd(s)}
            m = 128
        elif isinstance(op, g.RmsNormIntOp):
            M, s = abs(int(op.M)), int(op.s)          # magnitudes: a negative multiplier flips no bound
            d, n = g.qt(op.x).dims[-1], g.qt(op.lut).dims[0]
            c, e = op.ss_shift_int, op.ss_init_int
            if g.qt(op.x).dtype == "i8" and c == 0 and e == 0:
                kmax = rsqrt_kmax(d, n, mag[op.x])
                xwr = mag[op.x] * mag[op.w] * mag[op.lut]
                checks = {"sum x^2": d * mag[op.x] ** 2, "x*w*r": xwr, "x*w*r*M + round": xwr * M + _rnd(s + kmax)}
            else:
                if op.lut not in cval:
                    raise ValueError(f"{name}: the wide rmsnorm bound needs the rsqrt LUT's values")
                xm = rms_xmax_table(d, n, c, mag[op.x], e)
                kmax = max(xm)
                lut = cval[op.lut]
                xwr = max(int((v * mag[op.w] * lut).max()) for v in xm.values())
                checks = {"x^2 + round": mag[op.x] ** 2 + _rnd(c),
                          "sum x^2": d * ((mag[op.x] ** 2 + _rnd(c)) >> c) + e, "x*w": mag[op.x] * mag[op.w],
                          "x*w*r": xwr, "x*w*r*M + round": max(rms_wide_bounds(lut, mag[op.w], M, s, xm).values())}
            if s + kmax > 31:
                bad.append(f"{name}: shift s + kmax = {s + kmax} > 31")
            m = 128
        elif isinstance(op, g.SoftmaxLutOp):
            one, emax, t = int(op.one), mag[op.lut], g.qt(op.x).dims[-1]
            checks = {"exp sum": t * emax, "e*one + S/2": emax * one + t * emax // 2}
            m = one
        elif isinstance(op, g.AddRequantOp):
            Ma, Mb, s = abs(int(op.Ma)), abs(int(op.Mb)), int(op.s)
            checks = {"a*Ma + b*Mb + round": mag[op.a] * Ma + mag[op.b] * Mb + _rnd(s)}
            m = 128 if g.qt(r).dtype == "i8" else 1 << 15
        elif isinstance(op, (g.TransposeOp, g.ReshapeOp)):
            m = mag[op.x]
            if op.x in cval:
                cval[r] = cval[op.x]
        else:
            raise NotImplementedError(f"prove_no_overflow: {op.name}")
        mag[r] = m
        if checks:
            worst[name] = max(checks.values())
            bad += [f"{name}: {k} reaches {v} > {INT32_MAX}" for k, v in checks.items() if v > INT32_MAX]
    if bad:
        raise OverflowError("int32 overflow possible: " + "; ".join(bad))
    return worst
