"""ORACLE (test infrastructure only): numpy restatement of the reference's checked-int32 tensor semantics.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker or the timed CPU baseline. The product path (anvil_mi355x) never imports it.

Restates `anvil/semantics.py` (all tensor ops) and the `xf.golden` ops it re-exports
(`anvil/semantics.py:15-28`). `xf.golden` lives in the reference's un-vendored submodule `sim/`
(github.com/Ashtonantony28/Didactic_GPU_Simulator @ 096c6ef, absent from /root/reference), so its ops are restated
from the reference's own in-tree restatements of them, each cited below:

    requant          anvil/semantics.py:146-155 (requant_dtype, identical for i8), anvil/backend/idioms.py:1-23,
                     anvil/vortexv/codegen.py:10-13, docs/vortexv-backend.md:24-29
    matmul_i8        numpy int64 `@` checked against int32 (docs/decisions/ADR-003-multihead.md:31)
    residual_add     anvil/semantics.py:106-115 (the all-i8 case of add_requant)
    swiglu_lut       anvil/interp/graph.py:67-68, anvil/lower/graph_to_tensor.py:293-296,
                     anvil/vortexv/codegen.py:414-427
    rsqrt_index      anvil/codegen/lower.py:107-113, anvil/vortexv/codegen.py:512-519
    rmsnorm_int      anvil/semantics.py:158-182 (rmsnorm_wide with c = e = 0), anvil/lower/graph_to_tensor.py:319-349,
                     anvil/vortexv/codegen.py:480-543
    softmax_lut      anvil/lower/graph_to_tensor.py:352-398, anvil/vortexv/codegen.py:545-615,
                     tests/interp/test_tensor_interp.py:103-128

Every value is an int64 numpy array. Intermediates are checked against int32 in the reference's order and raise
OverflowError when they leave it; int8 operands outside int8 raise ValueError.

Pinning (tests/test_oracle_*.py): the known answers the reference's tests hold (requant, add_requant clamps,
i16 clamps, fixed_point), brute-force scalar loops, closed forms (softmax of a constant row, rmsnorm of a zero row),
float64-exact matmul, and the independent scalar C restatement oracle/scalar_oracle.c on random graphs.
Which exception type xf.golden raises on out-of-contract inputs is parity unpinned (only an import could pin it).
"""
import numpy as np

I8 = (-128, 127)
I16 = (-(1 << 15), (1 << 15) - 1)
I32 = (-(1 << 31), (1 << 31) - 1)
DT_RANGE = {"i8": I8, "i16": I16, "i32": I32}


# ---------------------------------------------------------------------------------------------- checked ints

def check_i32(x, what="value"):
    """x as int64, OverflowError if any element leaves int32 (reference semantics.py:47-49)."""
    x = np.asarray(x, dtype=np.int64)
    if x.size and (x.min() < I32[0] or x.max() > I32[1]):
        raise OverflowError(f"{what} overflows int32")
    return x


def check_i8(x, what="value"):
    """x as int64, ValueError if any element leaves int8 (reference semantics.py:52-54)."""
    x = np.asarray(x, dtype=np.int64)
    if x.size and (x.min() < I8[0] or x.max() > I8[1]):
        raise ValueError(f"{what} is not int8")
    return x


def check_dtype(x, dtype, what="value"):
    """Range check at a graph dtype (reference semantics.py:129-139)."""
    if dtype == "i32":
        return check_i32(x, what)
    if dtype == "i8":
        return check_i8(x, what)
    lo, hi = DT_RANGE[dtype]
    x = np.asarray(x, dtype=np.int64)
    if x.size and (x.min() < lo or x.max() > hi):
        raise ValueError(f"{what} is not int{dtype[1:]}")
    return x


def clamp_dtype(x, dtype):
    return np.clip(np.asarray(x, dtype=np.int64), *DT_RANGE[dtype])


def clamp_i8(x):
    return clamp_dtype(x, "i8")


def round_term(s):
    """2^(s-1), 0 when s == 0; ValueError outside [0, 31] (reference semantics.py:57-62)."""
    s = int(s)
    if not 0 <= s <= 31:
        raise ValueError(f"shift {s} outside [0, 31]")
    return (1 << (s - 1)) if s else 0


# -------------------------------------------------------------------------------------------- golden ops

def requant_dtype(acc, m, s, dtype="i8"):
    """clamp_dtype(chk(chk(chk(acc) * M) + rnd(s)) >> s): arithmetic (floor) shift (reference
    semantics.py:146-155; the i8 case is golden.requant)."""
    rnd = round_term(s)
    acc = check_i32(acc, "acc")
    prod = check_i32(acc * int(m), "acc*M")
    rounded = check_i32(prod + rnd, "acc*M + round")
    return clamp_dtype(rounded >> int(s), dtype)


def requant(acc, m, s):
    return requant_dtype(acc, m, s, "i8")


def matmul_i8(a, b, fast=False):
    """int8 x int8 -> int32-checked int64: numpy `@` over int64 (batched over leading dims), the reference's
    literal path. fast=True multiplies in float64 BLAS instead: every product and partial sum is an integer of
    magnitude <= K * 2^14 < 2^53, so the float64 result is exact (a speed-up of the checker, not the baseline)."""
    a, b = check_i8(a, "a"), check_i8(b, "b")
    if fast and a.shape[-1] < (1 << 38):
        return check_i32(np.rint(a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64), "matmul")
    return check_i32(a @ b, "matmul")


def lut_i8(x, table):
    """table[x + 128], 256 int8 entries (reference semantics.py:87-92)."""
    x, table = check_i8(x, "x"), check_i8(table, "lut")
    if table.shape != (256,):
        raise ValueError("int8 LUT must have 256 entries")
    return table[x + 128]


def qmatmul(a, b, m, s, lut=None, dtype="i8", fast=False):
    """requant(a @ b, M, s) [-> lut[. + 128]]; an i16 result (no LUT) clamps to int16 (reference
    semantics.py:95-103)."""
    if dtype != "i8":
        if lut is not None:
            raise ValueError("a LUT epilogue needs an i8 result")
        return requant_dtype(matmul_i8(a, b, fast), m, s, dtype)
    out = requant(matmul_i8(a, b, fast), m, s)
    return out if lut is None else lut_i8(out, lut)


def swiglu_lut(x, y, table, m, s):
    """lut_mul: requant(table[x + 128] * y, M, s)."""
    t = lut_i8(x, table)
    y = check_i8(y, "y")
    return requant(check_i32(t * y, "lut*y"), m, s)


def _is_i8(x):
    return not x.size or (x.min() >= I8[0] and x.max() <= I8[1])


def residual_add(a, b, ma, mb, s):
    """clamp_i8((chk(chk(a*Ma) + chk(b*Mb)) + rnd(s)) >> s) on int8 operands."""
    a, b = check_i8(a, "a"), check_i8(b, "b")
    acc = check_i32(check_i32(a * int(ma), "a*Ma") + check_i32(b * int(mb), "b*Mb"), "a*Ma + b*Mb")
    return requant(acc, 1, s)


def add_requant(a, b, ma, mb, s, dtype="i8"):
    """Scale-aligned residual add (reference semantics.py:106-115): all-i8 operands and result are
    golden.residual_add; otherwise a, b may each be i8 or i16 and the result clamps to `dtype`."""
    a, b = np.asarray(a, dtype=np.int64), np.asarray(b, dtype=np.int64)
    if dtype == "i8" and _is_i8(a) and _is_i8(b):
        return residual_add(a, b, ma, mb, s)
    a, b = check_dtype(a, "i16", "a"), check_dtype(b, "i16", "b")
    acc = check_i32(check_i32(a * int(ma), "a*Ma") + check_i32(b * int(mb), "b*Mb"), "a*Ma + b*Mb")
    return requant_dtype(acc, 1, s, dtype)


def rsqrt_index(ss, n):
    """(idx, k): shift ss right by 2 until it is below n, counting the steps (reference codegen/lower.py:107-113).
    Vectorised over ss."""
    ss = np.asarray(ss, dtype=np.int64).copy()
    k = np.zeros_like(ss)
    n = int(n)
    while True:
        big = ss >= n
        if not big.any():
            return ss, k
        ss[big] >>= 2
        k[big] += 1


def sq_shift(x, c):
    """(x*x + 2^(c-1)) >> c, checked (reference semantics.py:158-161)."""
    sq = check_i32(x * x, "x*x")
    return check_i32(sq + round_term(c), "x*x + round") >> int(c)


def _requant_rows(acc, m, s, k):
    """requant with a per-row shift s + k (k broadcast over the last axis); one pass per distinct k, as the
    reference's requant_var (semantics.py:65-73)."""
    out = np.empty(acc.shape, dtype=np.int64)
    kk = np.broadcast_to(np.asarray(k)[..., None], acc.shape)
    for kv in np.unique(kk):
        sel = kk == kv
        out[sel] = requant(acc[sel], m, int(s) + int(kv))
    return out


def rmsnorm_wide(x, w, rsqrt_lut, m, s, ss_shift=0, ss_init=0, xdtype="i8"):
    """rmsnorm_int over the last axis (reference semantics.py:164-182): ss = e + sum((x^2 + 2^(c-1)) >> c),
    (i, k) = rsqrt_index(ss, len(lut)), out = requant(x * w * lut[i], M, s + k). With an i8 row and c = e = 0 this
    is golden.rmsnorm_int."""
    x = check_dtype(np.asarray(x, dtype=np.int64), xdtype, "x")
    w = check_i8(w, "w")
    lut = check_i32(rsqrt_lut, "rsqrt_lut")
    if lut.ndim != 1 or (lut.size and lut.min() < 0):
        raise ValueError("rsqrt_lut must be a non-negative 1-D table")
    c, e = int(ss_shift), int(ss_init)
    sq = sq_shift(x, c) if c else check_i32(x * x, "x*x")
    ss = check_i32(sq.sum(axis=-1) + e, "sum of squares")
    idx, k = rsqrt_index(ss, len(lut))
    xwr = check_i32(check_i32(x * w, "x*w") * lut[idx][..., None], "x*w*r")
    return _requant_rows(xwr, m, s, k)


def rmsnorm_int(x, w, rsqrt_lut, m, s):
    return rmsnorm_wide(x, w, rsqrt_lut, m, s)


def softmax_lut(x, lut, one, causal):
    """LUT softmax over the last axis of (..., T1, T2) (reference lower/graph_to_tensor.py:352-398):
    kept_j = j <= i when causal; m = max(-128, max_kept x); e_j = lut[x_j - m + 255] if kept else 0;
    S = chk(sum e); p_j = chk(e_j * one + S // 2) // S (masked p_j = 0)."""
    x = check_i8(x, "scores")
    lut = check_i32(lut, "exp_lut")
    if lut.shape != (256,):
        raise ValueError("exp LUT must have 256 entries")
    t1, t2 = x.shape[-2], x.shape[-1]
    if causal:
        keep = np.arange(t2)[None, :] <= np.arange(t1)[:, None]
    else:
        keep = np.ones((t1, t2), dtype=bool)
    keep = np.broadcast_to(keep, x.shape)
    m = np.where(keep, x, I8[0]).max(axis=-1, keepdims=True)
    e = np.where(keep, lut[np.where(keep, x - m + 255, 255)], 0)
    tot = check_i32(e.sum(axis=-1, keepdims=True), "exp sum")
    if (tot <= 0).any():
        raise ZeroDivisionError("softmax row sums to zero")
    num = check_i32(e * int(one) + tot // 2, "e*one + S/2")
    return num // tot
