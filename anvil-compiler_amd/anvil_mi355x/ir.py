"""anvil.graph without xDSL: quantized tensor ops on SSA values of type qtensor<shape x dtype[, scale]>.

Mirrors the op set, properties and verifier rules of the reference dialect (anvil/ir/graph.py:63-348) and its
GraphBuilder (anvil/ir/graph.py:361-455), so graphs built for the reference's interpreter build here with the same
calls:

    g = GraphBuilder("mlp"); x = g.input("x", [4, 8], scale=0.03); ...; g.output(out); module = g.module()

Every value is a whole tensor. Requant constants (M, s, Ma, Mb, one, ...) are plain int properties of the op;
weights and LUTs are `const` ops bound by sym (or carried inline as `value`).

    input {sym}                         -> t     graph input
    const {sym[, value]}                -> t     weight / LUT
    qmatmul (a, b[, lut]) {M, s}        -> i8|i16  requant(a @ b), optional lut[. + 128] epilogue (i8 only);
                                                 a (..., M, K) @ b (K, N) or head-batched b (..., K, N)
    qlinear (x, w[, lut]) {M, s}        -> i8|i16  qmatmul whose w is a 2-D const (K, N)
    lut (x, table)                      -> i8    table[x + 128]
    lut_mul (x, y, table) {M, s}        -> i8    requant(table[x + 128] * y, M, s)
    rmsnorm_int (x, w, lut) {M, s, ss_shift, ss_init} -> i8
    softmax_lut (x, lut) {one, causal}  -> i8|i32
    add_requant (a, b) {Ma, Mb, s}      -> i8|i16
    transpose (x) {perm}, reshape (x)            layout
    output (values...)
"""
from __future__ import annotations

import math
from dataclasses import dataclass

DTYPES = {"i8": 8, "i16": 16, "i32": 32}
WIDE = ("i8", "i16")                       # residual-stream dtypes (reference ADR-004)


class VerifyException(Exception):
    """A graph op that breaks the dialect's typing rules (the reference raises xDSL's VerifyException)."""


@dataclass(frozen=True)
class QTensorType:
    """qtensor<dims x dtype[, scale]> (anvil/ir/graph.py:67-113). scale is None for LUTs and scale-free ints."""
    shape: tuple
    dtype: str = "i8"
    scale: float | None = None

    def __init__(self, shape, dtype="i8", scale=None):
        if dtype not in DTYPES:
            raise ValueError(f"dtype {dtype!r} not in {sorted(DTYPES)}")
        object.__setattr__(self, "shape", tuple(int(d) for d in shape))
        object.__setattr__(self, "dtype", dtype)
        object.__setattr__(self, "scale", None if scale is None else float(scale))
        if any(d < 1 for d in self.shape):
            raise VerifyException(f"qtensor dims must be positive, got {list(self.shape)}")

    @property
    def dims(self) -> list:
        return list(self.shape)

    @property
    def qscale(self):
        return self.scale

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    def __str__(self):
        s = "".join(f"{d}x" for d in self.shape) + self.dtype
        return f"qtensor<{s}{'' if self.scale is None else f', {self.scale:.17e}'}>"


class Value:
    """An SSA value: the single result of `owner`."""
    __slots__ = ("type", "owner")

    def __init__(self, type_: QTensorType, owner):
        self.type, self.owner = type_, owner

    def __repr__(self):
        return f"Value({self.owner.name} {self.owner.sym_str!r}: {self.type})"


def qt(value) -> QTensorType:
    t = getattr(value, "type", None)
    if not isinstance(t, QTensorType):
        raise VerifyException(f"expected a qtensor, got {t}")
    return t


class Op:
    """A graph op: named operands (Values or None), int/bool/list properties, at most one result."""
    name = "anvil.graph.op"
    OPERANDS: tuple = ()
    OPTIONAL: tuple = ()
    PROPS: tuple = ()

    def __init__(self, operands: dict, props: dict, result_type: QTensorType | None, sym: str | None = None):
        self.sym = sym
        self.props = dict(props)
        self._operands = {}
        for n in self.OPERANDS:
            v = operands.get(n)
            if v is None and n not in self.OPTIONAL:
                raise VerifyException(f"{self.name}: missing operand {n!r}")
            self._operands[n] = v
        self.results = [] if result_type is None else [Value(result_type, self)]

    def __getattr__(self, item):
        d = self.__dict__
        if item in d.get("_operands", {}):
            return d["_operands"][item]
        if item in d.get("props", {}):
            return d["props"][item]
        raise AttributeError(item)

    @property
    def sym_str(self):
        return self.sym

    @property
    def result(self):
        return self.results[0]

    @property
    def operands(self) -> list:
        return [v for v in self._operands.values() if v is not None]

    def operand_items(self):
        return [(n, v) for n, v in self._operands.items() if v is not None]

    def verify(self):
        pass

    def _expect(self, cond, msg):
        if not cond:
            raise VerifyException(f"{self.name}: {msg}")

    def _check_shift(self, *names):
        for n in names:
            s = int(self.props[n])
            if not 0 <= s <= 31:
                raise VerifyException(f"{self.name}: {n}={s} outside [0, 31]")

    def _lut256_i8(self, value):
        t = qt(value)
        self._expect(t.dims == [256] and t.dtype == "i8", f"LUT must be 256 x i8, got {t.dims} x {t.dtype}")

    def __repr__(self):
        return f"<{self.name} {self.sym!r}>"


class InputOp(Op):
    name = "anvil.graph.input"


class ConstOp(Op):
    name = "anvil.graph.const"
    PROPS = ("value",)

    def verify(self):
        self._expect(self.sym is not None or self.props.get("value") is not None, "needs a sym or an inline value")
        v = self.props.get("value")
        if v is not None:
            import numpy as np
            self._expect(list(np.shape(v)) == qt(self.result).dims, "value shape != result shape")

    @property
    def value(self):
        return self.props.get("value")


class _MatmulBase(Op):
    OPERANDS = ("a", "b", "lut")
    OPTIONAL = ("lut",)
    PROPS = ("M", "s")

    def verify(self):
        a, b, r = qt(self.a), qt(self.b), qt(self.result)
        self._expect(a.dtype == b.dtype == "i8" and r.dtype in WIDE, "operands must be i8, the result i8 or i16")
        self._expect(r.dtype == "i8" or self.lut is None, "a LUT epilogue needs an i8 result")
        self._expect(len(a.dims) >= 2 and (len(b.dims) == 2 or (len(b.dims) == len(a.dims)
                                                                 and b.dims[:-2] == a.dims[:-2])),
                     f"shapes {a.dims} @ {b.dims}: need (..., M, K) @ (K, N) or (..., M, K) @ (..., K, N)")
        self._expect(a.dims[-1] == b.dims[-2], f"contraction mismatch {a.dims} @ {b.dims}")
        self._expect(r.dims == a.dims[:-1] + [b.dims[-1]], f"result {r.dims} != {a.dims[:-1] + [b.dims[-1]]}")
        self._check_shift("s")
        if self.lut is not None:
            self._lut256_i8(self.lut)


class QMatmulOp(_MatmulBase):
    name = "anvil.graph.qmatmul"


class QLinearOp(_MatmulBase):
    name = "anvil.graph.qlinear"

    def verify(self):
        super().verify()
        self._expect(isinstance(self.b.owner, ConstOp), "weight operand must be an anvil.graph.const")
        self._expect(len(qt(self.b).dims) == 2, "weight operand must be (K, N)")


class LutOp(Op):
    name = "anvil.graph.lut"
    OPERANDS = ("x", "table")

    def verify(self):
        self._expect(qt(self.x).dtype == qt(self.result).dtype == "i8", "x and result must be i8")
        self._expect(qt(self.x).dims == qt(self.result).dims, "shape changes")
        self._lut256_i8(self.table)


class LutMulOp(Op):
    name = "anvil.graph.lut_mul"
    OPERANDS = ("x", "y", "table")
    PROPS = ("M", "s")

    def verify(self):
        x, y, r = qt(self.x), qt(self.y), qt(self.result)
        self._expect(x.dtype == y.dtype == r.dtype == "i8", "operands and result must be i8")
        self._expect(x.dims == y.dims == r.dims, f"shapes {x.dims}, {y.dims} -> {r.dims}")
        self._lut256_i8(self.table)
        self._check_shift("s")


class RmsNormIntOp(Op):
    name = "anvil.graph.rmsnorm_int"
    OPERANDS = ("x", "w", "lut")
    PROPS = ("M", "s", "ss_shift", "ss_init")

    @property
    def ss_shift_int(self) -> int:
        return int(self.props.get("ss_shift") or 0)

    @property
    def ss_init_int(self) -> int:
        return int(self.props.get("ss_init") or 0)

    def verify(self):
        x, w, lut, r = qt(self.x), qt(self.w), qt(self.lut), qt(self.result)
        self._expect(w.dtype == r.dtype == "i8" and x.dtype in WIDE, "x must be i8 or i16, w and result i8")
        self._expect(0 <= self.ss_shift_int <= 30, f"ss_shift={self.ss_shift_int} outside [0, 30]")
        self._expect(0 <= self.ss_init_int < 1 << 31, f"ss_init={self.ss_init_int} outside int32")
        self._expect(w.dims == x.dims[-1:], f"weight {w.dims} != [{x.dims[-1]}]")
        self._expect(len(lut.dims) == 1 and lut.dtype == "i32", "rsqrt LUT must be 1-D i32")
        self._expect(r.dims == x.dims, "shape changes")
        self._check_shift("s")


class SoftmaxLutOp(Op):
    name = "anvil.graph.softmax_lut"
    OPERANDS = ("x", "lut")
    PROPS = ("one", "causal")

    def verify(self):
        x, lut, r = qt(self.x), qt(self.lut), qt(self.result)
        self._expect(x.dtype == "i8" and len(x.dims) >= 2, "scores must be i8 with rank >= 2")
        self._expect(lut.dims == [256] and lut.dtype == "i32", "exp LUT must be 256 x i32")
        self._expect(r.dims == x.dims, "shape changes")
        one = int(self.one)
        self._expect(one >= 1 and (r.dtype == "i32" or one <= 127), f"one={one} does not fit result {r.dtype}")


class AddRequantOp(Op):
    name = "anvil.graph.add_requant"
    OPERANDS = ("a", "b")
    PROPS = ("Ma", "Mb", "s")

    def verify(self):
        a, b, r = qt(self.a), qt(self.b), qt(self.result)
        self._expect({a.dtype, b.dtype, r.dtype} <= set(WIDE), "operands and result must be i8 or i16")
        self._expect(a.dims == b.dims == r.dims, f"shapes {a.dims} + {b.dims} -> {r.dims}")
        self._check_shift("s")


class TransposeOp(Op):
    name = "anvil.graph.transpose"
    OPERANDS = ("x",)
    PROPS = ("perm",)

    @property
    def perm_list(self) -> list:
        return [int(p) for p in self.perm]

    def verify(self):
        x, r, p = qt(self.x), qt(self.result), self.perm_list
        self._expect(sorted(p) == list(range(len(x.dims))), f"perm {p} is not a permutation of rank {len(x.dims)}")
        self._expect(r.dims == [x.dims[i] for i in p] and r.dtype == x.dtype, "result type mismatch")


class ReshapeOp(Op):
    name = "anvil.graph.reshape"
    OPERANDS = ("x",)

    def verify(self):
        x, r = qt(self.x), qt(self.result)
        self._expect(math.prod(x.dims) == math.prod(r.dims) and x.dtype == r.dtype, "reshape changes size or dtype")


class OutputOp(Op):
    name = "anvil.graph.output"

    def __init__(self, values):
        super().__init__({}, {}, None)
        self.values = list(values)

    @property
    def operands(self):
        return list(self.values)

    def operand_items(self):
        return [(f"v{i}", v) for i, v in enumerate(self.values)]


OPS = {c.name: c for c in (InputOp, ConstOp, QMatmulOp, QLinearOp, LutOp, LutMulOp, RmsNormIntOp, SoftmaxLutOp,
                           AddRequantOp, TransposeOp, ReshapeOp, OutputOp)}


class FuncOp:
    """anvil.graph.func {sym_name}: one block of ops in program order."""
    name = "anvil.graph.func"

    def __init__(self, sym_name: str, ops=()):
        self.sym_name = sym_name
        self.ops = list(ops)
        self.parent = None


class Module:
    """builtin.module holding graph funcs."""

    def __init__(self, *funcs):
        self.ops = list(funcs)
        for f in funcs:
            f.parent = self


def funcs(module) -> list:
    return [op for op in module.ops if isinstance(op, FuncOp)]


def func_of(m) -> FuncOp:
    """The single graph func of a module (or the func itself), as the reference interpreter's _func."""
    if isinstance(m, FuncOp):
        return m
    fs = funcs(m)
    if len(fs) != 1:
        raise ValueError(f"expected one anvil.graph.func, found {len(fs)}")
    return fs[0]


class GraphBuilder:
    """Appends verified graph ops to a func; every method returns the result value (reference
    anvil/ir/graph.py:361-455, same signatures)."""

    def __init__(self, sym_name: str):
        self.func = FuncOp(sym_name)
        self._module = None

    def _add(self, op):
        self.func.ops.append(op)
        try:
            op.verify()
        except Exception:
            self.func.ops.pop()
            raise
        return op.results[0] if op.results else op

    def input(self, sym, shape, dtype="i8", scale=None):
        return self._add(InputOp({}, {}, QTensorType(shape, dtype, scale), sym))

    def const(self, sym, shape, dtype="i8", scale=None, value=None):
        if value is not None:
            import numpy as np
            value = np.asarray(value, dtype=np.int64).reshape(list(shape))
        return self._add(ConstOp({}, {"value": value}, QTensorType(shape, dtype, scale), sym))

    def _mm(self, cls, sym, a, b, m, s, scale, lut, dtype="i8"):
        out = qt(a).dims[:-1] + [qt(b).dims[-1]]
        return self._add(cls({"a": a, "b": b, "lut": lut}, {"M": int(m), "s": int(s)},
                             QTensorType(out, dtype, scale), sym))

    def qmatmul(self, sym, a, b, m, s, scale=None, lut=None, dtype="i8"):
        return self._mm(QMatmulOp, sym, a, b, m, s, scale, lut, dtype)

    def qlinear(self, sym, x, w, m, s, scale=None, lut=None, dtype="i8"):
        return self._mm(QLinearOp, sym, x, w, m, s, scale, lut, dtype)

    def lut(self, sym, x, table, scale=None):
        return self._add(LutOp({"x": x, "table": table}, {}, QTensorType(qt(x).dims, "i8", scale), sym))

    def lut_mul(self, sym, x, y, table, m, s, scale=None):
        return self._add(LutMulOp({"x": x, "y": y, "table": table}, {"M": int(m), "s": int(s)},
                                  QTensorType(qt(x).dims, "i8", scale), sym))

    def rmsnorm_int(self, sym, x, w, lut, m, s, scale=None, ss_shift=0, ss_init=0):
        return self._add(RmsNormIntOp({"x": x, "w": w, "lut": lut},
                                      {"M": int(m), "s": int(s), "ss_shift": int(ss_shift), "ss_init": int(ss_init)},
                                      QTensorType(qt(x).dims, "i8", scale), sym))

    def softmax_lut(self, sym, x, lut, one, causal=True, scale=None, dtype="i8"):
        return self._add(SoftmaxLutOp({"x": x, "lut": lut}, {"one": int(one), "causal": bool(causal)},
                                      QTensorType(qt(x).dims, dtype, scale), sym))

    def add_requant(self, sym, a, b, ma, mb, s, scale=None, dtype="i8"):
        return self._add(AddRequantOp({"a": a, "b": b}, {"Ma": int(ma), "Mb": int(mb), "s": int(s)},
                                      QTensorType(qt(a).dims, dtype, scale), sym))

    def transpose(self, sym, x, perm=None, scale=None):
        t = qt(x)
        perm = [int(p) for p in perm] if perm is not None else list(range(len(t.dims)))[::-1]
        sc = t.qscale if scale is None else scale
        if sorted(perm) != list(range(len(t.dims))):
            raise VerifyException(f"{TransposeOp.name}: perm {perm} is not a permutation of rank {len(t.dims)}")
        return self._add(TransposeOp({"x": x}, {"perm": perm}, QTensorType([t.dims[i] for i in perm], t.dtype, sc),
                                     sym))

    def reshape(self, sym, x, shape, scale=None):
        t = qt(x)
        return self._add(ReshapeOp({"x": x}, {}, QTensorType(shape, t.dtype, t.qscale if scale is None else scale),
                                   sym))

    def output(self, *values):
        self._add(OutputOp(values))

    def module(self) -> Module:
        """The module holding the func (built once; later calls return the same module)."""
        if self._module is None:
            self._module = Module(self.func)
        return self._module


def print_ir(module) -> str:
    """The module in the reference's textual (MLIR generic) form (anvil/ir/__init__.py:22-25)."""
    from .ir_text import print_ir as _print
    return _print(module)


def parse_ir(text: str):
    """A module from the reference's textual form (anvil/ir/__init__.py:28-31)."""
    from .ir_text import parse_ir as _parse
    return _parse(text)
