"""ORACLE (test infrastructure only): restatement of the reference's graph interpreter, anvil/interp/graph.py:16-92.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

    run(module, {"x": x}, consts)               one sample: x has the graph input's shape
    run(module, {"x": xs}, consts, batch=True)  xs has a leading batch dim that every non-const value keeps

Walks the graph's ops in order, evaluates each through oracle.semantics on int64 numpy arrays, and checks every
result's shape and dtype range after the op (reference interp/graph.py:35-40). `values` holds every op that has
a sym, consts and inputs included. Transposes of batched values shift their perm by the batch dim; consts stay
unbatched (interp/graph.py:49-51,76-81,87-89). The graph is any object with the anvil.graph op structure
(op.name strings, named operands, int properties), so this module depends on no product code.

fast=True computes matmuls in float64 BLAS, which is exact for int8 operands (oracle.semantics.matmul_i8).
"""
from dataclasses import dataclass, field

import numpy as np

from . import semantics as sem


@dataclass
class GraphResult:
    outputs: list                                   # graph.output operands, in order
    values: dict = field(default_factory=dict)      # sym -> array for every op that carries a sym


def _func(m):
    if getattr(m, "name", None) == "anvil.graph.func":
        return m
    fs = [op for op in m.ops if getattr(op, "name", None) == "anvil.graph.func"]
    if len(fs) != 1:
        raise ValueError(f"expected one anvil.graph.func, found {len(fs)}")
    return fs[0]


def _check_type(op, val, lead=()):
    t = op.results[0].type
    if list(val.shape) != list(lead) + list(t.dims):
        raise ValueError(f"{op.name} {op.sym_str!r}: shape {list(val.shape)} != declared {t.dims}")
    sem.check_dtype(val, t.dtype, f"{op.name} {op.sym_str!r}")
    return val


def run(m, inputs: dict, consts: dict | None = None, *, batch: bool = False, fast: bool = False) -> GraphResult:
    """Evaluate the graph (reference interp/graph.py:43-92)."""
    consts = consts or {}
    env, res = {}, GraphResult([])
    lead, nb, is_const = (), 0, set()
    if batch:
        first = next(iter(inputs.values()))
        lead, nb = (int(np.shape(first)[0]),), 1
    for op in _func(m).ops:
        v = env.__getitem__
        n = op.name
        if n == "anvil.graph.input":
            val = np.asarray(inputs[op.sym_str], dtype=np.int64)
        elif n == "anvil.graph.const":
            is_const.add(op.results[0])
            if op.value is not None:
                val = np.asarray(op.value, dtype=np.int64).reshape(op.results[0].type.dims)
            else:
                val = np.asarray(consts[op.sym_str], dtype=np.int64)
        elif n in ("anvil.graph.qmatmul", "anvil.graph.qlinear"):
            lut = None if op.lut is None else v(op.lut)
            val = sem.qmatmul(v(op.a), v(op.b), int(op.M), int(op.s), lut, op.results[0].type.dtype, fast)
        elif n == "anvil.graph.lut":
            val = sem.lut_i8(v(op.x), v(op.table))
        elif n == "anvil.graph.lut_mul":
            val = sem.swiglu_lut(v(op.x), v(op.y), v(op.table), int(op.M), int(op.s))
        elif n == "anvil.graph.rmsnorm_int":
            val = sem.rmsnorm_wide(v(op.x), v(op.w), v(op.lut), int(op.M), int(op.s), op.ss_shift_int,
                                   op.ss_init_int, op.x.type.dtype)
        elif n == "anvil.graph.softmax_lut":
            val = sem.softmax_lut(v(op.x), v(op.lut), int(op.one), bool(op.causal))
        elif n == "anvil.graph.add_requant":
            val = sem.add_requant(v(op.a), v(op.b), int(op.Ma), int(op.Mb), int(op.s), op.results[0].type.dtype)
        elif n == "anvil.graph.transpose":
            k = 0 if op.x in is_const else nb
            val = np.transpose(v(op.x), list(range(k)) + [p + k for p in op.perm_list])
        elif n == "anvil.graph.reshape":
            k = () if op.x in is_const else lead
            val = v(op.x).reshape(list(k) + op.results[0].type.dims)
        elif n == "anvil.graph.output":
            res.outputs = [v(x) for x in op.values]
            continue
        else:
            raise NotImplementedError(n)
        if n in ("anvil.graph.transpose", "anvil.graph.reshape") and op.x in is_const:
            is_const.add(op.results[0])
        env[op.results[0]] = _check_type(op, val, () if op.results[0] in is_const else lead)
        if op.sym_str is not None:
            res.values[op.sym_str] = env[op.results[0]]
    return res
