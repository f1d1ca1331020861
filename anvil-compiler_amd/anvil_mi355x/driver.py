"""compile -> CompiledModel -> run(x, "mi355x") -> RunOutput: the reference driver's surface on MI355X.

    cm = anvil_mi355x.compile((module, consts))          # reference anvil/driver.py:330-335
    res = cm.run(x_float, "mi355x")                       # quantize x, run every graph op on the GPU, read back
    res.output, res.ints["out"], res.cycles               # dequantized output, int values, per-op device us
    cm.run(xs, "mi355x", batch=True, keep="all")          # leading batch dim (reference interp batch=True)

The reference's CompiledModel.run (anvil/driver.py:305-322) binds inputs, builds a tiny-gpu Job and dispatches it
by backend string (anvil/runtime/api.py:127-141). Here "mi355x" branches at graph level instead, as the
reference's Vortex-V backend does (anvil/vortexv/__init__.py:102-123): weights and LUTs are uploaded once per
compiled model, every value stays in HBM, ops run in graph order on one stream, and only the values `keep` asks
for come back. Transposes and reshapes are strided views (no kernel) unless a consumer needs a dense layout.

Per batch size a plan is built once and cached: buffers, views and the list of kernel launches with their
arguments, so a run is a walk over prepared calls.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import hostpar
from . import ir as g
from . import quantize as Q
from . import runtime as rt
from .layout import Buf, View, contig_strides

BACKENDS = ("mi355x",)


@dataclass
class RunOutput:
    """Reference anvil/driver.py:56-76. cycles: op sym -> device microseconds (profile=True), else None."""
    output: np.ndarray
    outputs: list
    ints: dict
    cycles: dict
    result: dict
    job: object = None
    _consts: frozenset = frozenset()
    _model: object = field(default=None, repr=False)

    def stray_writes(self, *, scratch_ok: bool = True) -> list:
        """Consts whose device copy no longer equals the uploaded values (the reference's check that a run
        wrote nothing inside a const, driver.py:66-71). Empty for a correct run."""
        return [] if self._model is None else self._model.changed_consts()

    @property
    def total_cycles(self):
        c = list(self.cycles.values())
        return None if any(v is None for v in c) else sum(c)


def _graph_meta(module):
    out = {}
    for op in g.func_of(module).ops:
        if isinstance(op, g.OutputOp) or not op.results:
            continue
        ty = g.qt(op.results[0])
        out[op.sym_str] = (ty.qscale, tuple(ty.dims), ty.dtype)
    return out


def _resolve_model(model, consts, prove=True):
    from .models import Built
    from .ir_text import parse_ir
    if isinstance(model, Built):
        return model.module, dict(model.consts)
    if isinstance(model, tuple) and len(model) == 2 and isinstance(model[0], (g.Module, str)):
        model, consts = model
    if isinstance(model, str):                  # the reference's printed IR (anvil.ir.print_ir)
        model = parse_ir(model)
    if isinstance(model, g.Module):
        return _checked_graph(model, dict(consts or {}), prove)
    raise TypeError(f"cannot compile a {type(model).__name__}: expected an anvil graph module or its printed IR, "
                    "(module, consts) or a built model (the torch capture frontend is not part of this backend)")


def _checked_graph(module, consts, prove=True):
    """Every non-inline const needs values, no unknown consts, and the int32 overflow proof must hold
    (reference driver.py:119-132)."""
    need = [op.sym_str for op in g.func_of(module).ops if isinstance(op, g.ConstOp) and op.value is None]
    missing = [s for s in need if s not in consts]
    if missing:
        raise ValueError(f"no values for graph consts {missing}: pass consts= or a (module, consts) pair")
    unknown = sorted(set(consts) - set(need))
    if unknown:
        raise ValueError(f"consts {unknown} name no graph const of the module")
    if prove:
        Q.prove_no_overflow(module, consts)
    return module, consts


PINNED_MAX = 1 << 28       # read-back buffers up to this size download into page-locked host memory
PINNED_PLAN_MAX = 1 << 30  # page-locked read-back memory one plan keeps at most; larger reads go pageable


class _Plan:
    """Buffers, views and launches of one (batch, keep) configuration."""

    def __init__(self):
        self.bufs: list[Buf] = []
        self.views: dict = {}
        self.steps: list = []          # (label, fn, args)
        self.works: list = []          # per step: (kind, algorithmic int ops, algorithmic HBM bytes)
        self.fused_adds: set = set()   # add_requant ops computed in a GEMM epilogue
        self.norm_of: dict = {}        # fused add_requant -> the rmsnorm_int of its sum that may share its epilogue
        self.fused_norms: set = set()  # rmsnorm_int ops computed in a GEMM epilogue
        self.stage: dict = {}          # device staging buffers of float inputs and token ids
        self.host_stage: dict = {}     # page-locked host buffers the read-back downloads into, by device buffer
        self.graph = None              # the steps captured as one HIP graph (run(..., graph=True))
        self.eager_ms: list = []       # device ms of the plan's first eager runs (run's default launch choice)
        self.graph_ms = None           # device ms of its first replay of the captured graph
        self.replay = None             # run's choice once measured: True = replay the graph, False = launch eagerly
        self.kb_values: set = set()    # values stored K-blocked (read only by GEMMs)

    def buf(self, nbytes, name=""):
        b = Buf(nbytes, name)
        self.bufs.append(b)
        return b

    def dense(self, dims, dtype, name=""):
        dims = tuple(int(d) for d in dims)
        b = self.buf(math.prod(dims) * rt.ITEMSIZE[dtype], name)
        return View(b, dtype, dims, contig_strides(dims))

    def kblocked(self, dims, dtype, name=""):
        """Storage for a value read only as a GEMM operand: the last dim in 64-element blocks, each block holding
        all rows consecutively (block stride rows * 64)."""
        dims = tuple(int(d) for d in dims)
        b = self.buf(math.prod(dims) * rt.ITEMSIZE[dtype], name)
        lead = contig_strides(dims[:-1])
        return View(b, dtype, dims, tuple(64 * x for x in lead) + (1,), kb=64 * math.prod(dims[:-1]))


class CompiledModel:
    """A graph compiled for the mi355x backend: consts resident on the device, plans per batch size."""

    def __init__(self, module, consts, *, device: int = 0, proven: bool = False):
        self.module, self.consts = module, dict(consts)
        # proven: the sound int32 analysis (|multipliers|) holds, so kernels may skip their int32 checks. A graph
        # that passes only the reference's looser check (a negative multiplier) runs on the checked kernels.
        bounds = Q.int32_bounds(module, self.consts) if proven else None
        self.proven = bool(proven) and bounds.ok
        self.func = g.func_of(module)
        self.ops = [op for op in self.func.ops if not isinstance(op, g.OutputOp)]
        outs = [op for op in self.func.ops if isinstance(op, g.OutputOp)]
        if len(outs) != 1:
            raise ValueError("the graph needs exactly one output op")
        self.output_values = outs[0].values
        if not any(not isinstance(op, (g.InputOp, g.ConstOp)) for op in self.ops):
            raise ValueError("the graph has no operations to compile (its outputs are its inputs)")
        self.meta = _graph_meta(module)
        self.in_dtypes = {op.sym_str: g.qt(op.result).dtype for op in self.ops if isinstance(op, g.InputOp)}
        self.input_ops = [op for op in self.ops if isinstance(op, g.InputOp)]
        self.users = {}
        for op in self.func.ops:
            for v in op.operands:
                self.users.setdefault(v, []).append(op)
        self.is_const = set()
        for op in self.ops:
            if isinstance(op, g.ConstOp) or (isinstance(op, (g.TransposeOp, g.ReshapeOp)) and op.x in self.is_const):
                self.is_const.add(op.result)
        self.phys = self._choose_layouts()
        self.acc_bounds = bounds.acc if self.proven else {}    # matmul result -> proven bound on |accumulator|
        self.device_index = device
        self.dev = None
        self.embedding = None             # (wte, wpe) float32 host tables of a token model
        self._embed_dev = None
        self._const_views = {}
        self._const_bt = {}
        self._const_kb = {}
        self._const_bt_host = {}
        self._plans = {}
        self.group_gemms = True           # independent consecutive GEMMs as one anvil_gemm_i8_group call

    # --------------------------------------------------------------------------------------- layout choice
    def _choose_layouts(self) -> dict:
        """Physical dim order of matmul results read only through one transpose that keeps the last dim last
        (the head merge o (H, T, d) -> (T, H, d) -> reshape (T, C)): storing the result in the transposed order
        makes the transpose and the reshape free views."""
        phys = {}
        for op in self.ops:
            if not isinstance(op, (g.QMatmulOp, g.QLinearOp)):
                continue
            us = self.users.get(op.result, [])
            if len(us) != 1 or not isinstance(us[0], g.TransposeOp):
                continue
            p = us[0].perm_list
            if p[-1] == len(p) - 1 and p != list(range(len(p))):
                phys[op.result] = p
        for op in self.ops:
            if isinstance(op, (g.QMatmulOp, g.QLinearOp)):
                if self._t16_chain(op):           # the T = 16 attention reads V's rows as they are
                    continue
                root = self._transposed_producer(op.b, phys)
                if root is not None:
                    phys[root] = _swap_last2(len(g.qt(root).dims))
        return phys

    def _chain_of(self, o_op):
        """(scores matmul, softmax) when o_op is the P.V product of a chain the fused attention evaluates (the
        structure only: proven, int8 throughout, scores and p read by nothing else, square scores with T a multiple
        of 32 up to 1024 and a head dim of 16, 32, 64 or 128, or T = 16 and a head dim of 16 or 32), else None."""
        if not self.proven or not isinstance(o_op, g.QMatmulOp) or o_op.lut is not None:
            return None
        if g.qt(o_op.result).dtype != "i8":
            return None
        sm = o_op.a.owner
        if not isinstance(sm, g.SoftmaxLutOp) or g.qt(sm.result).dtype != "i8" or not 1 <= int(sm.one) <= 127:
            return None
        s_op = sm.x.owner
        if (not isinstance(s_op, g.QMatmulOp) or s_op.lut is not None or g.qt(s_op.result).dtype != "i8"
                or not self._softmax_lut_ok(sm)):
            return None
        if any(v in self.is_const or self.users.get(v, []) != [u] for v, u in ((s_op.result, sm), (sm.result, o_op))):
            return None
        sd, od = g.qt(s_op.result).dims, g.qt(o_op.result).dims
        T, D = sd[-1], g.qt(s_op.a).dims[-1]
        if (sd[-2] != T or (T % 32 and T != 16) or T > 1024 or D not in (16, 32, 64, 128) or (T == 16 and D > 32)
                or od[-1] != D or od[-2] != T):
            return None
        return s_op, sm

    def _t16_chain(self, o_op) -> bool:
        chain = self._chain_of(o_op)
        return chain is not None and g.qt(chain[0].result).dims[-1] == 16

    def _const_array(self, v):
        """The int64 values of a graph const, None for a computed value."""
        op = v.owner
        if not isinstance(op, g.ConstOp):
            return None
        src = op.value if op.value is not None else self.consts[op.sym_str]
        return np.asarray(src, dtype=np.int64).reshape(-1)

    def _transposed_producer(self, b, phys):
        """The matmul result whose transposed storage (last two dims swapped) makes the right operand `b` -- a
        view chain of transposes / reshapes over that result -- K-contiguous, so no transpose copy is needed
        (attention's v -> vh read as P.V's right operand). None when b is already K-contiguous, is a const, or
        the chain does not end at a single-use matmul result."""
        chain, v = [], b
        while isinstance(v.owner, (g.TransposeOp, g.ReshapeOp)) and v not in self.is_const:
            if len(self.users.get(v, [])) != 1:
                return None
            chain.append(v.owner)
            v = v.owner.x
        root = v
        if (not isinstance(root.owner, (g.QMatmulOp, g.QLinearOp)) or root in self.is_const or root in phys
                or len(self.users.get(root, [])) != 1 or not chain):
            return None

        def view_of(perm):
            dims = [2] + g.qt(root).dims
            pf = [0] + [p + 1 for p in perm]
            st = contig_strides([dims[i] for i in pf])
            vw = View(None, "i8", tuple([dims[i] for i in pf]), st).permute([pf.index(i) for i in range(len(pf))])
            for o in reversed(chain):
                if isinstance(o, g.TransposeOp):
                    vw = vw.permute([0] + [p + 1 for p in o.perm_list])
                else:
                    vw = vw.reshape((2, *g.qt(o.result).dims))
                    if vw is None:
                        return None
            return vw

        n = len(g.qt(root).dims)
        plain, swapped = view_of(list(range(n))), view_of(_swap_last2(n))
        k_contig = lambda vw: vw is not None and (vw.strides[-2] == 1 or vw.dims[-2] == 1)   # noqa: E731
        return root if not k_contig(plain) and k_contig(swapped) else None

    # ----------------------------------------------------------------------------------------- device state
    def _ensure_device(self):
        if self.dev is not None:
            return
        self.dev = rt.device(self.device_index)
        for op in self.ops:
            if not isinstance(op, g.ConstOp):
                continue
            t = g.qt(op.result)
            vals = np.asarray(op.value if op.value is not None else self.consts[op.sym_str], dtype=np.int64)
            vals = vals.reshape(t.dims)
            mem = self.dev.upload(vals.astype(rt.NP_DTYPE[t.dtype]))
            b = Buf(mem.nbytes, op.sym_str or "const")
            b.mem = mem
            self._const_views[op.result] = View(b, t.dtype, tuple(t.dims), contig_strides(t.dims))

    def changed_consts(self) -> list:
        bad = []
        for op in self.ops:
            if isinstance(op, g.ConstOp) and op.result in self._const_views:
                v = self._const_views[op.result]
                want = np.asarray(op.value if op.value is not None else self.consts[op.sym_str], dtype=np.int64)
                got = v.buf.mem.download(v.dims, rt.NP_DTYPE[v.dtype]).astype(np.int64)
                if not np.array_equal(got, want.reshape(v.dims)):
                    bad.append(op.sym_str)
        return bad

    # ------------------------------------------------------------------------------------------- planning
    def _plan(self, nb: int, keep: str) -> _Plan:
        P = _Plan()
        dev = self.dev
        views = P.views

        def step(label, fn, *args):
            P.steps.append((label, fn, args))
            P.works.append(_work(fn, args))

        def lead(v):
            return () if v in self.is_const else (nb,)

        def dense_copy(src: View, label):
            return _dense_copy_into(P, step, dev, src, label)

        def dense(v: View, label) -> View:
            return v if v.is_contiguous() else dense_copy(v, label)

        fused = self._attention_chains(keep)
        skip = {o for s_op, sm in fused.values() for o in (s_op, sm)}
        adds = self._residual_fusions(keep)
        P.norm_of = self._norm_fusions(adds)
        P.kb_values = self._kblocked_values(keep, fused, skip, adds)
        for op in self.ops:
            if op in skip or op in P.fused_adds or op in P.fused_norms:
                continue
            r = op.results[0]
            t = g.qt(r)
            label = op.sym_str or op.name.split(".")[-1]
            if isinstance(op, g.InputOp):
                views[r] = P.dense((nb, *t.dims), t.dtype, label)
                continue
            if isinstance(op, g.ConstOp):
                views[r] = self._const_views[r]
                continue
            if isinstance(op, g.TransposeOp):
                src = views[op.x]
                k = 0 if op.x in self.is_const else 1
                views[r] = src.permute(list(range(k)) + [p + k for p in op.perm_list])
                continue
            if isinstance(op, g.ReshapeOp):
                src = views[op.x]
                nd = (*lead(op.x), *t.dims)
                v = src.merge_kblocked(nd) if r in P.kb_values else src.reshape(nd)
                if v is None:
                    v = dense_copy(src, label).reshape(nd)
                views[r] = v
                continue
            out_dims = (*lead(r), *t.dims)
            if op in fused:
                views[r] = self._plan_attention(P, op, *fused[op], views, nb, label, dense, step, keep)
                continue
            if isinstance(op, (g.QMatmulOp, g.QLinearOp)):
                views[r] = self._plan_matmul(P, op, views, out_dims, label, dense, step, keep, add=adds.get(op))
                continue
            if isinstance(op, g.SoftmaxLutOp):
                views[r] = self._plan_softmax(P, op, views, out_dims, label, dense, step)
                continue
            out = P.kblocked(out_dims, t.dtype, label) if r in P.kb_values else P.dense(out_dims, t.dtype, label)
            views[r] = out
            if isinstance(op, g.RmsNormIntOp):
                x = dense(views[op.x], label + ".x")
                lut = self._const_views[op.lut] if op.lut in self._const_views else dense(views[op.lut], label)
                w = dense(views[op.w], label + ".w")
                rows = math.prod(x.dims[:-1])
                flags = rt.OP_UNCHECKED if self.proven else 0
                lut_vals = self._const_array(op.lut)
                if flags and lut_vals is not None and int(np.abs(lut_vals).max()) * abs(int(op.M)) < (1 << 23):
                    flags |= rt.RMS_S24                          # x w (lut M) + rnd as one 24-bit multiply-add
                if out.kb:
                    flags |= rt.RMS_OUT_KBLOCK
                step(label, _call_ptrs, dev.rmsnorm_int, [x, g.qt(op.x).dtype, w, lut, lut.size, int(op.M),
                                                          int(op.s), op.ss_shift_int, op.ss_init_int, rows,
                                                          x.dims[-1], out, flags])
            elif isinstance(op, g.AddRequantOp):
                a = dense(views[op.a], label + ".a")
                b = dense(views[op.b], label + ".b")
                if op.a in self.is_const:
                    a = dense_copy(a.prepend(nb), label + ".a")
                if op.b in self.is_const:
                    b = dense_copy(b.prepend(nb), label + ".b")
                step(label, _call_ptrs, dev.add_requant, [a, g.qt(op.a).dtype, b, g.qt(op.b).dtype, int(op.Ma),
                                                          int(op.Mb), int(op.s), out.size, out, t.dtype,
                                                          rt.OP_UNCHECKED if self.proven else 0])
            elif isinstance(op, g.LutOp):
                x = dense(views[op.x], label + ".x")
                if op.x in self.is_const:
                    x = dense_copy(x.prepend(nb), label + ".x")
                step(label, _call_ptrs, dev.lut_i8, [x, dense(views[op.table], label + ".t"), out.size, out])
            elif isinstance(op, g.LutMulOp):
                x = dense(views[op.x], label + ".x")
                y = dense(views[op.y], label + ".y")
                if op.x in self.is_const:
                    x = dense_copy(x.prepend(nb), label + ".x")
                if op.y in self.is_const:
                    y = dense_copy(y.prepend(nb), label + ".y")
                step(label, _call_ptrs, dev.lut_mul, [x, y, dense(views[op.table], label + ".t"), int(op.M),
                                                      int(op.s), out.size, out,
                                                      rt.OP_UNCHECKED if self.proven else 0])
            else:
                raise NotImplementedError(op.name)
        if self.group_gemms:
            _group_gemms(P)
        return P

    def _softmax_lut_ok(self, op) -> bool:
        """The exp LUT is a const with every entry >= 0 and lut[255] >= 1: no row can sum to zero."""
        table = self._const_array(op.lut)
        return table is not None and table.size == 256 and table.min() >= 0 and table[-1] >= 1

    def _plan_softmax(self, P, op, views, out_dims, label, dense, step):
        t = g.qt(op.result)
        out = P.dense(out_dims, t.dtype, label)
        x = dense(views[op.x], label + ".x")
        lut = dense(views[op.lut], label + ".lut")
        t1, t2 = x.dims[-2], x.dims[-1]
        batch = math.prod(x.dims[:-2])
        sure = self.proven and self._softmax_lut_ok(op)
        step(label, _call_ptrs, self.dev.softmax_lut, [x, lut, int(op.one), bool(op.causal), batch, t1, t2, out,
                                                       t.dtype, rt.OP_UNCHECKED if sure else 0])
        return out

    def _attention_chains(self, keep) -> dict:
        """{P.V matmul: (scores matmul, softmax)} for every chain qmatmul -> softmax_lut -> qmatmul whose scores and
        probabilities are read by nothing else, in a proven graph with int8 values throughout, a square (T x T)
        score matrix with T a multiple of 32 up to 1024 and one head dim of 16, 32, 64 or 128, or T = 16 and a head
        dim of 16 or 32: the chains
        anvil_attention_i8 evaluates without materialising scores or p, or, when the run returns them (keep="all",
        or graph outputs), anvil_attention_i8_keep, which also stores them (_kept_chain)."""
        if not self.proven:
            return {}
        found = {}
        for o_op in self.ops:
            chain = self._chain_of(o_op)
            if chain is not None:
                found[o_op] = chain
        return found

    def _kept_chain(self, s_op, sm, keep) -> bool:
        """Whether a fused chain's scores and probabilities are returned, and so stored by the kernel."""
        return keep == "all" or s_op.result in self.output_values or sm.result in self.output_values

    def _plan_attention(self, P, o_op, s_op, sm, views, nb, label, dense, step, keep):
        """One anvil_attention_i8 launch for a fused chain (anvil_attention_i8_keep when the run returns its scores
        and probabilities), or the three ops when the operand views do not fit it."""
        n = len(g.qt(o_op.result).dims) + 1
        kept = self._kept_chain(s_op, sm, keep)
        qa = views[s_op.a]
        kb = views[s_op.b].permute(_swap_last2(n))           # key rows (..., T, d)
        vb = views[o_op.b].permute(_swap_last2(n))           # V^T rows (..., d, T)
        T0 = g.qt(s_op.result).dims[-1]
        vrows = T0 == 16 and vb.strides[-1] != 1 and views[o_op.b].strides[-1] == 1
        if vrows:                                           # the T = 16 kernel takes V's own rows (..., T, d)
            vb = views[o_op.b]
        om = self._merged_heads(o_op)
        if om is not None and om in P.kb_values:
            # o written head-blocked: om's K-blocked storage (block = head), split into heads and permuted back to
            # o's order, is a plain strided view (sequence T * 64, head rows * 64, row 64)
            omd = (nb, *g.qt(om).dims)
            split = P.kblocked(omd, "i8", label).reshape((*omd[:-1], omd[-1] // 64, 64))
            pfull = [0] + [p + 1 for p in self.users[o_op.result][0].perm_list]
            out = split.permute([pfull.index(i) for i in range(len(pfull))])
        else:
            out = self._alloc_result(P, o_op, (nb, *g.qt(o_op.result).dims), label)
        vs = [qa, kb, vb, out]
        if kept:
            sv = self._alloc_result(P, s_op, (nb, *g.qt(s_op.result).dims), label + ".scores")
            pv = P.dense((nb, *g.qt(sm.result).dims), "i8", label + ".p")
            vs += [sv, pv]
        lead = out.dims[:-2]
        idx = [i for i, d in enumerate(lead) if d != 1]
        fits = (all(len(v.dims) == n and v.dims[:-2] == lead and v.strides[-1] == 1 for v in vs)
                and len(idx) <= 2)
        if fits:
            idx = [None] * (2 - len(idx)) + idx
            strides = []
            for v in vs:
                strides += [0 if i is None else v.strides[i] for i in idx] + [v.strides[-2]]
            offs = [v.offset for v in vs]
            T, D = qa.dims[-2], qa.dims[-1]
            # K and V^T go through 32-bit buffer offsets over one head: rows at least D (keys) / T (V^T) apart; O's
            # 32-row tiles through 32-bit offsets too
            vrow_len, vrows_n = (D, T) if vrows else (T, D)   # V rows (T of D keys' values) or V^T rows
            fits = (all(st % 16 == 0 for st in strides[:9]) and all(st % 4 == 0 for st in strides[9:12])
                    and all(o % 16 == 0 for o in offs[:3]) and offs[3] % 4 == 0
                    and strides[5] >= D and strides[8] >= vrow_len and T * strides[5] < 1 << 31
                    and vrows_n * strides[8] < 1 << 31 and strides[11] >= D and 32 * strides[11] < 1 << 31)
            if kept:                     # S and P: 16-byte stores into 32-row tiles through 32-bit offsets
                fits = (fits and all(st % 16 == 0 for st in strides[12:]) and all(o % 16 == 0 for o in offs[4:])
                        and all(T <= st and 32 * st < 1 << 31 for st in (strides[14], strides[17])))
        if not fits:
            sv = self._plan_matmul(P, s_op, views, (nb, *g.qt(s_op.result).dims), label + ".scores", dense, step,
                                   keep)
            views[s_op.result] = sv
            views[sm.result] = self._plan_softmax(P, sm, views, (nb, *g.qt(sm.result).dims), label + ".p", dense,
                                                  step)
            return self._plan_matmul(P, o_op, views, (nb, *g.qt(o_op.result).dims), label, dense, step, keep,
                                     out=out)
        b0, b1 = [1 if i is None else lead[i] for i in idx]
        T, D = qa.dims[-2], qa.dims[-1]
        flags = rt.OP_UNCHECKED | (rt.ATTN_V_ROWS if vrows else 0)
        if self.acc_bounds.get(s_op.result, 1 << 31) < (1 << 23) and abs(int(s_op.M)) < (1 << 23):
            flags |= rt.ATTN_S24
        if kept:
            views[s_op.result], views[sm.result] = sv, pv
            step(label, _call_attention_keep, self.dev, qa, kb, vb, out, sv, pv, b0, b1, T, D, strides, s_op, sm,
                 o_op, views[sm.lut], flags)
        else:
            step(label, _call_attention, self.dev, qa, kb, vb, out, b0, b1, T, D, strides, s_op, sm, o_op,
                 views[sm.lut], flags)
        return out

    def _alloc_result(self, P, op, out_dims, label):
        """Dense storage of a matmul result in its chosen physical order, viewed in the logical order."""
        t = g.qt(op.result)
        perm = self.phys.get(op.result)
        if op.result in P.kb_values:
            return P.kblocked(out_dims, t.dtype, label)
        if perm is None:
            return P.dense(out_dims, t.dtype, label)
        k = 0 if op.result in self.is_const else 1
        pfull = list(range(k)) + [p + k for p in perm]
        st = P.dense([out_dims[i] for i in pfull], t.dtype, label)
        return st.permute([pfull.index(i) for i in range(len(pfull))])

    def _bt_const(self, op):
        """A const right operand (K, N) stored once transposed (N, K) so its K dim is contiguous."""
        key = op.b
        if key not in self._const_bt:
            c = op.b                              # a const, or a transpose / reshape chain of one: replay on host
            chain = []
            while c not in self._const_views:
                chain.append(c.owner)
                c = c.owner.x
            vals = np.asarray(self._host_const(c), dtype=np.int64)
            for o in reversed(chain):
                vals = np.transpose(vals, o.perm_list) if isinstance(o, g.TransposeOp) else vals.reshape(
                    g.qt(o.result).dims)
            bt = np.ascontiguousarray(np.swapaxes(vals, -1, -2)).astype(np.int8)
            mem = self.dev.upload(bt)
            b = Buf(mem.nbytes, f"{op.sym_str}.Bt")
            b.mem = mem
            self._const_bt_host[id(b)] = bt
            self._const_bt[key] = View(b, "i8", bt.shape, contig_strides(bt.shape))
        return self._const_bt[key]

    def _bt_kblocked(self, op):
        """The same transposed const (N, K), K-blocked for the fast GEMM kernels: (ceil(K / 64), N, 64), row n's K block j
        at j N 64 + n 64, as a K-blocked view."""
        key = op.b
        if key not in self._const_kb:
            bt = self._bt_const(op)
            N, K = bt.dims
            host = np.zeros((N, -(-K // 64) * 64), np.int8)
            host[:, :K] = self._bt_host(bt)
            kb = np.ascontiguousarray(host.reshape(N, -1, 64).transpose(1, 0, 2))
            mem = self.dev.upload(kb)
            b = Buf(mem.nbytes, f"{op.sym_str}.Bt.kblocked")
            b.mem = mem
            self._const_kb[key] = View(b, "i8", (N, K), (64, 1), kb=N * 64)
        return self._const_kb[key]

    def _bt_host(self, bt):
        """Host copy of a const operand view made by _bt_const (kept on the host when it was uploaded)."""
        return self._const_bt_host[id(bt.buf)]

    def _kblock_weight(self, op, rows1, rows2, strides, K, swapped):
        """Proven 2-D products whose const right operand is read through _bt_const take its K-blocked copy: the
        operand's loads then fetch whole 64-byte blocks of consecutive rows, where row-major rows give 64-byte pieces
        of separate lines. Only for the fast kernels (proven, K and the other operand's strides multiples of 16);
        returns (rows1, rows2) for the call (_kb_call then sets the strides and flags)."""
        if not self.proven or K % 16 or op.b not in self._const_bt:
            return rows1, rows2
        if (rows1 if swapped else rows2).buf is not self._const_bt[op.b].buf:
            return rows1, rows2
        other = rows2 if swapped else rows1
        if any(v % 16 for v in (strides[3:6] if swapped else strides[0:3])) or (other.offset * other.itemsize) % 16:
            return rows1, rows2
        kv = self._bt_kblocked(op)
        return (kv, rows2) if swapped else (rows1, kv)

    @staticmethod
    def _kb_call(rows1, rows2, c, strides, flags):
        """Strides and flags of a GEMM call for its operands' and result's layouts: a K-blocked view passes its block
        stride in place of its row stride, with the ANVIL_GEMM_*_KBLOCK flag."""
        strides = list(strides)
        if rows1.kb:
            strides[2], flags = rows1.kb, flags | rt.GEMM_A_KBLOCK
        if rows2.kb:
            strides[5], flags = rows2.kb, flags | rt.GEMM_B_KBLOCK
        if c is not None and c.kb:
            strides[8], flags = c.kb, flags | rt.GEMM_C_KBLOCK
        return strides, flags

    def _kblocked_values(self, keep, fused, skip, adds) -> set:
        """Values stored K-blocked in this plan: int8 results of an rmsnorm or of a plain linear product (a 2-D const
        right operand, stored unpermuted, no fused add) that are read only as the left operand of plain linear
        products and are not graph outputs, in a proven graph, with a last dim that is a multiple of 64 (keep="all"
        reads such a value back from its blocks, View.view).
        Their readers then load whole 64-byte blocks of consecutive rows (ANVIL_GEMM_*_KBLOCK). Linear results read
        only by fused attention chains through a split into heads of 64 (q and k) are stored head-blocked too: each
        head's rows are then one contiguous block, read as a plain strided view. So is a fused attention's output
        merged back from its heads of 64 when only linear products read the merged value (om)."""
        if not self.proven:
            return set()
        fused_ops = set(fused) | skip

        def linear(op):
            return (isinstance(op, (g.QMatmulOp, g.QLinearOp)) and op.b in self.is_const
                    and len(g.qt(op.b).dims) == 2 and op not in fused_ops)
        scores_ops = {s_op for s_op, _ in fused.values()}

        def to_attention(v):
            """v reaches only fused attention chains' score products, through transposes."""
            us = self.users.get(v, [])
            return bool(us) and v not in self.output_values and all(
                (isinstance(u, g.TransposeOp) and to_attention(u.result)) or u in scores_ops for u in us)

        def head_split(u, r):
            """u splits r's last dim into heads of 64 (a view of head-blocked storage) and feeds attention only."""
            d = g.qt(u.result).dims
            return (isinstance(u, g.ReshapeOp) and len(d) >= 2 and d[-1] == 64 and d[-2] * 64 == g.qt(r).dims[-1]
                    and to_attention(u.result))
        out = set()
        for op in self.ops:
            r = op.results[0] if op.results else None
            if r is None or r in self.output_values or r in self.is_const or g.qt(r).dtype != "i8":
                continue
            producer = isinstance(op, g.RmsNormIntOp) or (linear(op) and op not in adds and r not in self.phys)
            users = self.users.get(r, [])
            if producer and g.qt(r).dims[-1] % 64 == 0 and users and (
                    all(linear(u) and u.a is r and u.b is not r for u in users)
                    or (linear(op) and all(head_split(u, r) for u in users))):
                out.add(r)
        for o_op in fused:                     # attention outputs merged back from heads of 64 for linear readers
            om = self._merged_heads(o_op)
            users = self.users.get(om, []) if om is not None else []
            if users and g.qt(om).dtype == "i8" and all(linear(u) and u.a is om and u.b is not om for u in users):
                out.add(om)
        return out

    def _merged_heads(self, o_op):
        """om when a fused attention's output o (..., H, T, 64) reaches the graph only as om = reshape(transpose(o))
        of dims (..., T, H * 64), the transpose swapping the head and sequence dims; none of the three returned. o can
        then be written straight into om's K-blocked storage, one block per head."""
        o = o_op.result
        us = self.users.get(o, [])
        d = g.qt(o).dims
        n = len(d)
        if len(us) != 1 or not isinstance(us[0], g.TransposeOp) or o in self.output_values or n < 3 or d[-1] != 64:
            return None
        t = us[0]
        if list(t.perm_list) != list(range(n - 3)) + [n - 2, n - 3, n - 1]:
            return None
        us2 = self.users.get(t.result, [])
        if len(us2) != 1 or not isinstance(us2[0], g.ReshapeOp) or t.result in self.output_values:
            return None
        om = us2[0].result
        rd = g.qt(om).dims
        if om in self.output_values or tuple(rd) != (*d[:-3], d[-2], d[-3] * 64):
            return None
        return om

    def _host_const(self, value):
        op = value.owner
        return op.value if op.value is not None else self.consts[op.sym_str]

    def _residual_fusions(self, keep) -> dict:
        """{matmul: add_requant} for matmul results y that feed an add_requant with a residual computed earlier in the
        graph, in a proven graph, where y, the residual and the sum share one dtype (all int8, or all int16: the wide
        residual stream of docs/decisions/ADR-004-small-inputs.md:59-82): the add runs in the GEMM's epilogue (y itself
        is still written when it is returned or read elsewhere)."""
        if not self.proven:
            return {}
        order = {op: i for i, op in enumerate(self.ops)}
        found, taken = {}, set()
        for op in self.ops:
            dt = g.qt(op.result).dtype if isinstance(op, (g.QMatmulOp, g.QLinearOp)) else None
            if dt not in ("i8", "i16") or op.result in self.phys:
                continue
            for u in self.users.get(op.result, []):
                if (not isinstance(u, g.AddRequantOp) or u in taken or g.qt(u.result).dtype != dt
                        or g.qt(u.a).dtype != dt or g.qt(u.b).dtype != dt or u.a is u.b):
                    continue
                other = u.b if u.a is op.result else u.a
                own = other.owner
                if other in self.is_const or order.get(own, len(order)) > order[op]:
                    continue
                if g.qt(other).dims != g.qt(op.result).dims:
                    continue
                found[op] = u
                taken.add(u)
                break
        return found

    def _norm_fusions(self, adds) -> dict:
        """{add_requant: rmsnorm_int} for fused adds (_residual_fusions) whose int8 sum feeds a plain int8 rmsnorm
        (ss_shift = ss_init = 0, const weights and a const non-negative table with |table x M| < 2^23) over rows
        of 128, with add multipliers below 2^24: the rmsnorm can then run in the same epilogue
        (anvil_gemm_i8_add_norm), which _plan_fused_add takes when the rows allow it. At C = 128 (config 4) these are
        each block's h2 = rmsnorm(r1), the next layer's h1 and the final norm: 0.1042 -> 0.0972 ms a step. The entry
        point also takes rows of 256 (64 x 256 tiles), but at config 3 that measured level with the two launches
        (0.0736 against 0.0737 ms), so the planner leaves those unfused."""
        found = {}
        for add in adds.values():
            t = g.qt(add.result)
            if t.dtype != "i8" or t.dims[-1] != 128 or max(abs(int(add.Ma)), abs(int(add.Mb))) >= 1 << 24:
                continue
            for u in self.users.get(add.result, []):
                if (not isinstance(u, g.RmsNormIntOp) or u.x is not add.result or u.ss_shift_int
                        or u.ss_init_int or g.qt(u.w).dtype != "i8"):
                    continue
                w, lut = self._const_array(u.w), self._const_array(u.lut)
                if w is None or lut is None or lut.size < 1 or int(lut.min()) < 0:
                    continue
                if int(np.abs(lut).max()) * abs(int(u.M)) >= 1 << 23 or not 0 <= int(u.s) <= 31:
                    continue
                found[add] = u
                break
        return found

    def _plan_matmul(self, P, op, views, out_dims, label, dense, step, keep, out=None, add=None):
        t = g.qt(op.result)
        M, N = out_dims[-2], out_dims[-1]
        K = g.qt(op.a).dims[-1]
        # result storage: dense in the chosen physical order, logical view by permuting back
        perm = self.phys.get(op.result)
        if out is None:
            out = self._alloc_result(P, op, out_dims, label)
        swapped = perm is not None and perm == _swap_last2(len(perm))
        # A rows: (lead..., M, K) with K contiguous
        a = views[op.a]
        if a.strides[-1] != 1 and a.dims[-1] != 1:
            a = dense(a, label + ".a")
        # Bt rows: (lead..., N, K) with K contiguous
        if op.b in self.is_const and len(g.qt(op.b).dims) == 2:
            bt = self._bt_const(op)
        else:
            bv = views[op.b]
            bt = bv.permute(_swap_last2(len(bv.dims)))
            if bt.strides[-1] != 1 and bt.dims[-1] != 1:
                bt = _dense_copy_into(P, step, self.dev, bt, label + ".bt")
        lut = None if op.lut is None else views[op.lut]
        flags = rt.GEMM_UNCHECKED if self.proven else 0
        if self.proven and self.acc_bounds.get(op.result, 1 << 31) < (1 << 23) and abs(int(op.M)) < (1 << 23):
            flags |= rt.GEMM_MUL24
        if swapped:
            # the result is stored transposed: compute C^T = Bt . A^T, whose rows are N
            rows1, rows2, c, Mx, Nx = bt, a, out.permute(_swap_last2(len(out.dims))), N, M
        else:
            rows1, rows2, c, Mx, Nx = a, bt, out, M, N
            if self._causal_skip_ok(op, keep):
                flags |= rt.GEMM_CAUSAL_SKIP
            elif self._causal_k_ok(op):
                flags |= rt.GEMM_CAUSAL_K
        # lead dims: broadcast an operand over lead dims it lacks (stride 0)
        lc = list(zip(c.dims[:-2], c.strides[:-2]))
        l1 = list(zip(rows1.dims[:-2], rows1.strides[:-2]))
        l2 = list(zip(rows2.dims[:-2], rows2.strides[:-2]))
        l1 = [(d, 0) for d, _ in lc[:len(lc) - len(l1)]] + l1
        l2 = [(d, 0) for d, _ in lc[:len(lc) - len(l2)]] + l2
        # fold every lead dim into the row dim when rows1 and C allow it and rows2 does not vary over them
        if all(s == 0 for _, s in l2) and not (flags & (rt.GEMM_CAUSAL_SKIP | rt.GEMM_CAUSAL_K)):
            r1 = rows1.reshape((math.prod(rows1.dims[:-1]), K)) if len(rows1.dims) == len(c.dims) else None
            c2 = c.reshape((math.prod(c.dims[:-1]), Nx))
            if r1 is not None and c2 is not None and (r1.strides[-1] == 1 or K == 1):
                strides = [0, 0, r1.strides[0], 0, 0, rows2.strides[-2], 0, 0, c2.strides[0]]
                if add is not None and self._plan_fused_add(P, op, add, views, r1, rows2, c2, strides, lut, flags,
                                                            label, step, keep):
                    return out
                r1, rows2 = self._kblock_weight(op, r1, rows2, strides, K, swapped)
                strides, flags = self._kb_call(r1, rows2, c2, strides, flags)
                step(label, _call_gemm, self.dev, r1, rows2, c2, 1, 1, r1.dims[0], Nx, K, strides, op, lut, t.dtype,
                     flags)
                return out
        # merge adjacent lead dims that nest in all three alike, down to at most two batch dims
        lead = [(d, s1, s2, sc) for (d, s1), (_, s2), (_, sc) in zip(l1, l2, lc) if d != 1]
        merged = []
        for d, s1, s2, sc in lead:
            if merged:
                D, S1, S2, SC = merged[-1]
                if S1 == s1 * d and S2 == s2 * d and SC == sc * d:
                    merged[-1] = (D * d, s1, s2, sc)
                    continue
            merged.append((d, s1, s2, sc))
        if len(merged) > 2:
            raise NotImplementedError(f"{op.name} {op.sym_str!r}: {len(merged)} batch dims that do not merge")
        while len(merged) < 2:
            merged.insert(0, (1, 0, 0, 0))
        (b0, sa0, sb0, sc0), (b1, sa1, sb1, sc1) = merged
        strides = [sa0, sa1, rows1.strides[-2], sb0, sb1, rows2.strides[-2], sc0, sc1, c.strides[-2]]
        rows1, rows2 = self._kblock_weight(op, rows1, rows2, strides, K, swapped)
        strides, flags = self._kb_call(rows1, rows2, c, strides, flags)
        step(label, _call_gemm, self.dev, rows1, rows2, c, b0, b1, Mx, Nx, K, strides, op, lut, t.dtype, flags)
        return out

    def _plan_fused_add(self, P, op, add, views, a2, bt, c2, strides, lut, flags, label, step, keep) -> bool:
        """Plan y = op(...) with add_requant(y, R) in its epilogue over the 2-D (rows, N) views; False when the views
        do not allow it (the add is then planned as its own launch)."""
        rows, N = c2.dims
        K = a2.dims[-1]
        y_first = add.a is op.result
        other = add.b if y_first else add.a
        rv = views[other].reshape((rows, N))
        ok16 = lambda v: v % 16 == 0                                         # noqa: E731
        if (rv is None or rv.strides[-1] != 1 or K % 16 or not ok16(a2.strides[0]) or not ok16(bt.strides[-2])
                or not ok16(a2.offset) or not ok16(bt.offset) or 256 * max(a2.strides[0], bt.strides[-2]) >= 1 << 31):
            return False
        dt = g.qt(op.result).dtype
        d = P.dense((rows, N), dt, (add.sym_str or "add"))
        store_y = keep == "all" or op.result in self.output_values or len(self.users.get(op.result, [])) > 1
        ma, mb = (int(add.Mb), int(add.Ma)) if y_first else (int(add.Ma), int(add.Mb))   # (residual, y)
        rstrides = [0, 0, rv.strides[0], 0, 0, d.strides[0]]
        a2, bt = self._kblock_weight(op, a2, bt, strides, K, False)
        strides, flags = self._kb_call(a2, bt, c2 if store_y else None, strides, flags)
        norm = P.norm_of.get(add)
        if norm is not None and dt == "i8" and rows % 128 == 0 and N == 128 and ok16(rv.offset):
            # the sum's rmsnorm in the same epilogue: each 128 x N tile spans its rows
            hdims = tuple(views[other].dims)
            h = (P.kblocked(hdims, "i8", norm.sym_str or "norm") if norm.result in P.kb_values
                 else P.dense(hdims, "i8", norm.sym_str or "norm"))
            nw = self._const_views[norm.w]
            nlut = self._const_views[norm.lut]
            step(f"{label}+{norm.sym_str or 'norm'}", _call_gemm_add_norm, self.dev, a2, bt, c2 if store_y else None,
                 rows, N, K, strides, op, lut, rv, ma, mb, int(add.s), d, rstrides, nw, nlut, norm, h,
                 flags | rt.GEMM_NORM_S24)
            views[norm.result] = h
            P.fused_norms.add(norm)
        else:
            step(label, _call_gemm_add, self.dev, a2, bt, c2 if store_y else None, rows, N, K, strides, op, lut, rv,
                 ma, mb, int(add.s), d, rstrides, flags, dt)
        views[add.result] = d.reshape(tuple(views[other].dims))
        P.fused_adds.add(add)
        return True

    def _causal_skip_ok(self, op, keep) -> bool:
        """Scores read only by causal softmaxes, and not returned: tiles above the diagonal are never read."""
        r = op.result
        us = self.users.get(r, [])
        return (keep == "outputs" and r not in self.output_values and bool(us) and r not in self.is_const
                and all(isinstance(u, g.SoftmaxLutOp) and bool(u.causal) for u in us))

    def _causal_k_ok(self, op) -> bool:
        """A is a causal softmax output read as is: A[m][k] = 0 for k > m."""
        own = op.a.owner
        return isinstance(own, g.SoftmaxLutOp) and bool(own.causal) and op.a not in self.is_const

    def plan(self, nb: int, keep: str = "outputs") -> _Plan:
        """The cached plan for batch size nb and read-back policy keep."""
        self._ensure_device()
        key = (nb, keep)
        if key not in self._plans:
            P = self._plan(nb, keep)
            total = 0
            for b in P.bufs:
                if b.mem is None:
                    b.mem = self.dev.alloc(b.nbytes)
                    total += b.nbytes
            P.footprint = total
            self._plans[key] = P
        return self._plans[key]

    # ------------------------------------------------------------------------------------ (de)quantization
    @property
    def inputs(self) -> list:
        return [op.sym_str for op in self.input_ops]

    @property
    def outputs(self) -> list:
        return [v.owner.sym_str for v in self.output_values]

    def scale(self, sym):
        return self.meta[sym][0]

    def quantize_input(self, x, sym=None):
        """Float -> integers at the input's scale, round half to even, saturating (reference driver.py:233-241)."""
        sym = sym or self.inputs[0]
        s = self.scale(sym)
        if s is None:
            raise ValueError(f"input {sym!r} has no scale: pass integer inputs with quantized=True")
        lo, hi = {"i8": (-128, 127), "i16": (-(1 << 15), (1 << 15) - 1)}.get(self.meta[sym][2],
                                                                             (-(1 << 31), (1 << 31) - 1))
        return np.clip(np.rint(np.asarray(x, dtype=np.float64) / s), lo, hi).astype(np.int64)

    def dequantize(self, sym, ints):
        s = self.scale(sym)
        return hostpar.scaled_f64(ints, 1.0 if s is None else s)

    def set_embedding(self, wte, wpe):
        """Token and position tables of a token model (float32 (vocab, C), (>= T, C)); the graph's single input is
        x = wte[ids] + wpe[positions]."""
        if len(self.inputs) != 1:
            raise ValueError("a token embedding needs a graph with exactly one input")
        wte, wpe = np.asarray(wte, dtype=np.float32), np.asarray(wpe, dtype=np.float32)
        dims = self.meta[self.inputs[0]][1]
        if len(dims) != 2 or wte.ndim != 2 or wpe.ndim != 2 or wte.shape[1] != dims[1] or wpe.shape[1] != dims[1] \
                or wpe.shape[0] < dims[0]:
            raise ValueError(f"embedding tables {wte.shape}, {wpe.shape} do not fit the input {tuple(dims)}")
        self.embedding = (np.ascontiguousarray(wte), np.ascontiguousarray(wpe))
        self._embed_dev = None

    def _bind_tokens(self, ids, batch):
        """Token ids for the embedding prelude: (T,) or, with batch=True, (batch, T) integers."""
        if self.embedding is None:
            raise ValueError("tokens=True needs embedding tables: compile(..., embedding=(wte, wpe))")
        ids = np.asarray(ids)
        T = self.meta[self.inputs[0]][1][0]
        if ids.dtype.kind not in "iu":
            raise ValueError(f"token ids must be integers, got dtype {ids.dtype}")
        want = 2 if batch else 1
        if ids.ndim != want or ids.shape[-1] != T:
            raise ValueError(f"token ids of shape {ids.shape}: expected {'(batch, ' if batch else '('}{T})")
        ids = ids.astype(np.int64).reshape(-1, T)
        return ids, ids.shape[0]

    def _bind_inputs(self, x, quantized, batch):
        """Reference driver.py:248-280, plus batch=True: every input has one extra leading batch dim."""
        xs = list(x) if isinstance(x, (list, tuple)) else [x]
        if len(xs) != len(self.inputs):
            raise ValueError(f"{len(xs)} inputs for graph inputs {self.inputs}")
        out, nb = {}, None
        for sym, v in zip(self.inputs, xs):
            v = np.asarray(v)
            shape = tuple(self.meta[sym][1])
            if batch:
                if v.ndim != len(shape) + 1 or tuple(v.shape[1:]) != shape:
                    raise ValueError(f"input {sym!r}: batched shape {v.shape} != (batch, *{shape})")
                if nb is not None and v.shape[0] != nb:
                    raise ValueError(f"inputs disagree on the batch size ({nb} vs {v.shape[0]})")
                nb = v.shape[0]
            elif v.shape != shape:
                squeeze = lambda sh: tuple(d for d in sh if d != 1)   # noqa: E731
                if v.size != math.prod(shape) or (v.ndim > 1 and squeeze(v.shape) != squeeze(shape)):
                    raise ValueError(f"input {sym!r}: shape {v.shape} != {shape}")
                v = v.reshape(shape)
            if quantized:
                out[sym] = self._check_int_input(sym, v)
            else:
                if self.scale(sym) is None:
                    raise ValueError(f"input {sym!r} has no scale: pass integer inputs with quantized=True")
                # quantized on the device (clamp(rint(x / scale)) in float64, as quantize_input does on the host);
                # the kernel also flags NaN and infinite values, which upload_inputs turns into the reference's
                # ValueError (anvil/driver.py:265-266) before the forward is launched
                out[sym] = _FloatInput(np.ascontiguousarray(v, dtype=np.float32 if v.dtype == np.float32
                                                            else np.float64))
            if not batch:
                out[sym] = out[sym][None]
        return out, (nb if batch else 1)

    def _check_int_input(self, sym, v):
        if v.dtype.kind not in "iub":
            raise ValueError(f"input {sym!r}: quantized=True needs integer values, got dtype {v.dtype}")
        dt = self.in_dtypes.get(sym, "i8")
        bits = {"i8": 8, "i16": 16, "i32": 32}.get(dt, 32)
        lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
        v = np.asarray(v, dtype=np.int64)
        if v.size and (v.min() < lo or v.max() > hi):
            raise ValueError(f"input {sym!r}: values in [{v.min()}, {v.max()}] outside {dt} [{lo}, {hi}]")
        return v

    # ----------------------------------------------------------------------------------------------- runs
    def readable(self, keep="outputs") -> list:
        """Syms a run with this keep policy returns: graph outputs and inputs, or every non-const sym."""
        if keep == "outputs":
            syms = self.inputs + self.outputs
        elif keep == "all":
            syms = [op.sym_str for op in self.ops if op.result not in self.is_const]
        else:
            raise ValueError(f"keep must be 'outputs' or 'all', not {keep!r}")
        return [s for s in dict.fromkeys(syms) if s is not None]

    def upload_inputs(self, plan, ints: dict):
        """Integer inputs, or float inputs (quantized on the device), into the plan's input buffers."""
        for op in self.input_ops:
            v = plan.views[op.result]
            x = ints[op.sym_str]
            if isinstance(x, _FloatInput):
                f = x.a
                stage = self._stage(plan, op.sym_str + ".float", f.nbytes)
                stage.upload(f)
                self.dev.quantize(stage, f.dtype == np.float64, self.scale(op.sym_str), f.size, v.ptr, v.dtype)
                try:
                    self.dev.sync()
                except ValueError as e:
                    if "NaN or infinite" in str(e):
                        raise ValueError(f"input {op.sym_str!r} has NaN or infinite values") from None
                    raise
            else:
                v.buf.mem.upload(np.ascontiguousarray(x).astype(rt.NP_DTYPE[v.dtype]))

    def upload_tokens(self, plan, ids):
        """Token ids through the embedding prelude into the input buffer: gather, add and quantize on the device."""
        if self._embed_dev is None:
            wte, wpe = self.embedding
            self._embed_dev = (self.dev.upload(wte), self.dev.upload(wpe), wte.shape[0])
        wte_d, wpe_d, vocab = self._embed_dev
        sym = self.inputs[0]
        v = plan.views[self.input_ops[0].result]
        T, Cdim = self.meta[sym][1]
        stage = self._stage(plan, sym + ".ids", ids.nbytes)
        stage.upload(np.ascontiguousarray(ids, dtype=np.int64))
        self.dev.embed_quantize(stage, ids.size, T, Cdim, wte_d, vocab, wpe_d, self.scale(sym), v.ptr, v.dtype)

    def _stage(self, plan, key, nbytes):
        """A device staging buffer of the plan, kept for later runs of the same size."""
        b = plan.stage.get(key)
        if b is None or b.nbytes < nbytes:
            b = self.dev.alloc(max(nbytes, 16))
            plan.stage[key] = b
        return b

    def launch(self, plan, profile=False, graph=False):
        """Enqueue every kernel of the plan on the device stream (asynchronous unless profile). graph=True replays
        the steps as one HIP graph, captured on the plan's first such launch right after an ordinary launch of the
        same steps (which allocates every workspace they need, so the capture records kernels only)."""
        times = {}
        if not profile and graph:
            if plan.graph is None:
                _launch_steps(plan)
                plan.graph = self.dev.capture(_launch_steps, plan)
            plan.graph.launch()
            return times
        if not profile:
            _launch_steps(plan)
            return times
        # each step's kernels carry their own pair of events (anvil_time_kernels): device time of the kernels alone
        for label, fn, args in plan.steps:
            self.dev.timed(4, 5, fn, *args)
            times[label] = times.get(label, 0.0) + 1e3 * self.dev.elapsed_ms(4, 5)
        return times

    def read(self, plan, syms, nb=None, batch=True, narrow=None) -> dict:
        """sym -> int64 array of each of syms, read back from the device. A device buffer of up to PINNED_MAX bytes
        is downloaded into a page-locked buffer of the plan (DMA straight into it, no pageable staging) and widened
        from there, while the plan's page-locked buffers stay within PINNED_PLAN_MAX bytes in total; beyond that a
        read downloads into ordinary (pageable) memory. With a dict `narrow`, also sym -> the same values as a view at their stored dtype (no copy, into
        that buffer: use it before the plan's next read). Reads of one plan from several threads need the device
        lock around them, as run() holds it."""
        by_sym = {op.sym_str: op.result for op in self.ops if op.sym_str is not None}
        cache, out = {}, {}
        for s in syms:
            v = plan.views[by_sym[s]]
            key = id(v.buf)
            if key not in cache:
                into = None
                if v.buf.nbytes <= PINNED_MAX:
                    into = plan.host_stage.get(key)
                    if into is None or into.nbytes < v.buf.nbytes:
                        held = sum(h.nbytes for k, h in plan.host_stage.items() if k != key)
                        if held + v.buf.nbytes <= PINNED_PLAN_MAX:
                            into = plan.host_stage[key] = self.dev.host_alloc(v.buf.nbytes)
                        else:
                            into = None
                cache[key] = v.buf.mem.download((v.buf.nbytes // v.itemsize,), rt.NP_DTYPE[v.dtype], into=into)
            whole = batch or by_sym[s] in self.is_const
            a = v.read(cache[key])
            out[s] = a if whole else a[0]
            if narrow is not None:
                n = v.view(cache[key])
                narrow[s] = n if whole else n[0]
        return out

    AUTO_EAGER_RUNS = 2                # eager runs a plan times before its graph is captured and timed

    def _auto_graph(self, plan) -> bool:
        """run's default launch: a plan's first AUTO_EAGER_RUNS runs launch eagerly, the next captures the steps
        as a HIP graph (after running them once more), the one after replays it; from then on the faster of the
        two, compared on the device time of the forward (launch gaps included)."""
        if plan.replay is not None:
            return plan.replay
        return len(plan.eager_ms) >= self.AUTO_EAGER_RUNS

    def _note_auto(self, plan, graph, captured, ms):
        """Record one auto run's device time; captured: this run captured the graph (it also ran the steps eagerly
        first, so its time is no replay time)."""
        if plan.replay is not None or captured:
            return
        if not graph:
            plan.eager_ms.append(ms)
        else:
            plan.graph_ms = ms
            plan.replay = ms < min(plan.eager_ms)

    def run(self, x, backend: str = "mi355x", *, quantized=False, keep="outputs", batch=False, profile=False,
            tokens=False, graph=None, **run_kw) -> RunOutput:
        """Quantize x (unless quantized=True), run the graph on the GPU, read back (reference driver.py:305-322).
        Float inputs are quantized on the device. tokens=True: x holds token ids of a model compiled with embedding
        tables, gathered and quantized on the device. graph=True runs the forward as one HIP graph of the plan
        (captured on first use): the same kernels with no launch gaps between them; graph=False launches every kernel
        from the host; graph=None (the default) measures both on the plan's first runs and keeps the faster
        (small batches gain most: their kernels are short and the launch gaps between them a large share)."""
        if backend not in BACKENDS:
            raise ValueError(f"unknown backend {backend!r}: {', '.join(BACKENDS)}")
        if run_kw:
            raise TypeError(f"run() got unexpected keyword argument(s) {sorted(run_kw)}")
        syms = self.readable(keep)
        if tokens:
            ids, nb = self._bind_tokens(x, batch)
        else:
            ints_in, nb = self._bind_inputs(x, quantized, batch)
        plan = self.plan(nb, keep)
        with self.dev.lock:
            if tokens:
                self.upload_tokens(plan, ids)
            else:
                self.upload_inputs(plan, ints_in)
            auto = graph is None and not profile
            if auto:
                graph = self._auto_graph(plan)
            captured = bool(graph) and plan.graph is None
            self.dev.record(2)
            times = self.launch(plan, profile, graph)
            self.dev.record(3)
            self.dev.sync()
            total_ms = self.dev.elapsed_ms(2, 3)
            if auto:
                self._note_auto(plan, graph, captured, total_ms)
            narrow = {}
            ints = self.read(plan, syms, nb, batch, narrow)
            # from the stored dtype (1-2 bytes an element), before another run reuses the plan's host buffers
            outs = [self.dequantize(s, narrow[s]) for s in self.outputs]
        cycles = {label: (times.get(label) if profile else None) for label, _, _ in plan.steps}
        consts = frozenset(op.sym_str for op in self.ops if isinstance(op, g.ConstOp))
        result = {"device_ms": total_ms, "batch": nb, "kernels": len(plan.steps), "footprint": plan.footprint,
                  "hip_graph": bool(graph) and not profile}
        return RunOutput(outs[0], outs, ints, cycles, result, None, consts, self)

    def summary(self) -> str:
        plan = self.plan(1)
        return "\n".join(f"{label:>16} {getattr(fn, '__name__', str(fn))}" for label, fn, _ in plan.steps)


# ------------------------------------------------------------------------------------------ launch helpers

def _launch_steps(plan):
    for _, fn, args in plan.steps:
        fn(*args)


class _FloatInput:
    """A float input array (float32 or float64, batch dim included) to be quantized on the device."""

    def __init__(self, a):
        self.a = a

    def __getitem__(self, idx):
        return _FloatInput(self.a[idx])


def _p(v):
    return v.ptr if isinstance(v, View) else v


def _call_ptrs(fn, args):
    fn(*[_p(a) for a in args])


def _copy_view(dev, src: View, dst: View):
    dev.copy_strided(src.ptr, dst.ptr, src.itemsize, src.dims, src.strides)


def _dense_copy_into(P, step, dev, src: View, label):
    if src.kb:
        raise RuntimeError(f"{label}: a K-blocked value has no strided copy (it is planned for GEMM readers only)")
    dst = P.dense(src.dims, src.dtype, label + ".dense")
    step(label + ".copy", _copy_view, dev, src, dst)
    return dst


def _work(fn, args):
    """(kind, algorithmic int ops, algorithmic HBM bytes) of one launch: every graph operand and result counted
    once at its dtype (LUTs and weights included), layout views free."""
    isz = rt.ITEMSIZE
    if fn is _call_gemm:
        _, a, bt, c, b0, b1, M, N, K, strides, _, _, dt, _ = args
        nb = b0 * b1
        b_batches = nb if (strides[3] or strides[4]) else 1
        return "gemm", 2 * nb * M * N * K, nb * M * K + b_batches * N * K + nb * M * N * isz[dt]
    if fn is _call_gemm_add:
        _, a, bt, c, M, N, K = args[:7]
        osz = isz[args[-1]] if len(args) > 17 else 1
        return "gemm", 2 * M * N * K, M * K + N * K + M * N * osz * (3 if c is not None else 2)
    if fn is _call_gemm_add_norm:                 # also reads the norm's weights and table and writes H
        _, a, bt, c, M, N, K = args[:7]
        nw, nlut = args[16], args[17]
        return "gemm", 2 * M * N * K, M * K + N * K + M * N * (4 if c is not None else 3) + N + 4 * nlut.size
    if fn is _call_attention:
        _, q, k, v, o, b0, b1, T, D = args[:9]
        nb = b0 * b1
        return "attention", 4 * nb * T * T * D, 4 * nb * T * D + 1024
    if fn is _call_attention_keep:               # also writes the T x T scores and probabilities
        _, q, k, v, o, s, p, b0, b1, T, D = args[:11]
        nb = b0 * b1
        return "attention", 4 * nb * T * T * D, 4 * nb * T * D + 2 * nb * T * T + 1024
    if fn is _copy_view:
        src = args[1]
        return "copy", 0, 2 * src.size * src.itemsize
    f, a = args
    name = getattr(f, "__name__", "")
    if name == "rmsnorm_int":
        rows, cols = a[9], a[10]
        return "rmsnorm", 0, rows * cols * (isz[a[1]] + 1) + cols + 4 * a[4]
    if name == "softmax_lut":
        n = a[4] * a[5] * a[6]
        return "softmax", 0, n * (1 + isz[a[8]]) + 1024
    if name == "add_requant":
        return "add", 0, a[7] * (isz[a[1]] + isz[a[3]] + isz[a[9]])
    if name == "lut_i8":
        return "lut", 0, 2 * a[2] + 256
    if name == "lut_mul":
        return "lut_mul", 0, 3 * a[5] + 256
    return name or "other", 0, 0


def _call_gemm(dev, a: View, bt: View, c: View, b0, b1, M, N, K, strides, op, lut, out_dtype, flags=0):
    dev.gemm_i8(a.ptr, bt.ptr, c.ptr, b0, b1, M, N, K, strides, int(op.M), int(op.s),
                None if lut is None else lut.ptr, out_dtype, flags)


def _call_gemm_group(dev, calls):
    dev.gemm_i8_group([(a.ptr, bt.ptr, c.ptr, b0, b1, M, N, K, strides, int(op.M), int(op.s),
                        None if lut is None else lut.ptr, out_dtype, flags)
                       for _, a, bt, c, b0, b1, M, N, K, strides, op, lut, out_dtype, flags in calls])


def _gemm_bufs(args):
    """(buffers read, buffers written) of a _call_gemm step."""
    _, a, bt, c, *_rest = args
    lut = args[11]
    return {id(a.buf), id(bt.buf)} | ({id(lut.buf)} if lut is not None else set()), {id(c.buf)}


def _group_gemms(P):
    """Merge runs of consecutive _call_gemm steps of which none writes a buffer another one reads or writes (q, k and
    v of one input) into _call_gemm_group steps of at most GEMM_GROUP_MAX products: the library runs such a group as
    one launch when its members share a kernel."""
    steps, works = [], []
    i, n = 0, len(P.steps)
    while i < n:
        j = i + 1
        if P.steps[i][1] is _call_gemm:
            reads, writes = _gemm_bufs(P.steps[i][2])
            while j < n and j - i < rt.GEMM_GROUP_MAX and P.steps[j][1] is _call_gemm:
                r, w = _gemm_bufs(P.steps[j][2])
                if w & (reads | writes) or r & writes:
                    break
                reads, writes = reads | r, writes | w
                j += 1
        if j - i == 1:
            steps.append(P.steps[i])
            works.append(P.works[i])
        else:
            run = P.steps[i:j]
            steps.append(("+".join(lb for lb, _, _ in run), _call_gemm_group, (run[0][2][0], [a for _, _, a in run])))
            works.append(("gemm", sum(w[1] for w in P.works[i:j]), sum(w[2] for w in P.works[i:j])))
        i = j
    P.steps, P.works = steps, works


def _call_attention(dev, q: View, k: View, v: View, o: View, b0, b1, T, D, strides, s_op, sm, o_op, lut: View,
                    flags):
    dev.attention_i8(q.ptr, k.ptr, v.ptr, o.ptr, b0, b1, T, D, strides, int(s_op.M), int(s_op.s), lut.ptr,
                     int(sm.one), bool(sm.causal), int(o_op.M), int(o_op.s), flags)


def _call_attention_keep(dev, q: View, k: View, v: View, o: View, s: View, p: View, b0, b1, T, D, strides, s_op, sm,
                         o_op, lut: View, flags):
    dev.attention_i8_keep(q.ptr, k.ptr, v.ptr, o.ptr, s.ptr, p.ptr, b0, b1, T, D, strides, int(s_op.M), int(s_op.s),
                          lut.ptr, int(sm.one), bool(sm.causal), int(o_op.M), int(o_op.s), flags)


def _call_gemm_add(dev, a: View, bt: View, c, M, N, K, strides, op, lut, r: View, ma, mb, shift2, d: View, rstrides,
                   flags, out_dtype="i8"):
    dev.gemm_i8_add(a.ptr, bt.ptr, None if c is None else c.ptr, 1, 1, M, N, K, strides, int(op.M), int(op.s),
                    None if lut is None else lut.ptr, r.ptr, ma, mb, shift2, d.ptr, rstrides, flags, out_dtype)


def _call_gemm_add_norm(dev, a: View, bt: View, c, M, N, K, strides, op, lut, r: View, ma, mb, shift2, d: View,
                        rstrides, nw: View, nlut: View, norm, h: View, flags):
    dev.gemm_i8_add_norm(a.ptr, bt.ptr, None if c is None else c.ptr, M, N, K, strides, int(op.M), int(op.s),
                         None if lut is None else lut.ptr, r.ptr, ma, mb, shift2, d.ptr, rstrides, nw.ptr, nlut.ptr,
                         nlut.size, int(norm.M), int(norm.s), h.ptr, 64 if h.kb else h.strides[-2], h.kb, flags)


def _swap_last2(n):
    return list(range(n - 2)) + [n - 1, n - 2]


def compile(model, example_inputs=None, calib_inputs=None, params=None, schedules=None, *, consts=None,
            device: int = 0, prove: bool = True, embedding=None, **kw) -> CompiledModel:   # noqa: A001
    """anvil.compile for the mi355x backend (reference anvil/driver.py:330-335). params / schedules configure the
    reference's tiny-gpu targets and are ignored here; example_inputs / calib_inputs only apply to torch modules,
    which this backend does not capture. prove=False skips the static int32 proof for a hand-built graph, as the
    reference's graph-level Vortex-V compile does (anvil/vortexv/__init__.py:117-123): every kernel still checks
    each intermediate on the device, so a run that leaves int32 raises OverflowError like the interpreter.
    embedding=(wte, wpe): the token and position tables (float32, (vocab, C) and (>= T, C)) of a token model whose
    graph input is x = wte[ids] + wpe[positions]; cm.run(ids, tokens=True) then gathers and quantizes on the device.
    A built token model (models.config(4)) brings its own tables."""
    if kw:
        raise TypeError(f"compile() got unexpected keyword argument(s) {sorted(kw)}")
    module, cs = _resolve_model(model, consts, prove)
    from .models import Built
    cm = CompiledModel(module, cs, device=device, proven=prove or isinstance(model, Built))
    if embedding is None and isinstance(model, Built) and model.spec.vocab:
        embedding = (model.params["wte"], model.params["wpe"])
    if embedding is not None:
        cm.set_embedding(*embedding)
    return cm
