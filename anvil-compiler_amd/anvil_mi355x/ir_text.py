"""The textual form of anvil.graph modules: MLIR's generic op syntax, as the reference prints and parses it.

    text = print_ir(module); module2 = parse_ir(text)          # reference anvil/ir/__init__.py:22-31

The reference round-trips this text through xDSL (its `print_ir` / `parse_ir`, tested as
`print_ir(parse_ir(text)) == text` in tests/model/test_multihead_ir.py:49-50). xDSL is not a dependency here, so
this module reads and writes the subset of the generic syntax that anvil.graph modules use:

    builtin.module {
      "anvil.graph.func"() <{sym_name = "model"}> ({
        %0 = "anvil.graph.input"() <{sym = "x"}> : () -> !anvil.graph.qtensor<16x32xi16, 4.02106646095407375e-04>
        %5 = "anvil.graph.qlinear"(%3, %4) <{M = 6102 : i64, s = 21 : i64, sym = "L0.q"}> : (...) -> !anvil.graph....
        "anvil.graph.output"(%74) : (!anvil.graph.qtensor<16x32xi16, ...>) -> ()
      }) : () -> ()
    }

Properties print in the order the op holds them (a parsed op keeps the text's order). Integers print as
`N : i64`, booleans as `true` / `false`, permutations as `array<i64: ...>`, inline const values as
`dense<...> : tensor<...xi64>`, and qtensor scales with 17 significant decimals (anvil/ir/graph.py:99-113).
"""
from __future__ import annotations

import re

import numpy as np

from . import ir as g

_TYPE_RE = re.compile(r"!anvil\.graph\.qtensor<((?:\d+x)+)(i8|i16|i32)(?:,\s*([-+0-9.eE]+))?>")


# ------------------------------------------------------------------------------------------------- printing

def print_type(t: g.QTensorType) -> str:
    dims = "".join(f"{d}x" for d in t.shape)
    scale = "" if t.scale is None else f", {t.scale:.17e}"
    return f"!anvil.graph.qtensor<{dims}{t.dtype}{scale}>"


def _print_value(key, v) -> str:
    if isinstance(v, (bool, np.bool_)):
        return "true" if v else "false"
    if isinstance(v, str):
        return '"' + v.replace("\\", "\\\\").replace('"', '\\"') + '"'
    if key == "perm":
        return "array<i64: " + ", ".join(str(int(p)) for p in v) + ">"
    if key == "value":
        a = np.asarray(v, dtype=np.int64)
        return f"dense<{_nested(a)}> : tensor<{''.join(f'{d}x' for d in a.shape)}i64>"
    return f"{int(v)} : i64"


def _nested(a) -> str:
    if a.ndim == 0:
        return str(int(a))
    return "[" + ", ".join(_nested(x) for x in a) + "]"


def _props(op) -> list:
    """(key, value) pairs in the op's order, then sym: the order the reference's builder gives them."""
    items = list(getattr(op, "prop_order", None) or [])
    if not items:
        items = [k for k in op.props if op.props[k] is not None and not (k in ("ss_shift", "ss_init")
                                                                             and not op.props[k])]
        if op.sym is not None:
            items.append("sym")
    return [(k, op.sym if k == "sym" else op.props[k]) for k in items]


def print_ir(module) -> str:
    """The module as the reference's print_ir writes it (trailing newline included)."""
    lines = ["builtin.module {"]
    for f in g.funcs(module):
        lines.append(f'  "anvil.graph.func"() <{{sym_name = "{f.sym_name}"}}> ({{')
        names = {}
        for op in f.ops:
            operands = op.operands
            args = ", ".join(names[v] for v in operands)
            props = _props(op) if not isinstance(op, g.OutputOp) else []
            ptxt = (" <{" + ", ".join(f"{k} = {_print_value(k, v)}" for k, v in props) + "}>") if props else ""
            in_types = ", ".join(print_type(v.type) for v in operands)
            if op.results:
                name = f"%{len(names)}"
                names[op.result] = name
                lines.append(f'    {name} = "{op.name}"({args}){ptxt} : ({in_types}) -> {print_type(op.result.type)}')
            else:
                lines.append(f'    "{op.name}"({args}){ptxt} : ({in_types}) -> ()')
        lines.append("  }) : () -> ()")
    lines.append("}")
    return "\n".join(lines) + "\n"


# -------------------------------------------------------------------------------------------------- parsing

class _Cursor:
    def __init__(self, text: str, line: int):
        self.s, self.i, self.line = text, 0, line

    def error(self, msg):
        return ValueError(f"anvil IR line {self.line}: {msg} at {self.s[self.i:self.i + 40]!r}")

    def ws(self):
        while self.i < len(self.s) and self.s[self.i] in " \t":
            self.i += 1

    def peek(self, tok: str) -> bool:
        self.ws()
        return self.s.startswith(tok, self.i)

    def take(self, tok: str):
        self.ws()
        if not self.s.startswith(tok, self.i):
            raise self.error(f"expected {tok!r}")
        self.i += len(tok)

    def balanced(self, stop: str) -> str:
        """Text up to the first `stop` outside <...>, [...] and quotes."""
        self.ws()
        depth, j, quoted = 0, self.i, False
        while j < len(self.s):
            c = self.s[j]
            if quoted:
                if c == "\\":
                    j += 1
                elif c == '"':
                    quoted = False
            elif c == '"':
                quoted = True
            elif c in "<[(":
                depth += 1
            elif c in ">])":
                if depth == 0 and self.s.startswith(stop, j):
                    break
                depth -= 1
            elif depth == 0 and self.s.startswith(stop, j):
                break
            j += 1
        out, self.i = self.s[self.i:j], j
        return out.strip()


def _split_top(text: str) -> list:
    parts, depth, cur, quoted = [], 0, [], False
    for c in text:
        if quoted:
            cur.append(c)
            quoted = c != '"' or (len(cur) > 1 and cur[-2] == "\\")
            continue
        if c == '"':
            quoted = True
        elif c in "<[(":
            depth += 1
        elif c in ">])":
            depth -= 1
        if c == "," and depth == 0:
            parts.append("".join(cur).strip())
            cur = []
        else:
            cur.append(c)
    if "".join(cur).strip():
        parts.append("".join(cur).strip())
    return parts


def parse_type(text: str) -> g.QTensorType:
    m = _TYPE_RE.fullmatch(text.strip())
    if not m:
        raise ValueError(f"not an anvil.graph.qtensor type: {text!r}")
    dims = [int(d) for d in m.group(1).split("x") if d]
    return g.QTensorType(dims, m.group(2), None if m.group(3) is None else float(m.group(3)))


def _parse_value(key: str, text: str):
    text = text.strip()
    if text in ("true", "false"):
        return text == "true"
    if text.startswith('"'):
        return bytes(text[1:-1], "utf-8").decode("unicode_escape")
    if text.startswith("array<"):
        body = text[len("array<"):-1]
        _, _, nums = body.partition(":")
        return [int(x) for x in nums.split(",") if x.strip()]
    if text.startswith("dense<"):
        body, _, ttype = text.rpartition(":")
        inner = body.strip()[len("dense<"):-1]
        dims = [int(d) for d in re.findall(r"(\d+)x", ttype)]
        vals = np.array([int(x) for x in re.findall(r"-?\d+", inner)], dtype=np.int64)
        return vals.reshape(dims) if dims else vals.reshape(())
    m = re.fullmatch(r"(-?\d+)\s*:\s*i\d+", text)
    if m:
        return int(m.group(1))
    raise ValueError(f"property {key}: unsupported value {text!r}")


def _parse_op(cur: _Cursor, values: dict):
    result = None
    if cur.peek("%"):
        result = cur.balanced("=")
        cur.take("=")
    cur.take('"')
    j = cur.s.index('"', cur.i)
    name, cur.i = cur.s[cur.i:j], j + 1
    cur.take("(")
    args = [a.strip() for a in cur.balanced(")").split(",") if a.strip()]
    cur.take(")")
    props = []
    if cur.peek("<{"):
        cur.take("<{")
        body = cur.balanced("}>")
        cur.take("}>")
        for item in _split_top(body):
            k, _, v = item.partition("=")
            props.append((k.strip(), _parse_value(k.strip(), v)))
    cur.take(":")
    cur.take("(")
    in_types = [parse_type(t) for t in _split_top(cur.balanced(")"))]
    cur.take(")")
    cur.take("->")
    out = cur.s[cur.i:].strip()
    if name not in g.OPS:
        raise NotImplementedError(f"anvil IR line {cur.line}: op {name!r} is not an anvil.graph op")
    try:
        operands = [values[a] for a in args]
    except KeyError as e:
        raise ValueError(f"anvil IR line {cur.line}: undefined value {e.args[0]}") from None
    for v, t in zip(operands, in_types):
        if v.type != t:
            raise ValueError(f"anvil IR line {cur.line}: operand type {t} != the value's {v.type}")
    cls = g.OPS[name]
    pd = dict(props)
    sym = pd.pop("sym", None)
    if cls is g.OutputOp:
        if out != "()":
            raise ValueError(f"anvil IR line {cur.line}: output has results")
        return None, g.OutputOp(operands)
    names = [n for n in cls.OPERANDS]
    if len(operands) > len(names) or len(operands) < len(names) - len(cls.OPTIONAL):
        raise ValueError(f"anvil IR line {cur.line}: {name} takes {len(names)} operands, got {len(operands)}")
    op = cls(dict(zip(names, operands)), pd, parse_type(out), sym)
    op.prop_order = [k for k, _ in props]
    op.verify()
    return result, op


def parse_ir(text: str):
    """A Module from the reference's textual form (one anvil.graph.func per module, as the reference writes)."""
    lines = text.splitlines()
    funcs, cur_func, values = [], None, {}
    for n, raw in enumerate(lines, 1):
        line = raw.strip()
        if not line or line in ("builtin.module {", "}"):
            continue
        m = re.fullmatch(r'"anvil\.graph\.func"\(\)\s*<\{sym_name = "([^"]*)"\}>\s*\(\{', line)
        if m:
            cur_func, values = g.FuncOp(m.group(1)), {}
            continue
        if line == "}) : () -> ()":
            if cur_func is None:
                raise ValueError(f"anvil IR line {n}: unbalanced region")
            funcs.append(cur_func)
            cur_func = None
            continue
        if cur_func is None:
            raise ValueError(f"anvil IR line {n}: op outside an anvil.graph.func: {line[:60]!r}")
        name, op = _parse_op(_Cursor(line, n), values)
        cur_func.ops.append(op)
        if name is not None:
            if name in values:
                raise ValueError(f"anvil IR line {n}: {name} defined twice")
            values[name] = op.result
    if cur_func is not None:
        raise ValueError("anvil IR: unterminated anvil.graph.func")
    if not funcs:
        raise ValueError("anvil IR: no anvil.graph.func")
    return g.Module(*funcs)
