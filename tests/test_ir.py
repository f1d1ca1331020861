"""Graph IR: the builder's types and the verifier rules of the reference dialect (anvil/ir/graph.py:189-342)."""
import numpy as np
import pytest

from anvil_mi355x.ir import GraphBuilder, QTensorType, VerifyException, funcs


def test_builder_types_and_module():
    g = GraphBuilder("mha")
    x = g.input("x", [4, 8], scale=0.03)
    w = g.const("w", [8, 6])
    y = g.qlinear("y", x, w, 600, 12, scale=0.05)
    r = g.reshape("y.r", y, [4, 2, 3])
    t = g.transpose("yh", r, [1, 0, 2])
    assert y.type == QTensorType([4, 6], "i8", 0.05)
    assert t.type.dims == [2, 4, 3] and t.type.qscale == 0.05
    assert g.transpose("tt", y).type.dims == [6, 4]               # default perm reverses the axes
    g.output(y)
    m = g.module()
    assert m is g.module() and len(funcs(m)) == 1 and funcs(m)[0].sym_name == "mha"


def test_head_batched_qmatmul_shapes():
    """tests/model/test_multihead_ir.py:47-59."""
    g = GraphBuilder("bad")
    a = g.input("a", [2, 4, 3])
    b = g.input("b", [3, 3, 5])
    with pytest.raises(VerifyException, match="need"):
        g.qmatmul("c", a, b, 1, 0)
    g = GraphBuilder("bad2")
    a = g.input("a", [2, 4, 3])
    w = g.const("w", [2, 3, 5])
    with pytest.raises(VerifyException, match=r"\(K, N\)"):
        g.qlinear("c", a, w, 1, 0)
    g = GraphBuilder("ok")
    a = g.input("a", [2, 4, 3])
    assert g.qmatmul("c", a, g.input("b", [2, 3, 5]), 1, 0).type.dims == [2, 4, 5]


def test_wide_types():
    """tests/lower/test_wide_residual.py:82-89: matmul operands stay i8; a LUT epilogue needs an i8 result."""
    b = GraphBuilder("bad")
    x = b.input("x", [4, 8], "i16", 1.0)
    with pytest.raises(VerifyException):
        b.qlinear("q", x, b.const("w", [8, 8]), 1, 0)
    h = b.input("h", [4, 8], "i8", 1.0)
    with pytest.raises(VerifyException):
        b.qlinear("q", h, b.const("w2", [8, 8]), 1, 0, lut=b.const("l", [256]), dtype="i16")


def test_verifier_rejections():
    b = GraphBuilder("v")
    x = b.input("x", [4, 8])
    lut32 = b.const("e", [256], "i32")
    with pytest.raises(VerifyException):
        b.qlinear("q", x, b.const("w", [8, 8]), 1, 32)                 # shift outside [0, 31]
    with pytest.raises(VerifyException):
        b.qlinear("q", x, b.input("nw", [8, 8]), 1, 3)                 # qlinear weight must be a const
    with pytest.raises(VerifyException):
        b.softmax_lut("p", x, lut32, 128)                              # one does not fit i8
    b.softmax_lut("p32", x, lut32, 4096, dtype="i32")
    with pytest.raises(VerifyException):
        b.softmax_lut("p", x, b.const("e8", [256]), 127)               # exp LUT must be i32
    with pytest.raises(VerifyException):
        b.rmsnorm_int("h", x, b.const("nw", [7]), b.const("r", [64], "i32"), 1, 3)   # weight length
    with pytest.raises(VerifyException):
        b.rmsnorm_int("h", x, b.const("nw2", [8]), b.const("r2", [64], "i32"), 1, 3, ss_shift=31)
    with pytest.raises(VerifyException):
        b.lut("l", x, b.const("t", [255]))                             # LUT must be 256 x i8
    with pytest.raises(VerifyException):
        b.add_requant("r", x, b.input("y", [4, 9]), 1, 1, 0)           # shapes differ
    with pytest.raises(VerifyException):
        b.transpose("t", x, [0, 0])
    with pytest.raises(VerifyException):
        b.reshape("r", x, [5, 7])
    with pytest.raises(VerifyException):
        b.lut_mul("lm", x, b.input("y2", [4, 8], "i16"), b.const("t2", [256]), 1, 0)
    with pytest.raises(VerifyException):
        QTensorType([0, 3])
    with pytest.raises(ValueError):
        QTensorType([3], "i4")


def test_inline_const_values():
    g = GraphBuilder("c")
    v = g.const("w", [2, 3], value=np.arange(6).reshape(2, 3))
    assert v.owner.value.shape == (2, 3)
    with pytest.raises(ValueError):
        g.const("bad", [4], value=np.arange(6))
