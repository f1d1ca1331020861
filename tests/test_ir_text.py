"""The reference's textual IR: exact round trips of the reference's own frozen model files, error reporting, and
the planner (CPU stand-in of the C ABI) on those models against the oracle (reference anvil/ir/__init__.py:22-31,
tests/model/test_multihead_ir.py:49-50, anvil/codesign/workloads.py:62-72)."""
import numpy as np
import pytest

import anvil_mi355x
import fake_device
import helpers
from anvil_mi355x import ir as g
from anvil_mi355x import models
from anvil_mi355x import runtime as rt
from oracle import interp

fixture = helpers.reference_model


@pytest.mark.parametrize("name", ["v1", "v2"])
def test_reference_model_files_round_trip_exactly(name):
    text, consts, _ = fixture(name)
    m = anvil_mi355x.parse_ir(text)
    assert anvil_mi355x.print_ir(m) == text
    ops = g.func_of(m).ops
    assert sum(isinstance(o, g.ConstOp) for o in ops) == len(consts) == 26
    wide = name == "v2"
    assert (g.qt(ops[0].result).dtype == "i16") == wide
    norm = [o for o in ops if isinstance(o, g.RmsNormIntOp)]
    assert (norm[0].ss_shift_int, norm[0].ss_init_int) == ((5, 6) if wide else (0, 0))


@pytest.mark.parametrize("n", [1, 3, 4])
def test_built_configs_print_parse_print(n):
    built, _ = models.config(n)
    text = anvil_mi355x.print_ir(built.module)
    again = anvil_mi355x.parse_ir(text)
    assert anvil_mi355x.print_ir(again) == text
    t = g.qt(next(o for o in g.func_of(again).ops if isinstance(o, g.InputOp)).result)
    assert t == g.qt(next(o for o in g.func_of(built.module).ops if isinstance(o, g.InputOp)).result)
    xq = np.random.default_rng(n).integers(-128, 128, (2, *t.shape))
    a = interp.run(built.module, {"x": xq}, built.consts, batch=True)
    b = interp.run(again, {"x": xq}, built.consts, batch=True)
    assert all(np.array_equal(a.values[k], b.values[k]) for k in a.values)


def test_parse_errors():
    text, _, _ = fixture("v1")
    with pytest.raises(ValueError, match="undefined value"):
        anvil_mi355x.parse_ir(text.replace('"anvil.graph.qlinear"(%3, %4)', '"anvil.graph.qlinear"(%3, %99)', 1))
    with pytest.raises(NotImplementedError, match="anvil.graph.conv"):
        anvil_mi355x.parse_ir(text.replace('"anvil.graph.lut_mul"', '"anvil.graph.conv"', 1))
    with pytest.raises(g.VerifyException):
        anvil_mi355x.parse_ir(text.replace("perm = array<i64: 1, 0, 2>", "perm = array<i64: 1, 1, 2>", 1))
    with pytest.raises(ValueError, match="operand type"):
        anvil_mi355x.parse_ir(text.replace('<{sym = "L0.qh.r"}> : (!anvil.graph.qtensor<16x32xi8',
                                           '<{sym = "L0.qh.r"}> : (!anvil.graph.qtensor<16x32xi16', 1))
    with pytest.raises(g.VerifyException, match="reshape"):
        anvil_mi355x.parse_ir(text.replace("-> !anvil.graph.qtensor<16x2x16xi8", "-> !anvil.graph.qtensor<16x2x16xi16",
                                           1))
    with pytest.raises(ValueError, match="qtensor"):
        anvil_mi355x.parse_ir(text.replace("qtensor<16x32xi8", "qtensor<16x32xf8", 1))


@pytest.fixture
def fake(monkeypatch):
    dev = fake_device.FakeDevice()
    monkeypatch.setattr(rt, "device", lambda index=0: dev)
    return dev


@pytest.mark.parametrize("name", ["v1", "v2"])
def test_planner_runs_the_reference_models(fake, name):
    text, consts, x = fixture(name)
    m = anvil_mi355x.parse_ir(text)
    cm = anvil_mi355x.compile((m, consts))
    xs = x[None] if x is not None else np.random.default_rng(3).integers(-128, 128, (3, 16, 32))
    want = interp.run(m, {"x": xs}, consts, batch=True)
    res = cm.run(xs, quantized=True, batch=True, keep="all")
    for k, v in want.values.items():
        if k not in consts:
            assert np.array_equal(res.ints[k], v), k
    out = cm.run(xs, quantized=True, batch=True).ints
    assert np.array_equal(out["L1.out"], want.values["L1.out"])


def test_compile_accepts_printed_ir(fake):
    text, consts, x = fixture("v2")
    a = anvil_mi355x.compile((text, consts)).run(x, quantized=True).ints["L1.out"]
    b = anvil_mi355x.compile(anvil_mi355x.parse_ir(text), consts=consts).run(x, quantized=True).ints["L1.out"]
    assert np.array_equal(a, b)
    assert np.array_equal(a, interp.run(anvil_mi355x.parse_ir(text), {"x": x}, consts).values["L1.out"])
