"""The reference-side binding in the integration guide at the repository root, executed as written against a
stand-in `anvil` package.

The stand-in's CompiledModel lowers and memory-plans for tiny-gpu the way the reference's does
(anvil/driver.py:178-210), except that both steps raise here: a graph that reaches them fails the test. The
config-5 graph must go compile(..., backend="mi355x") -> run(x, "mi355x") without them, and its outputs must equal
the oracle's (the device calls run on the CPU stand-in of the C ABI, tests/fake_device.py)."""
import re
import sys
import types
from pathlib import Path

import numpy as np
import pytest

import anvil_mi355x
import fake_device
from anvil_mi355x import models
from anvil_mi355x import quantize as Q
from anvil_mi355x import runtime as rt
from anvil_mi355x.ir_text import print_ir
from oracle import interp

ROOT = Path(__file__).resolve().parents[1]
GUIDE = ROOT / "INTEGRATION.md"


def snippet(tag):
    text = GUIDE.read_text()
    m = re.search(rf"<!-- binding:{tag} -->\s*```python\n(.*?)```", text, re.S)
    assert m, f"{GUIDE.name} has no binding:{tag} block"
    return m.group(1)


class TinyGpuReached(AssertionError):
    pass


def stand_in_driver(monkeypatch):
    """anvil.driver's namespace with what the compile snippet uses; tiny-gpu lowering and planning raise."""
    anvil = types.ModuleType("anvil")
    ir = types.ModuleType("anvil.ir")
    ir.print_ir = print_ir
    anvil.ir = ir
    monkeypatch.setitem(sys.modules, "anvil", anvil)
    monkeypatch.setitem(sys.modules, "anvil.ir", ir)

    def lower(module):
        raise TinyGpuReached("tiny-gpu lowering ran")

    def memory_plan(*a, **k):
        raise TinyGpuReached("tiny-gpu memory planning ran")

    class GpuParams:
        pass

    class CompiledModel:
        def __init__(self, module, consts, params, schedules=None, **kw):
            self.program = lower(module)
            self.plan = memory_plan(self.program)

    def _resolve_model(model, example_inputs, calib_inputs, consts, quant_kw):
        module, cs = model                            # a (module, consts) pair: the reference's _checked_graph
        Q.prove_no_overflow(module, cs)
        return module, dict(cs), None

    ns = {"lower": lower, "memory_plan": memory_plan, "GpuParams": GpuParams, "CompiledModel": CompiledModel,
          "_resolve_model": _resolve_model}
    exec(snippet("compile"), ns)
    return ns


def test_compile_snippet_runs_config5_without_tiny_gpu(monkeypatch):
    dev = fake_device.FakeDevice(heap_bytes=1 << 27, fast=True)
    monkeypatch.setattr(rt, "device", lambda index=0: dev)
    ns = stand_in_driver(monkeypatch)
    built, _ = models.config(5)
    with pytest.raises(TinyGpuReached):                       # today's path builds tiny-gpu artefacts
        ns["compile"]((built.module, built.consts))
    with pytest.raises(ValueError, match="unknown backend"):
        ns["compile"]((built.module, built.consts), backend="isasim-gpu")
    cm = ns["compile"]((built.module, built.consts), backend="mi355x")
    from anvil_mi355x.driver import CompiledModel
    assert isinstance(cm, CompiledModel) and cm.proven
    x = models.eval_inputs(built.spec, 1, 77)[0]
    res = cm.run(x, "mi355x")
    want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, fast=True)
    assert np.array_equal(res.ints["out"], want.values["out"])
    assert np.allclose(res.output, want.values["out"] * built.scales["out"])
    assert any(c[0] == "attention" for c in dev.calls)       # the benchmarked plan: fused attention


def test_run_snippet_is_valid_python():
    body = "\n".join(("    " + ln if ln.startswith("#") else ln) for ln in snippet("run").splitlines())
    compile("class CompiledModel:\n" + body.replace("        ...", "        pass"), GUIDE.name, "exec")
