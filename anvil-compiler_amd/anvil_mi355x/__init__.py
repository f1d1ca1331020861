"""anvil_mi355x: an MI355X (gfx950) backend for the int8 graph evaluation that Anvil's interpreter defines.

    import anvil_mi355x as anvil
    cm = anvil.compile((module, consts))         # built with GraphBuilder, or anvil.parse_ir(text) of the
                                                 # reference's printed IR
    res = cm.run(x, "mi355x")                    # res.output, res.outputs, res.ints[sym], res.cycles

Mirrors the reference's public surface (anvil/__init__.py:9-12 -> anvil/driver.py:330-335) for the graph path:
the graph IR and builder (anvil/ir/graph.py), the quantizer's numeric recipe (anvil/frontend/quantize.py), and
compile / CompiledModel.run / RunOutput (anvil/driver.py), with "mi355x" as the backend. Every op runs as a
hand-written HIP kernel for gfx950 through the C ABI of libanvil_mi355x.so (include/anvil_mi355x.h).
"""
from . import ir
from .ir import GraphBuilder, QTensorType, VerifyException, parse_ir, print_ir


def compile(*args, **kw):  # noqa: A001  (the public entry point shadows the builtin inside this package only)
    """anvil_mi355x.driver.compile (imported lazily so `import anvil_mi355x` stays light)."""
    from .driver import compile as _compile
    return _compile(*args, **kw)


__all__ = ["compile", "ir", "GraphBuilder", "QTensorType", "VerifyException", "parse_ir", "print_ir"]
