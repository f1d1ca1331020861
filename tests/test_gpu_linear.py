"""Config 2 on the production path: a one-qlinear graph through anvil_mi355x.compile (proven, so the unchecked fast
GEMM kernels run), all six shapes, every output element compared with the oracle (float64 BLAS matmul, exact for
these magnitudes, then the reference's requant: anvil/semantics.py:95-103)."""
import numpy as np
import pytest

import anvil_mi355x
from anvil_mi355x import models
from anvil_mi355x import runtime as rt
from oracle import semantics as sem

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K", models.LINEAR_SHAPES)
def test_linear_sweep_full_output(M, K):
    lin = models.linear_config(M, K)
    cm = anvil_mi355x.compile((lin.module, lin.consts))
    assert cm.proven
    plan = cm.plan(1)
    flags = [a[-1] for _, fn, a in plan.steps if getattr(fn, "__name__", "") == "_call_gemm"]
    assert flags and all(f & rt.GEMM_UNCHECKED for f in flags)
    got = cm.run(lin.x, "mi355x", quantized=True).ints["y"]
    want = sem.qmatmul(lin.x, lin.consts["w"], lin.mult, lin.shift, fast=True)
    assert got.shape == (M, K)
    mism = np.argwhere(got != want)
    assert mism.size == 0, f"{len(mism)} mismatches, first at {mism[:4].tolist()}"
    # the outputs spread over int8 rather than collapsing to a few values
    assert len(np.unique(got)) > 100
