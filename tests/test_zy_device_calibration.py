"""The calibration forward on the MI355X (models.calibrate_on_device, reference anvil/frontend/quantize.py:276-300,
with torch on "cuda") against the host forward, and the graph built from it against the oracle. Collected after
every other GPU test: its child process makes the box's first `import torch`, which can take a minute or two."""
import json
import subprocess
import sys

import numpy as np
import pytest

import anvil_mi355x
import helpers
from anvil_mi355x import models
from oracle import interp


@pytest.mark.gpu
@pytest.mark.timeout(300)
def test_device_calibration_on_the_gpu():
    """The calibration forward on the MI355X (models.calibrate_on_device with torch on "cuda", run in a child
    process so that this test process keeps one GPU client): the host's input scale and activation symbols, max-abs
    values equal to the host forward's to float32 rounding, and the graph built from them bit-exact against the
    oracle in every value."""
    spec = models.BlockSpec(n_embd=256, n_head=4, seq=256, calib_batches=2, calib_batch=8)
    child = ("import json, sys; sys.path.insert(0, %r); from anvil_mi355x import models; "
             "spec = models.BlockSpec(n_embd=256, n_head=4, seq=256, calib_batches=2, calib_batch=8); "
             "sin, amax = models.calibrate_on_device(spec, models.init_params(spec), 13, 'cuda'); "
             "print(json.dumps({'sin': sin, 'amax': amax}))" % str(helpers.ROOT / "anvil-compiler_amd"))
    print("device calibration child: n_embd 256, 4 heads, seq 256, 2 x 8 sequences", flush=True)
    out = subprocess.run([sys.executable, "-c", child], capture_output=True, text=True, timeout=280)
    assert out.returncode == 0, out.stderr[-2000:]
    dev = json.loads(out.stdout.strip().splitlines()[-1])
    params = models.init_params(spec)
    sin, amax = models.calibrate(spec, params, 13)
    assert dev["sin"] == sin and sorted(dev["amax"]) == sorted(amax)
    assert max(abs(dev["amax"][k] / amax[k] - 1) for k in amax) < 1e-4
    built = models.build_graph(spec, params, dev["sin"], dev["amax"])
    cm = anvil_mi355x.compile(built)
    x = models.eval_inputs(spec, 2, 13)
    res = cm.run(x, "mi355x", batch=True, keep="all")
    want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
    for k, v in res.ints.items():
        assert np.array_equal(v, want.values[k]), k
