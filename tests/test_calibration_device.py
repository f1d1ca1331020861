"""The calibration forward on a torch device (models.calibrate_on_device) against the host forward
(models.calibrate, reference anvil/frontend/quantize.py:276-300): the same input scale, the same activation
symbols, and max-abs values equal to float32 rounding. Run here with torch's CPU device; the GPU test runs it on the
MI355X and evaluates the graph built from it against the oracle."""
import numpy as np
import pytest

from anvil_mi355x import models

SPECS = [
    models.BlockSpec(n_embd=128, n_head=2, seq=64, calib_batches=2, calib_batch=4),
    models.BlockSpec(n_embd=64, n_head=2, seq=32, causal=False, calib_batches=2, calib_batch=3),
    models.BlockSpec(n_embd=128, n_head=4, seq=64, layers=2, vocab=256, calib_batches=2, calib_batch=4),
]


@pytest.mark.parametrize("spec", SPECS, ids=["block", "noncausal", "vocab2"])
def test_device_forward_matches_the_host_forward(spec):
    params = models.init_params(spec)
    sin, amax = models.calibrate(spec, params, 7)
    sin_d, amax_d = models.calibrate_on_device(spec, params, 7, "cpu")
    assert sin_d == sin
    assert sorted(amax_d) == sorted(amax)
    for k, v in amax.items():
        assert v > 0 and abs(amax_d[k] / v - 1) < 1e-5, k


def test_build_takes_the_device_calibration():
    """build(calib_device=...) ignores the tracked calibration and uses the device forward's values."""
    spec = SPECS[0]
    built = models.build(spec, 7, calib_device="cpu")
    sin, amax = models.calibrate_on_device(spec, models.init_params(spec), 7, "cpu")
    want = models.build_graph(spec, models.init_params(spec), sin, amax)
    assert built.scales == want.scales
    assert all(np.array_equal(np.asarray(built.consts[k]), np.asarray(want.consts[k])) for k in want.consts)
