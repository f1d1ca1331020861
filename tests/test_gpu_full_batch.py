"""GPU parity on the whole evaluation batch of every block config, for both read-back policies.

keep="all" returns every graph value and plans every op on its own kernel (plus the fused residual adds);
keep="outputs" is the benchmarked plan (fused attention, causal tile skipping, grouped q/k/v GEMMs, fused adds).
Every sequence of every returned value is compared with the oracle's SHA-256 digest of the same sequence in
tests/golden/block_digests.json (written by tests/golden/make_block_digests.py from oracle/interp.py), so indexing
mistakes that hit only some batch entries or heads cannot pass.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import anvil_mi355x
from anvil_mi355x import models
from test_quantize_recipe import constants_digest

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "block_digests.json").read_text())
NP = {"i8": "<i1", "i16": "<i2", "i32": "<i4"}


@pytest.mark.parametrize("keep", ["outputs", "all"])
@pytest.mark.parametrize("n", [1, 3, 4, 5])
def test_full_batch_matches_oracle_digests(n, keep):
    gold = GOLDEN["configs"][str(n)]
    built, nb = models.config(n)
    assert constants_digest(built) == gold["constants_sha256"]
    cm = anvil_mi355x.compile(built)
    x = models.to_float_input(built.spec, built.params, models.eval_inputs(built.spec, nb, models.config_tag(n)))
    res = cm.run(x, "mi355x", batch=True, keep=keep)
    want_syms = set(gold["values"]) if keep == "all" else set(cm.inputs + cm.outputs)
    assert set(res.ints) == want_syms
    dtypes = {s: cm.meta[s][2] for s in res.ints}
    bad = []
    for s, a in res.ints.items():
        a = np.asarray(a).astype(NP[dtypes[s]])
        assert a.shape[0] == nb == gold["batch"]
        for i in range(nb):
            if hashlib.sha256(np.ascontiguousarray(a[i]).tobytes()).hexdigest()[:32] != gold["sequences"][i][s]:
                bad.append((s, i))
    assert not bad, f"config {n} keep={keep}: {len(bad)} mismatching (value, sequence) pairs, first {bad[:8]}"
