"""Write tests/golden/block_digests.json: per sequence, the SHA-256 of every graph value of block configs 1, 3, 4 and
5 on their evaluation batch, as the oracle (oracle/interp.py, float64-BLAS matmuls, exact) computes them.

    python tests/golden/make_block_digests.py [--jobs 8]

Each value is hashed at its graph dtype (little-endian i8 / i16 / i32), one sequence at a time, in the logical
(row-major) order of the value's dims. The inputs are the configs' seeded evaluation batches (models.eval_inputs with
the config's tag), quantized on the host (CompiledModel.quantize_input: float64 rint, clamp); the graphs are built
from the tracked calibration (anvil_mi355x/calib/), and each config's constants digest is stored beside its
sequence digests, so a graph that changes is reported as such rather than as a kernel mismatch.
"""
import argparse
import hashlib
import json
import multiprocessing as mp
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "anvil-compiler_amd"), str(ROOT), str(ROOT / "tests")]

import numpy as np  # noqa: E402

OUT = Path(__file__).resolve().parent / "block_digests.json"
CONFIGS = (1, 3, 4, 5)
NP = {"i8": "<i1", "i16": "<i2", "i32": "<i4"}
_STATE = {}


def value_digest(a, dtype) -> str:
    return hashlib.sha256(np.ascontiguousarray(np.asarray(a).astype(NP[dtype])).tobytes()).hexdigest()[:32]


def graph_values(built):
    """(sym, dtype) of every non-const value of the graph, in graph order (what keep="all" returns)."""
    from anvil_mi355x import ir as g
    consts, out = set(), []
    for op in g.func_of(built.module).ops:
        if isinstance(op, g.OutputOp):
            continue
        if isinstance(op, g.ConstOp) or (isinstance(op, (g.TransposeOp, g.ReshapeOp)) and op.x in consts):
            consts.add(op.result)
            continue
        out.append((op.sym_str, g.qt(op.result).dtype))
    return out


def _sequence(i):
    from oracle import interp
    built, xq, syms = _STATE["built"], _STATE["xq"], _STATE["syms"]
    r = interp.run(built.module, {"x": xq[i:i + 1]}, built.consts, batch=True, fast=True)
    return {s: value_digest(r.values[s][0], dt) for s, dt in syms}


def config_inputs(n):
    """(built, compiled model, quantized evaluation batch) of config n."""
    import anvil_mi355x
    from anvil_mi355x import models
    built, nb = models.config(n)
    cm = anvil_mi355x.compile(built)
    x = models.to_float_input(built.spec, built.params, models.eval_inputs(built.spec, nb, models.config_tag(n)))
    return built, cm, cm.quantize_input(x)


def main():
    from test_quantize_recipe import constants_digest
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    args = ap.parse_args()
    body = {"about": "per-sequence sha256[:32] of every non-const graph value at its dtype, from the oracle",
            "configs": {}}
    for n in CONFIGS:
        built, cm, xq = config_inputs(n)
        syms = graph_values(built)
        _STATE.update(built=built, xq=xq, syms=syms)
        with mp.get_context("fork").Pool(args.jobs) as pool:
            seqs = pool.map(_sequence, range(len(xq)))
        body["configs"][str(n)] = {"constants_sha256": constants_digest(built), "batch": len(xq),
                                   "values": [s for s, _ in syms], "sequences": seqs}
        print(f"config {n}: {len(xq)} sequences, {len(syms)} values", flush=True)
    OUT.write_text(json.dumps(body, indent=0, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
