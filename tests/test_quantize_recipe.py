"""The built configurations' constants, the tracked calibration they come from, and the two int32 proof policies."""
import hashlib
import json

import numpy as np
import pytest

import anvil_mi355x
from anvil_mi355x import models
from anvil_mi355x import quantize as Q
from anvil_mi355x.ir import GraphBuilder
from anvil_mi355x.ir_text import print_ir

# sha256 over each built graph's printed IR (every M, s, Ma, Mb, one, shift and scale) and its consts (weights and
# tables), taken before the quantizer's rewrite: configs must build bit-identical constants from the tracked
# calibration, whatever the recipe's code looks like.
CONSTANTS_SHA256 = {
    1: "f35b30277371215af612706cda78d128b788693df679a1260a178e2db566eb27",
    3: "d4fb22426b7e32afc19bae6feb08c9ff7905376fd3cfc3378263a958b79b8703",
    4: "4bfa855c871c2e77cd82ffe5afe93bc8c277705a5a9338e859cc33a3b3adae2d",
    5: "3cf296f9641b6a05906db90311d51c95079315b0cc2f6d0822654df7d39e9c4c",
}


def constants_digest(built) -> str:
    h = hashlib.sha256(print_ir(built.module).encode())
    for k in sorted(built.consts):
        h.update(k.encode())
        h.update(np.ascontiguousarray(built.consts[k], dtype="<i8").tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("n", [1, 3, 4, 5])
def test_config_constants_are_unchanged(n):
    spec, tag, _ = models.CONFIGS[n]
    assert models.calib_path(spec, tag).exists(), "no tracked calibration for the current calibration code"
    built, _ = models.config(n)
    assert constants_digest(built) == CONSTANTS_SHA256[n]


@pytest.mark.parametrize("n", [1, 4])
def test_tracked_calibration_equals_a_fresh_one(n):
    """The stored scales are what this code computes from the seeds (here, on this host's float arithmetic)."""
    spec, tag, _ = models.CONFIGS[n]
    body = json.loads(models.calib_path(spec, tag).read_text())
    sin, amax = models.calibrate(spec, models.init_params(spec), tag)
    assert body["key"] == models.calib_key(spec, tag)
    assert body["sin"] == sin and body["amax"] == amax


def _signed_graph(m):
    b = GraphBuilder("signed")
    x = b.input("x", [4, 8], scale=0.03)
    y = b.qlinear("y", x, b.const("w", [8, 16], value=np.full((8, 16), 127)), m, 10, scale=0.05)
    b.output(y)
    return b.module()


def test_negative_multiplier_passes_the_reference_check_but_not_the_sound_one():
    """The reference's proof bounds acc * M + round with M's sign (anvil/frontend/quantize.py:200-205): a large
    negative M passes it, so compile accepts the graph as the reference does; the sound bound (|M|) fails, so the
    model keeps the checked kernels, which raise OverflowError at run time as the interpreter would."""
    acc = 128 * 8 * 127
    m = -((1 << 31) // acc + 5)
    mod = _signed_graph(m)
    Q.prove_no_overflow(mod)
    assert not Q.int32_bounds(mod).ok
    cm = anvil_mi355x.compile(mod)
    assert not cm.proven
    ok = _signed_graph(-(((1 << 31) - 1 - (1 << 9)) // acc))
    assert Q.int32_bounds(ok).ok and anvil_mi355x.compile(ok).proven


def test_batched_const_operand_bounds():
    """A const right operand with a batch dim: the reference sums |w| over its first axis (the batch axis), the sound
    policy over K of each batch entry. With K = 2 and 6 heads the two differ by 3x."""
    b = GraphBuilder("heads")
    x = b.input("x", [6, 4, 2])
    w = b.const("w", [6, 2, 3], value=np.full((6, 2, 3), 100))
    b.output(b.qmatmul("y", x, w, 1, 0))
    mod = b.module()
    y = mod.ops[0].ops[2].result
    assert Q.int32_bounds(mod, reference=True).acc[y] == 128 * 600
    assert Q.int32_bounds(mod).acc[y] == 128 * 200


def test_transposed_const_operand_is_bounded_over_its_contracted_axis():
    """qmatmul(x, transpose(W)) with W (256, 3072): the product contracts W's second axis (K = 3072), so the sound
    bound is 128 * 3072 * 127. Summing the untransposed array's first axis would give 128 * 256 * 127, below 2^23,
    and wrongly admit the 24-bit requant."""
    b = GraphBuilder("tw")
    x = b.input("x", [4, 3072])
    w = b.const("w", [256, 3072], value=np.full((256, 3072), 127))
    wt = b.transpose("wt", w, [1, 0])
    b.output(b.qmatmul("y", x, wt, 1, 24))
    mod = b.module()
    y = mod.ops[0].ops[-2].result
    bounds = Q.int32_bounds(mod)
    assert bounds.acc[y] == 128 * 3072 * 127
    # a column of W^T is a row of W: one loud row of W bounds one column of the product
    v = np.zeros((256, 3072), dtype=np.int64)
    v[7] = 127
    b = GraphBuilder("tw1")
    x = b.input("x", [4, 3072])
    wt = b.transpose("wt", b.const("w", [256, 3072], value=v), [1, 0])
    b.output(b.qmatmul("y", x, wt, 1, 24))
    mod = b.module()
    assert Q.int32_bounds(mod).acc[mod.ops[0].ops[-2].result] == 128 * 3072 * 127


def test_reshaped_const_operand_is_bounded_in_its_new_shape():
    """A const of 12 entries reshaped to (3, 4) and used as the right operand: the sound bound sums each column of
    the (3, 4) array; the largest column of arange(12) so reshaped is 3 + 7 + 11 = 21."""
    b = GraphBuilder("rw")
    x = b.input("x", [5, 3])
    w = b.reshape("w2", b.const("w", [12], value=np.arange(12)), [3, 4])
    b.output(b.qmatmul("y", x, w, 1, 0))
    mod = b.module()
    y = mod.ops[0].ops[-2].result
    assert Q.int32_bounds(mod).acc[y] == 128 * 21
    Q.prove_no_overflow(mod)          # the reference policy still takes the graph as the reference does


def test_choose_shift_matches_a_brute_force_scan():
    """choose_shift equals the first admissible shift of a downward scan over [0, 31 - extra]."""
    rng = np.random.default_rng(11)
    for _ in range(200):
        ratios = list(rng.uniform(1e-6, 4.0, int(rng.integers(1, 4))))
        bounds = [int(v) for v in rng.integers(1, 1 << 26, len(ratios))]
        extra = int(rng.integers(0, 6))
        scan = None
        for s in range(31 - extra, -1, -1):
            mm = [round(r * (1 << s)) for r in ratios]
            if sum(b * v for b, v in zip(bounds, mm)) + ((1 << (s + extra - 1)) if s + extra else 0) < 1 << 31:
                scan = (mm, s)
                break
        if scan is None:
            with pytest.raises(OverflowError):
                Q.choose_shift(ratios, bounds, extra)
        elif min(scan[0]) < 1:
            with pytest.raises(ValueError):
                Q.choose_shift(ratios, bounds, extra)
        else:
            assert Q.choose_shift(ratios, bounds, extra) == scan


def test_wide_row_bound_is_tight_by_brute_force():
    """WideRow.xmax[k][i] is the largest |x| that one entry of a reachable row with (index, steps) = (i, k) can hold:
    checked against every row of 3 entries up to magnitude 40 with c = 2, e = 3 and a 16-entry table."""
    d, n, c, mag, e = 3, 16, 2, 40, 3
    row = Q.WideRow(d, n, c, mag, e)
    seen = {}
    sq = [(x * x + Q.half(c)) >> c for x in range(mag + 1)]
    for a in range(mag + 1):
        for b_ in range(a + 1):
            for c_ in range(b_ + 1):
                i, k = Q.rsqrt_steps(e + sq[a] + sq[b_] + sq[c_], n)
                seen[(k, i)] = max(seen.get((k, i), 0), a)
    for (k, i), x in seen.items():
        assert row.xmax[k][i] >= x                      # never below a reachable row's entry
    # tight where the bucket's largest sum is reachable by a row with one loud entry and quiet others
    assert max(row.xmax) == max(k for k, _ in seen)
    for k, col in row.xmax.items():
        assert col.max() == max(x for (kk, _), x in seen.items() if kk == k)


def test_block_digest_fixture_matches_the_oracle():
    """The committed per-sequence digests (tests/golden/block_digests.json) are the oracle's on the current graphs:
    config 1 in full, and the first and last sequence of config 3."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import make_block_digests as mk
    from oracle import interp
    gold = json.loads((Path(__file__).resolve().parent / "golden" / "block_digests.json").read_text())
    for n, seqs in ((1, [0]), (3, [0, 63])):
        built, cm, xq = mk.config_inputs(n)
        g = gold["configs"][str(n)]
        assert g["constants_sha256"] == CONSTANTS_SHA256[n] and g["batch"] == len(xq)
        syms = mk.graph_values(built)
        assert [s for s, _ in syms] == g["values"]
        for i in seqs:
            r = interp.run(built.module, {"x": xq[i:i + 1]}, built.consts, batch=True, fast=True)
            assert {s: mk.value_digest(r.values[s][0], dt) for s, dt in syms} == g["sequences"][i]
