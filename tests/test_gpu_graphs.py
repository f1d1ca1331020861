"""GPU parity per graph: every value of every block config and of seeded random graphs, bit-exact against the oracle.

The driver runs the whole graph on the device (values resident in HBM, layout ops as views) and reads back every
value (keep="all"). Configs 1, 3 and 4 are checked on their full batch; config 5 (B=32, T=1024, C=768) runs its
full batch on the GPU and is checked on sampled sequences, which is exact because batched evaluation equals
per-sample evaluation (reference tests/interp/test_graph_interp.py:61-73).
"""
import numpy as np
import pytest

import anvil_mi355x
import helpers
from anvil_mi355x import models
from oracle import interp

pytestmark = pytest.mark.gpu


def _check_all(got: dict, want: dict, consts):
    bad = [k for k, v in want.items() if k not in consts and not np.array_equal(got[k], v)]
    missing = [k for k in want if k not in consts and k not in got]
    assert not bad and not missing, (bad, missing)


@pytest.mark.parametrize("seed", range(24))
def test_random_graphs(seed):
    m, c, x, want = helpers.random_case(seed)
    cm = anvil_mi355x.compile((m, c), prove=False)
    res = cm.run([x["x"], x["xk"]], "mi355x", quantized=True, keep="all")
    _check_all(res.ints, want.values, c)
    assert len(res.outputs) == 2 and np.array_equal(res.ints["out"], want.values["out"])


def test_random_graphs_batched():
    m, c, x, _ = helpers.random_case(3)
    rng = np.random.default_rng(77)
    for _ in range(50):                      # inputs the oracle accepts (the draw was checked on its own inputs)
        xs = rng.integers(-128, 128, (5, *x["x"].shape))
        xks = rng.integers(-128, 128, (5, *x["xk"].shape))
        try:
            want = interp.run(m, {"x": xs, "xk": xks}, c, batch=True)
            break
        except (OverflowError, ValueError, ZeroDivisionError):
            continue
    res = anvil_mi355x.compile((m, c), prove=False).run([xs, xks], "mi355x", quantized=True, keep="all", batch=True)
    _check_all(res.ints, want.values, c)


def _config_case(n, batch=None, sample=None):
    built, nb = models.config(n)
    nb = batch or nb
    cm = anvil_mi355x.compile(built)
    raw = models.eval_inputs(built.spec, nb, models.config_tag(n))
    x = models.to_float_input(built.spec, built.params, raw)
    res = cm.run(x, "mi355x", batch=True, keep="all")
    xq = cm.quantize_input(x)
    idx = range(nb) if sample is None else sample
    for i in idx:
        want = interp.run(built.module, {"x": xq[i:i + 1]}, built.consts, batch=True, fast=True)
        _check_all({k: v[i:i + 1] for k, v in res.ints.items()}, want.values, built.consts)
    return cm, built, res


def test_config1_block():
    cm, built, res = _config_case(1, batch=8)
    assert res.stray_writes() == []
    # single-sample run (no batch dim) equals the batched run's first row
    x = models.to_float_input(built.spec, built.params, models.eval_inputs(built.spec, 8, models.config_tag(1)))
    one = cm.run(x[0], "mi355x", keep="all")
    for k in one.ints:
        assert np.array_equal(one.ints[k], res.ints[k][0]), k


def test_config3_block():
    _config_case(3, sample=[0, 31, 63])


def test_config4_two_layer_model():
    _config_case(4, sample=[0, 64, 127])


def test_config5_gpt2_small_block():
    _config_case(5, sample=[0, 31])


@pytest.mark.parametrize("n,sample", [(3, [0, 63]), (5, [7])])
def test_keep_outputs_fast_path_matches_oracle(n, sample):
    """keep="outputs" plans skip masked score tiles and bound P.V's K loop: the outputs stay bit-exact."""
    built, nb = models.config(n)
    cm = anvil_mi355x.compile(built)
    x = models.to_float_input(built.spec, built.params, models.eval_inputs(built.spec, nb, 1234))
    res = cm.run(x, "mi355x", batch=True)
    xq = cm.quantize_input(x)
    for i in sample:
        want = interp.run(built.module, {"x": xq[i:i + 1]}, built.consts, batch=True, fast=True)
        for s in cm.outputs:
            assert np.array_equal(res.ints[s][i:i + 1], want.values[s]), (n, i, s)


def test_keep_outputs_equals_keep_all_and_runs_repeat():
    built, _ = models.config(1)
    cm = anvil_mi355x.compile(built)
    x = models.eval_inputs(built.spec, 4, 99)
    a = cm.run(x, "mi355x", batch=True, keep="all")
    b = cm.run(x, "mi355x", batch=True)
    c = cm.run(x, "mi355x", batch=True)
    assert set(b.ints) == {"x", "out"}
    assert np.array_equal(a.ints["out"], b.ints["out"]) and np.array_equal(b.ints["out"], c.ints["out"])
    assert np.allclose(b.output, b.ints["out"] * built.scales["out"])


@pytest.mark.parametrize("name", ["v1", "v2"])
@pytest.mark.parametrize("keep", ["all", "outputs"])
def test_reference_frozen_model(name, keep):
    """The reference's frozen 2-layer model files, loaded from their printed IR: v2 (i16 residual stream, wide
    rmsnorm) on its held-out input and on seeded inputs of the full i16 range, v1 (int8) on seeded int8 inputs."""
    text, consts, x = helpers.reference_model(name)
    m = anvil_mi355x.parse_ir(text)
    cm = anvil_mi355x.compile((m, consts))
    rng = np.random.default_rng(11)
    lo, hi = (-32768, 32768) if name == "v2" else (-128, 128)
    xs = rng.integers(lo, hi, (6, 16, 32))
    if x is not None:
        xs[0] = x
    want = interp.run(m, {"x": xs}, consts, batch=True)
    res = cm.run(xs, "mi355x", quantized=True, batch=True, keep=keep)
    if keep == "all":
        _check_all(res.ints, want.values, consts)
    assert np.array_equal(res.ints["L1.out"], want.values["L1.out"])


def test_config4_from_token_ids():
    """The two-layer token model run from its token ids: the embedding gather, add and quantization run on the
    device, bit-exact with the host's float64 embedding and the oracle; an id past the vocabulary is a ValueError."""
    built, nb = models.config(4)
    cm = anvil_mi355x.compile(built)
    ids = models.eval_inputs(built.spec, nb, models.config_tag(4))
    res = cm.run(ids, "mi355x", tokens=True, batch=True, keep="all")
    x = models.to_float_input(built.spec, built.params, ids)
    xq = cm.quantize_input(x)
    assert np.array_equal(res.ints["x"], xq)
    for i in (0, nb - 1):
        want = interp.run(built.module, {"x": xq[i:i + 1]}, built.consts, batch=True, fast=True)
        _check_all({k: v[i:i + 1] for k, v in res.ints.items()}, want.values, built.consts)
    bad = ids.copy()
    bad[-1, -1] = built.spec.vocab
    with pytest.raises(ValueError):
        cm.run(bad, "mi355x", tokens=True, batch=True)
    again = cm.run(ids, "mi355x", tokens=True, batch=True)          # the context is usable after the error
    assert np.array_equal(again.ints[cm.outputs[0]], res.ints[cm.outputs[0]])


def test_kblocked_intermediates_on_the_device():
    """A graph where one linear result is read only by two linear products (stored K-blocked: the GEMM writes it with
    C_KBLOCK, its readers take it with A_KBLOCK) beside candidates that stay row-major (an rmsnorm output also read
    by an add, a returned result, a result read by a lut): every output equals the oracle's."""
    mod = helpers.kblock_graph()
    cm = anvil_mi355x.compile(mod)
    xs = np.random.default_rng(33).integers(-128, 128, (5, 16, 128))
    res = cm.run(xs, "mi355x", quantized=True, batch=True)
    want = interp.run(mod, {"x": xs}, cm.consts, batch=True)
    assert sorted(v.owner.sym_str for v in cm.plan(5).kb_values) == ["a"]
    for k in ("b", "r1", "d", "e"):
        assert np.array_equal(res.ints[k], want.values[k]), k


@pytest.mark.parametrize("n_embd,n_head,seq", [(64, 1, 96), (128, 2, 64), (256, 4, 128)])
def test_head_blocked_attention_blocks(n_embd, n_head, seq):
    """Blocks with head dim 64 and one, two or four heads, keep="outputs": q, k and the attention output o are
    head-blocked (o written into the K-blocked storage the y product reads, om planned K-blocked), and the output
    equals the oracle's for every sequence of the batch."""
    spec = models.BlockSpec(n_embd=n_embd, n_head=n_head, seq=seq, calib_batches=2, calib_batch=2)
    built = models.build(spec, 11, stored=False)
    cm = anvil_mi355x.compile(built)
    nb = 3
    x = models.eval_inputs(built.spec, nb, 11)
    res = cm.run(x, "mi355x", batch=True, keep="outputs")
    want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
    assert "om" in {v.owner.sym_str for v in cm.plan(nb).kb_values}
    assert np.array_equal(res.ints[cm.outputs[0]], want.values[cm.outputs[0]])




def test_nonfinite_input_is_refused_before_the_forward():
    """A float input with a NaN raises the reference's ValueError (anvil/driver.py:265-266), found by the device
    quantization; the next run on a finite input is unaffected and equals the oracle."""
    built, _ = models.config(1)
    cm = anvil_mi355x.compile(built)
    x = models.eval_inputs(built.spec, 2, 1)
    bad = x.copy()
    bad[1, 5, 9] = np.nan
    with pytest.raises(ValueError, match="input 'x' has NaN or infinite values"):
        cm.run(bad, "mi355x", batch=True)
    res = cm.run(x, "mi355x", batch=True)
    want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
    assert np.array_equal(res.ints["out"], want.values["out"])


@pytest.mark.parametrize("n", [1, 4, 5])
def test_hip_graph_replays_equal_ordinary_runs(n):
    """run(..., graph=True) replays the forward as one captured HIP graph. Three replays, each on a new input and
    each followed by an ordinary run of the same input (device synchronisations between them), equal those runs in
    every returned value; config 4 goes through its token prelude."""
    built, nb = models.config(n)
    cm = anvil_mi355x.compile(built)
    nb = min(nb, 4)
    tokens = bool(built.spec.vocab)
    for j in range(3):
        print(f"config {n}, graph replay {j}", flush=True)
        x = models.eval_inputs(built.spec, nb, n, j)
        g = cm.run(x, "mi355x", batch=True, graph=True, tokens=tokens)
        e = cm.run(x, "mi355x", batch=True, tokens=tokens)
        assert sorted(g.ints) == sorted(e.ints)
        for k, v in e.ints.items():
            assert np.array_equal(g.ints[k], v), (j, k)
    assert cm.plan(nb).graph is not None


def _workspace_sums(dev) -> int:
    import ctypes as C
    out = C.c_longlong(-1)
    dev.lib.call("anvil_workspace_sums", dev.ctx, C.byref(out))
    return int(out.value)


def split_k_graph_case():
    """The body of the split-K graph test, run in a child process whose context plans split-K products."""
    from anvil_mi355x import quantize as Q
    from anvil_mi355x.ir import GraphBuilder
    from oracle import semantics as sem

    rng = np.random.default_rng(2024)
    T, K, N = 128, 2048, 256
    w = rng.integers(-128, 128, (K, N))
    # about six standard deviations of a random int8 accumulator (sqrt(K) * 128^2 / 3) map to 127
    (m,), s = Q.choose_shift([127 / (6 * K ** 0.5 * 128 ** 2 / 3)], [128 * int(np.abs(w).sum(axis=0).max())])
    b = GraphBuilder("splitk_graph")
    x = b.input("x", [T, K])
    b.output(b.qlinear("y", x, b.const("w", [K, N]), m, s))
    cm = anvil_mi355x.compile((b.module(), {"w": w}))
    assert cm.proven

    def check(nb, graph):
        xs = rng.integers(-128, 128, (nb, T, K))
        got = cm.run(xs, "mi355x", quantized=True, batch=True, graph=graph).ints["y"]
        want = sem.qmatmul(xs, w, m, s, fast=True)
        assert np.array_equal(got, want), (nb, graph, int((got != want).sum()))

    check(1, True)                         # eager run, capture, first replay
    small = _workspace_sums(cm.dev)
    assert small > 0, "the one-sequence product did not split K"
    check(32, False)
    assert _workspace_sums(cm.dev) > small, "the 32-sequence product did not grow the workspace"
    for _ in range(3):
        check(1, True)                     # replays of the graph captured before the growth
    assert cm.plan(1).graph is not None


@pytest.mark.timeout(300)
def test_hip_graph_of_a_split_k_plan_survives_a_larger_workspace():
    """A one-sequence plan of a long-K, few-tile qlinear splits K into the context's workspace, and its captured HIP
    graph records that workspace's address. A 32-sequence run of the same graph then needs a larger workspace (64
    tiles of 128 x 128 instead of 1), which replaces the buffer. Replays of the first graph afterwards still write
    correct outputs: the outgrown buffer is kept alive for graphs that hold it (every output against the oracle).

    By default such few-tile products take the one-launch small-product kernel, which needs no workspace; the case
    runs in a child process whose context is created with the benchmarking override ANVIL_GEMM_CFG set to a value no
    product takes, which turns that kernel off and leaves the split-K rule in force."""
    import os
    import subprocess
    import sys

    child = "import test_gpu_graphs as t; t.split_k_graph_case(); print('split-K graph case ok')"
    env = dict(os.environ, ANVIL_GEMM_CFG="99",
               PYTHONPATH=os.pathsep.join(str(p) for p in (helpers.ROOT / "anvil-compiler_amd", helpers.ROOT,
                                                           helpers.ROOT / "tests")))
    print("split-K graph child: T 128, K 2048, N 256, 1 and 32 sequences, ANVIL_GEMM_CFG=99", flush=True)
    out = subprocess.run([sys.executable, "-c", child], capture_output=True, text=True, timeout=280, env=env)
    assert out.returncode == 0, (out.stdout[-2000:], out.stderr[-2000:])
    assert "split-K graph case ok" in out.stdout
