"""Driver host logic without a GPU: input binding and validation (reference anvil/driver.py:248-280), compile checks
(driver.py:119-132), backend dispatch (runtime/api.py:141), and the layout planner's views, strides and batch
folding, executed by a CPU stand-in of the C ABI (tests/fake_device.py) and compared with the oracle."""
import numpy as np
import pytest

import anvil_mi355x
import fake_device
import helpers
from anvil_mi355x import layout, models
from anvil_mi355x import runtime as rt
from anvil_mi355x.ir import GraphBuilder
from oracle import interp


@pytest.fixture
def fake(monkeypatch):
    dev = fake_device.FakeDevice()
    monkeypatch.setattr(rt, "device", lambda index=0: dev)
    return dev


@pytest.fixture(scope="module")
def cfg1():
    return models.config(1)[0]


def test_planner_matches_oracle_on_config1(fake, cfg1):
    cm = anvil_mi355x.compile(cfg1)
    x = models.eval_inputs(cfg1.spec, 3, 5)
    res = cm.run(x, "mi355x", batch=True, keep="all")
    want = interp.run(cfg1.module, {"x": cm.quantize_input(x)}, cfg1.consts, batch=True)
    for k, v in want.values.items():
        if k not in cfg1.consts:
            assert np.array_equal(res.ints[k], v), k
    kinds = [c[0] for c in fake.calls]
    assert kinds.count("copy") == 0                                  # no layout op is materialised
    assert ("gemm_group", 3) in fake.calls                           # q, k and v: one group call
    # both residual adds run in the epilogues of the y and proj GEMMs; keep="all" still stores y and proj
    assert kinds.count("gemm") == 4 and kinds.count("gemm_add") == 2 and kinds.count("add") == 0
    assert all(c[8] for c in fake.calls if c[0] == "gemm_add")
    gemms = [c for c in fake.calls if c[0] == "gemm"]
    assert all(c[1:4] == (1, 1, 96) for c in gemms[:2])              # q, k: batch and T fold into one M = 3 * 32
    assert gemms[2][1:6] == (1, 3, 64, 32, 64)                       # v is computed transposed, per sequence
    # the returned scores and p come from the fused kernel's kept form: no score product, softmax or P.V launch;
    # proven: unchecked (1), score bounds below 2^23 allow the 24-bit requant multiply (2)
    assert kinds.count("softmax") == 0 and kinds.count("attention") == 0
    (att,) = [c for c in fake.calls if c[0] == "attention_keep"]
    assert att[1:5] == (3, 4, 32, 16) and att[6] == 1 | 2


def test_keep_outputs_plan_fuses_attention(fake, cfg1):
    """Scores and p are not returned with keep="outputs": QK^T, softmax and P.V become one fused launch over the
    strided q, k, v^T and head-merged o buffers."""
    cm = anvil_mi355x.compile(cfg1)
    x = models.eval_inputs(cfg1.spec, 2, 6)
    a = cm.run(x, "mi355x", batch=True, keep="outputs")
    kinds = [c[0] for c in fake.calls]
    assert kinds.count("attention") == 1 and kinds.count("softmax") == 0 and kinds.count("gemm") == 4
    assert [c[8] for c in fake.calls if c[0] == "gemm_add"] == [False, False]   # y and proj are not returned
    att = [c for c in fake.calls if c[0] == "attention"][0]
    assert att[1:5] == (2, 4, 32, 16)                                 # batch 2 x 4 heads, T 32, head dim 16
    assert att[5] == (32 * 64, 16, 64, 32 * 64, 16, 64, 64 * 32, 16 * 32, 32, 32 * 64, 16, 64)
    assert "scores" not in a.ints and "p" not in a.ints
    b = cm.run(x, "mi355x", batch=True, keep="all").ints["out"]
    assert np.array_equal(a.ints["out"], b)


def test_unproven_keep_outputs_plan_skips_masked_score_tiles(fake, cfg1):
    """Without the overflow proof the chain is not fused; the scores GEMM still skips tiles no softmax reads."""
    cm = anvil_mi355x.compile((cfg1.module, cfg1.consts), prove=False)
    x = models.eval_inputs(cfg1.spec, 2, 6)
    a = cm.run(x, "mi355x", batch=True, keep="outputs").ints["out"]
    assert "attention" not in [c[0] for c in fake.calls]
    scores = [c for c in fake.calls if c[0] == "gemm"][3]
    assert scores[7] & 2                                              # causal tile skip when scores are not kept
    b = cm.run(x, "mi355x", batch=True, keep="all").ints["out"]
    assert np.array_equal(a, b)


def test_gemm_grouping_is_a_plan_choice(fake, cfg1):
    """Grouped and separate launches give the same results; without grouping every product is its own call."""
    x = models.eval_inputs(cfg1.spec, 2, 7)
    cm = anvil_mi355x.compile(cfg1)
    a = cm.run(x, "mi355x", batch=True, keep="all").ints
    assert [lb for lb, _, _ in cm.plan(2, "all").steps][:2] == ["h1", "q+k+v"]
    n = len(fake.calls)
    cm2 = anvil_mi355x.compile(cfg1)
    cm2.group_gemms = False
    b = cm2.run(x, "mi355x", batch=True, keep="all").ints
    assert not [c for c in fake.calls[n:] if c[0] == "gemm_group"]
    assert a.keys() == b.keys() and all(np.array_equal(a[k], b[k]) for k in a)


def test_dependent_gemms_are_not_grouped(fake):
    """Five qlinears of one input form a group of four and a single; a qlinear that reads another's output starts
    a new run: the members of a group never read or write each other's buffers."""
    g = GraphBuilder("grp")
    x = g.input("x", [8, 16], scale=0.1)
    ys = [g.qlinear(f"y{i}", x, g.const(f"w{i}", [16, 16]), 3, 9, scale=0.1) for i in range(5)]
    z = g.qlinear("z", ys[4], g.const("wz", [16, 16]), 3, 9, scale=0.1)
    u = g.qlinear("u", x, g.const("wu", [16, 16]), 3, 9, scale=0.1)
    g.output(*ys, z, u)
    rng = np.random.default_rng(5)
    consts = {f"w{i}": rng.integers(-20, 20, (16, 16)) for i in range(5)}
    consts.update(wz=rng.integers(-20, 20, (16, 16)), wu=rng.integers(-20, 20, (16, 16)))
    cm = anvil_mi355x.compile((g.module(), consts))
    xq = rng.integers(-128, 128, (8, 16))
    res = cm.run(xq, quantized=True, keep="all")
    assert [lb for lb, _, _ in cm.plan(1, "all").steps] == ["y0+y1+y2+y3", "y4", "z+u"]
    assert [c[1] for c in fake.calls if c[0] == "gemm_group"] == [4, 2]
    want = interp.run(g.module(), {"x": xq}, consts)
    for k in ("y0", "y3", "y4", "z", "u"):
        assert np.array_equal(res.ints[k], want.values[k]), k


@pytest.mark.parametrize("seed", range(12))
def test_planner_matches_oracle_on_random_graphs(fake, seed):
    m, c, x, want = helpers.random_case(seed)
    res = anvil_mi355x.compile((m, c), prove=False).run([x["x"], x["xk"]], quantized=True, keep="all")
    for k, v in want.values.items():
        if k not in c:
            assert np.array_equal(res.ints[k], v), k


def test_unknown_backend(fake, cfg1):
    cm = anvil_mi355x.compile(cfg1)
    with pytest.raises(ValueError, match="unknown backend 'isasim'"):
        cm.run(np.zeros((32, 64)), "isasim")


def test_input_binding_errors(fake, cfg1):
    cm = anvil_mi355x.compile(cfg1)
    with pytest.raises(ValueError, match="shape"):
        cm.run(np.zeros((31, 64)))
    with pytest.raises(ValueError, match="NaN"):
        cm.run(np.full((32, 64), np.nan))
    with pytest.raises(ValueError, match="integer"):
        cm.run(np.zeros((32, 64)), quantized=True)
    with pytest.raises(ValueError, match="outside i8"):
        cm.run(np.full((32, 64), 128), quantized=True)
    with pytest.raises(ValueError, match="inputs for graph inputs"):
        cm.run([np.zeros((32, 64)), np.zeros((32, 64))])
    with pytest.raises(ValueError, match="batched shape"):
        cm.run(np.zeros((32, 64)), batch=True)
    with pytest.raises(ValueError, match="keep"):
        cm.run(np.zeros((32, 64)), keep="some")
    r = cm.run(np.zeros((1, 32, 1, 64)))                                 # extra size-1 dims are accepted
    assert r.ints["out"].shape == (32, 64)
    with pytest.raises(TypeError):
        cm.run(np.zeros((32, 64)), bogus=1)


def test_quantize_input_rounds_half_to_even(fake, cfg1):
    cm = anvil_mi355x.compile(cfg1)
    s = cm.scale("x")
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 1e6, -1e6]) * s
    assert list(cm.quantize_input(x)) == [0, 2, 2, 0, -2, 127, -128]


def test_compile_checks():
    g = GraphBuilder("c")
    x = g.input("x", [2, 4], scale=0.1)
    y = g.qlinear("y", x, g.const("w", [4, 4]), 100, 10, scale=0.1)
    g.output(y)
    m = g.module()
    with pytest.raises(ValueError, match="no values"):
        anvil_mi355x.compile((m, {}))
    with pytest.raises(ValueError, match="name no graph const"):
        anvil_mi355x.compile((m, {"w": np.ones((4, 4), int), "zz": np.ones(3, int)}))
    with pytest.raises(OverflowError):
        anvil_mi355x.compile(_overflowing())
    with pytest.raises(TypeError):
        anvil_mi355x.compile(object())
    with pytest.raises(TypeError):
        anvil_mi355x.compile((m, {"w": np.ones((4, 4), int)}), bogus=1)


def _overflowing():
    g = GraphBuilder("o")
    x = g.input("x", [2, 4], scale=0.1)
    g.output(g.qlinear("y", x, g.const("w", [4, 4]), 1 << 30, 10, scale=0.1))
    return g.module(), {"w": np.full((4, 4), 127)}


def test_device_overflow_raises_like_the_interpreter(fake):
    m, c = _overflowing()
    cm = anvil_mi355x.compile((m, c), prove=False)
    x = np.full((2, 4), 100)
    with pytest.raises(OverflowError):
        interp.run(m, {"x": x}, c)
    with pytest.raises(OverflowError):
        cm.run(x, quantized=True)


def test_nocopy_strides_agree_with_numpy():
    rng = np.random.default_rng(5)
    for _ in range(300):
        dims = tuple(int(d) for d in rng.integers(1, 5, int(rng.integers(1, 5))))
        a = np.arange(int(np.prod(dims))).reshape(dims)
        perm = list(rng.permutation(len(dims)))
        v = np.transpose(a, perm)
        st = tuple(s // a.itemsize for s in v.strides)
        new = list(v.shape)
        rng.shuffle(new)
        if len(new) > 1 and rng.random() < 0.5:
            new = [new[0] * new[1]] + new[2:]
        got = layout.nocopy_strides(v.shape, st, new)
        if got is not None:
            view = np.lib.stride_tricks.as_strided(a, shape=new, strides=[s * a.itemsize for s in got])
            assert np.array_equal(view, v.reshape(new))
        if v.flags.c_contiguous:
            assert got is not None


def test_merge_kblocked_inverts_the_head_split():
    """View.merge_kblocked: the plain (B, T, H, 64) view of K-blocked (B, T, H * 64) storage (the attention output o,
    permuted from (B, H, T, 64)) merges back into the K-blocked view, element for element; views of any other form
    are refused."""
    B, T, H = 3, 5, 4
    kb = B * T * 64
    buf = layout.Buf(B * T * H * 64)
    om = layout.View(buf, "i8", (B, T, H * 64), (T * 64, 64, 1), 0, kb)
    split = om.reshape((B, T, H, 64))
    assert split.kb == 0 and split.strides == (T * 64, 64, kb, 1)
    o = split.permute([0, 2, 1, 3])                      # the attention writes o as (B, H, T, 64)
    back = o.permute([0, 2, 1, 3]).merge_kblocked((B, T, H * 64))
    assert (back.dims, back.strides, back.kb, back.offset) == (om.dims, om.strides, om.kb, om.offset)

    def addr_kb(v, idx):                                 # element address under the K-blocked layout
        *lead, k = idx
        return v.offset + sum(i * s for i, s in zip(lead, v.strides[:-1])) + (k // 64) * v.kb + k % 64

    def addr(v, idx):
        return v.offset + sum(i * s for i, s in zip(idx, v.strides))
    rng = np.random.default_rng(5)
    for _ in range(200):
        b, t, h, d = (int(rng.integers(0, n)) for n in (B, T, H, 64))
        assert addr_kb(back, (b, t, h * 64 + d)) == addr(o, (b, h, t, d))
    assert om.merge_kblocked((B, T, H * 64)) is None                        # already K-blocked
    assert split.merge_kblocked((B, T, H * 32)) is None                     # sizes differ
    half = layout.View(buf, "i8", (B, T, 2 * H, 32), (T * 32, 32, kb // 2, 1))
    assert half.merge_kblocked((B, T, H * 64)) is None                      # blocks of 32
    crossed = split.permute([1, 0, 2, 3])                                   # lead dims that do not fold into (T, B)
    assert crossed.merge_kblocked((T * B, H * 64)) is None


def test_layout_choice_makes_head_merge_free(cfg1):
    cm = anvil_mi355x.driver.CompiledModel(cfg1.module, cfg1.consts)
    phys = {v.owner.sym_str: p for v, p in cm.phys.items()}
    assert phys == {"o": [1, 0, 2], "v": [1, 0]}     # o stored head-merged, v stored transposed for P.V


@pytest.fixture(scope="module")
def cfg4():
    return models.config(4)[0]


def test_token_prelude_matches_the_host_embedding(fake, cfg4):
    """compile() of a token model attaches its tables; run(ids, tokens=True) gathers, adds and quantizes on the
    device and gives the same values as the host's float64 embedding followed by quantize_input."""
    cm = anvil_mi355x.compile(cfg4)
    ids = models.eval_inputs(cfg4.spec, 2, 9)
    a = cm.run(ids, tokens=True, batch=True, keep="all")
    x = models.to_float_input(cfg4.spec, cfg4.params, ids)
    b = cm.run(x, batch=True, keep="all")
    assert a.ints.keys() == b.ints.keys()
    assert all(np.array_equal(a.ints[k], b.ints[k]) for k in a.ints)
    assert np.array_equal(a.ints["x"], cm.quantize_input(x))
    assert [c for c in fake.calls if c[0] == "embed"][0][1:] == (2 * cfg4.spec.seq, cfg4.spec.seq, cfg4.spec.n_embd)
    with pytest.raises(ValueError):
        bad = ids.copy()
        bad[1, 3] = cfg4.spec.vocab
        cm.run(bad, tokens=True, batch=True)
    with pytest.raises(ValueError, match="expected"):
        cm.run(ids, tokens=True)
    with pytest.raises(ValueError, match="integers"):
        cm.run(ids.astype(float), tokens=True, batch=True)


def test_tokens_need_embedding_tables(fake, cfg1):
    cm = anvil_mi355x.compile(cfg1)
    with pytest.raises(ValueError, match="embedding tables"):
        cm.run(np.zeros((1, 32), int), tokens=True, batch=True)
    with pytest.raises(ValueError, match="do not fit"):
        cm.set_embedding(np.zeros((10, 8), np.float32), np.zeros((32, 64), np.float32))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_float_inputs_are_quantized_on_the_device_as_on_the_host(fake, cfg1, dtype):
    cm = anvil_mi355x.compile(cfg1)
    x = models.eval_inputs(cfg1.spec, 3, 12).astype(dtype)
    s = cm.scale("x")
    x[0, 0, :4] = np.array([0.5, 1.5, -2.5, 1e9]) * s                  # ties round to even; saturation
    r = cm.run(x, batch=True, keep="all")
    assert np.array_equal(r.ints["x"], cm.quantize_input(x))
    assert [c for c in fake.calls if c[0] == "quantize"][0][2] == (dtype == np.float64)


def test_wide_frozen_model_selects_the_fast_wide_rmsnorm(fake):
    """The reference's v2 frozen model (i16 residual stream) passes the proof, so its four wide rmsnorm steps run
    UNCHECKED (the wide kernel for int16 rows of 32 entries), with RMS_S24 where every |lut[i] M| < 2^23; results
    equal the oracle's."""
    text, consts, x = helpers.reference_model("v2")
    m = anvil_mi355x.parse_ir(text)
    cm = anvil_mi355x.compile((m, consts))
    assert cm.proven
    xs = np.random.default_rng(5).integers(-32768, 32768, (2, 16, 32))
    res = cm.run(xs, "mi355x", quantized=True, batch=True)
    want = interp.run(m, {"x": xs}, consts, batch=True)
    assert np.array_equal(res.ints["L1.out"], want.values["L1.out"])
    rms = [c for c in fake.calls if c[0] == "rmsnorm"]
    assert len(rms) == 4 and all(c[1:3] == (32, 32) and c[3] & rt.OP_UNCHECKED for c in rms)
    assert all(c[3] & rt.RMS_S24 for c in rms)


@pytest.mark.parametrize("keep", ["outputs", "all"])
def test_wide_frozen_model_fuses_its_i16_residual_adds(fake, keep):
    """The v2 frozen model's four int16 add_requant ops (i16 residual plus the i16 result of down / y) run in the
    epilogue of the GEMM that produces y: no standalone add launch is left, every fused call carries the i16 dtype,
    and every value equals the oracle's."""
    text, consts, x = helpers.reference_model("v2")
    m = anvil_mi355x.parse_ir(text)
    cm = anvil_mi355x.compile((m, consts))
    xs = np.random.default_rng(6).integers(-32768, 32768, (3, 16, 32))
    res = cm.run(xs, "mi355x", quantized=True, batch=True, keep=keep)
    want = interp.run(m, {"x": xs}, consts, batch=True)
    for k, v in res.ints.items():
        assert np.array_equal(v, want.values[k]), k
    kinds = [c[0] for c in fake.calls]
    adds = [c for c in fake.calls if c[0] == "gemm_add"]
    n_add = sum(isinstance(op, anvil_mi355x.ir.AddRequantOp) for op in anvil_mi355x.ir.func_of(m).ops)
    assert n_add == 4
    assert kinds.count("add") == 0 and len(adds) == n_add and all(c[-1] == "i16" for c in adds)
    # the products' own i16 results are stored only when they are returned
    assert all(c[8] == (keep == "all") for c in adds)
    # T = 16: the fused attention reads v's own rows, so v is one plain product grouped with q and k
    att = [c for c in fake.calls if c[0] in ("attention", "attention_keep")]
    assert len(att) == 2 and all(c[3] == 16 and c[-1] & rt.ATTN_V_ROWS for c in att)
    assert kinds.count("gemm_group") == 4 and ("gemm_group", 3) in fake.calls


def test_gemm_operands_are_planned_kblocked(fake, cfg1):
    """keep="outputs" on a proven block: values read only as the left operand of linear products (h1, h2 and the fc
    result) are stored K-blocked by their producers (RMS_OUT_KBLOCK, GEMM_C_KBLOCK) and read K-blocked (A_KBLOCK, or
    B_KBLOCK where the v product runs transposed); every constant weight is read K-blocked. keep="all" plans the same
    layouts and reads the K-blocked values back from their blocks. Results equal the oracle's either way."""
    cm = anvil_mi355x.compile(cfg1)
    x = models.eval_inputs(cfg1.spec, 2, 7)
    want = interp.run(cfg1.module, {"x": cm.quantize_input(x)}, cfg1.consts, batch=True)
    res = cm.run(x, "mi355x", batch=True, keep="outputs")
    assert np.array_equal(res.ints["out"], want.values["out"])
    rms = [c[3] for c in fake.calls if c[0] == "rmsnorm"]
    assert rms == [rt.OP_UNCHECKED | rt.RMS_S24 | rt.RMS_OUT_KBLOCK] * 2
    kb = rt.GEMM_A_KBLOCK | rt.GEMM_B_KBLOCK
    gemm_flags = [c[7] for c in fake.calls if c[0] in ("gemm", "gemm_add")]
    assert all(f & rt.GEMM_B_KBLOCK or f & rt.GEMM_A_KBLOCK for f in gemm_flags)
    assert sum(f & kb == kb for f in gemm_flags) == 5                  # q, k, v, fc, proj
    assert sum(bool(f & rt.GEMM_C_KBLOCK) for f in gemm_flags) == 1     # fc
    fake.calls.clear()
    res = cm.run(x, "mi355x", batch=True, keep="all")
    assert [c[3] for c in fake.calls if c[0] == "rmsnorm"] == rms
    assert sum(bool(c[7] & rt.GEMM_C_KBLOCK) for c in fake.calls if c[0] in ("gemm", "gemm_add")) == 1
    for k, v in want.values.items():
        if k not in cfg1.consts:
            assert np.array_equal(res.ints[k], v), k


def test_attention_inputs_are_planned_head_blocked(fake):
    """Head dim 64: q and k, read only by the fused attention through their split into heads, are written
    head-blocked by their products (GEMM_C_KBLOCK, block = head), and the attention reads each head's rows as one
    contiguous block (q / k strides: sequence T * 64, head B * T * 64, row 64). Its output o, read only by the y
    product through its merge back into rows (om), is written the same way and y reads om K-blocked
    (GEMM_A_KBLOCK, block stride B * T * 64). Results equal the oracle's."""
    spec = models.BlockSpec(n_embd=128, n_head=2, seq=64, calib_batches=2, calib_batch=2)
    built = models.build(spec, 9, stored=False)
    cm = anvil_mi355x.compile(built)
    nb = 3
    x = models.eval_inputs(built.spec, nb, 9)
    res = cm.run(x, "mi355x", batch=True, keep="outputs")
    want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
    assert np.array_equal(res.ints["out"], want.values["out"])
    att = [c for c in fake.calls if c[0] == "attention"][0]
    T = spec.seq
    assert att[1:5] == (nb, 2, T, 64)
    assert att[5][0:3] == (T * 64, nb * T * 64, 64) and att[5][3:6] == (T * 64, nb * T * 64, 64)
    members = [c for c in fake.calls if c[0] == "gemm"][:2]
    assert all(c[7] & rt.GEMM_C_KBLOCK and c[6][8] == nb * T * 64 for c in members)
    assert att[5][9:12] == (T * 64, nb * T * 64, 64)
    y = [c for c in fake.calls if c[0] == "gemm_add"][0]
    assert y[7] & rt.GEMM_A_KBLOCK and y[6][2] == nb * T * 64
    assert "om" in {v.owner.sym_str for v in cm.plan(nb).kb_values}


def test_single_head_attention_output_is_head_blocked(fake):
    """One head of 64: om is o itself, one 64-wide block. The attention batches over the sequences (one head, its
    stride unused) and writes o as T * 64-byte blocks of rows, which the y product reads K-blocked; the output
    equals the oracle's."""
    spec = models.BlockSpec(n_embd=64, n_head=1, seq=64, calib_batches=2, calib_batch=2)
    built = models.build(spec, 12, stored=False)
    cm = anvil_mi355x.compile(built)
    nb = 2
    x = models.eval_inputs(built.spec, nb, 12)
    res = cm.run(x, "mi355x", batch=True, keep="outputs")
    want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
    assert np.array_equal(res.ints["out"], want.values["out"])
    assert "om" in {v.owner.sym_str for v in cm.plan(nb).kb_values}
    att = [c for c in fake.calls if c[0] == "attention"][0]
    T = spec.seq
    assert att[1:5] == (1, nb, T, 64)                             # one head: the sequences are the batch
    assert att[5][9:12] == (0, T * 64, 64)
    y = [c for c in fake.calls if c[0] == "gemm_add"][0]
    assert y[7] & rt.GEMM_A_KBLOCK


def test_kblocked_planning_only_for_values_read_by_linear_products(fake):
    """Of the candidates, only `a` (an rmsnorm-fed linear result read by two linear products and nothing else) is
    stored K-blocked; `h` (also read by an add), `b` (returned) and `c` (read by a lut) stay row-major. Every
    output equals the oracle's."""
    mod = helpers.kblock_graph()
    cm = anvil_mi355x.compile(mod)
    assert cm.proven
    xs = np.random.default_rng(32).integers(-128, 128, (2, 16, 128))
    res = cm.run(xs, "mi355x", quantized=True, batch=True)
    want = interp.run(mod, {"x": xs}, cm.consts, batch=True)
    for k in ("b", "r1", "d", "e"):
        assert np.array_equal(res.ints[k], want.values[k]), k
    assert sorted(v.owner.sym_str for v in cm.plan(2).kb_values) == ["a"]
    rms = [c for c in fake.calls if c[0] == "rmsnorm"]
    assert rms and not rms[0][3] & rt.RMS_OUT_KBLOCK
    gemms = [c[7] for c in fake.calls if c[0] == "gemm"]
    assert sum(bool(f & rt.GEMM_C_KBLOCK) for f in gemms) == 1      # a
    assert sum(bool(f & rt.GEMM_A_KBLOCK) for f in gemms) == 2      # c and d read a K-blocked
    assert all(f & rt.GEMM_B_KBLOCK for f in gemms)             # every weight


def test_read_back_reuses_page_locked_buffers(fake):
    """cm.run downloads into the plan's page-locked host buffers (one per read-back device buffer, allocated once)
    and returns new arrays: a second run leaves the first run's ints and dequantized outputs as they were, and both
    equal the oracle's."""
    spec = models.BlockSpec(n_embd=64, n_head=1, seq=32, calib_batches=2, calib_batch=2)
    built = models.build(spec, 14, stored=False)
    cm = anvil_mi355x.compile(built)
    xa, xb = models.eval_inputs(built.spec, 2, 14, 0), models.eval_inputs(built.spec, 2, 14, 1)
    ra = cm.run(xa, "mi355x", batch=True)
    kept = {k: v.copy() for k, v in ra.ints.items()}, ra.output.copy()
    allocs = fake.host_allocs
    rb = cm.run(xb, "mi355x", batch=True)
    assert fake.host_allocs == allocs == 2                        # x and out, reused by the second run
    assert all(np.array_equal(ra.ints[k], v) for k, v in kept[0].items()) and np.array_equal(ra.output, kept[1])
    for x, r in ((xa, ra), (xb, rb)):
        want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
        assert np.array_equal(r.ints["out"], want.values["out"]) and np.array_equal(r.ints["x"], want.values["x"])
        assert np.array_equal(r.output, want.values["out"] * cm.scale("out"))
    assert not np.array_equal(ra.ints["out"], rb.ints["out"])


def test_page_locked_read_back_is_capped_per_plan(fake, monkeypatch):
    """With the plan's page-locked budget below the two read-back buffers (x and out), only the first gets a
    page-locked buffer; the second downloads into ordinary memory, and both still equal the oracle."""
    from anvil_mi355x import driver
    spec = models.BlockSpec(n_embd=64, n_head=1, seq=32, calib_batches=2, calib_batch=2)
    built = models.build(spec, 14, stored=False)
    cm = anvil_mi355x.compile(built)
    monkeypatch.setattr(driver, "PINNED_PLAN_MAX", 2 * 32 * 64 + 100)
    before = getattr(fake, "host_allocs", 0)
    x = models.eval_inputs(built.spec, 2, 14, 0)
    for _ in range(2):
        r = cm.run(x, "mi355x", batch=True)
        want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
        assert np.array_equal(r.ints["out"], want.values["out"]) and np.array_equal(r.ints["x"], want.values["x"])
    assert fake.host_allocs - before == 1
    assert sum(h.nbytes for h in cm.plan(2).host_stage.values()) <= driver.PINNED_PLAN_MAX


def test_graph_runs_replay_the_captured_steps(fake):
    """run(..., graph=True): the plan's steps run once and are captured on the first such run, then every run
    replays the capture over the freshly uploaded input; each result equals the oracle's, as an ordinary run's does."""
    spec = models.BlockSpec(n_embd=64, n_head=2, seq=32, calib_batches=2, calib_batch=2)
    built = models.build(spec, 15, stored=False)
    cm = anvil_mi355x.compile(built)
    for j in range(3):
        x = models.eval_inputs(built.spec, 2, 15, j)
        res = cm.run(x, "mi355x", batch=True, graph=True)
        want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
        assert np.array_equal(res.ints["out"], want.values["out"])
        eager = cm.run(x, "mi355x", batch=True, graph=False)
        assert np.array_equal(eager.ints["out"], res.ints["out"])
    plan = cm.plan(2)
    assert fake.captures == 1 and plan.graph.launches == 3


@pytest.mark.parametrize("graph_faster", [True, False])
def test_default_run_keeps_the_faster_launch(fake, monkeypatch, graph_faster):
    """run() without graph=: a plan's first two runs launch eagerly (timed on the device), the third captures the
    steps as a HIP graph, the fourth replays it (timed); later runs take whichever was faster. Every run's result
    equals the oracle's."""
    spec = models.BlockSpec(n_embd=64, n_head=2, seq=32, calib_batches=2, calib_batch=2)
    built = models.build(spec, 15, stored=False)
    cm = anvil_mi355x.compile(built)
    # device time of a run: 1.0 ms eager; a replay 0.5 ms or 2.0 ms
    monkeypatch.setattr(fake, "elapsed_ms", lambda a, b: (0.5 if graph_faster else 2.0) if fake._graph_run else 1.0)
    launches = []
    for j in range(6):
        plan = cm.plan(2)
        fake._graph_run = plan.graph is not None
        x = models.eval_inputs(built.spec, 2, 15, j)
        res = cm.run(x, "mi355x", batch=True)
        launches.append(res.result["hip_graph"])
        want = interp.run(built.module, {"x": cm.quantize_input(x)}, built.consts, batch=True)
        assert np.array_equal(res.ints["out"], want.values["out"])
    assert launches[:4] == [False, False, True, True]
    assert launches[4:] == [graph_faster] * 2
    assert cm.plan(2).replay is graph_faster and fake.captures == 1


@pytest.mark.parametrize("n", [1, 3, 4, 5])
@pytest.mark.parametrize("keep", ["outputs", "all"])
def test_gemm_operand_ranges_stay_inside_their_allocations(monkeypatch, n, keep):
    """Every GEMM the planner launches for the configs (two sequences each, both keep modes) has operands whose
    buffer-resource range -- base of the first row up to the last row's K-th byte, or the last K block of a K-blocked
    operand -- lies inside one allocation. The kernels read stages past K anywhere in that range (so a head's slice
    of q may be read into the next head's columns), which is only safe inside the operand's own buffer; the stand-in
    device asserts it on every call."""
    dev = fake_device.FakeDevice(heap_bytes=1 << 30, fast=True)
    monkeypatch.setattr(rt, "device", lambda index=0: dev)
    built, _ = models.config(n)
    cm = anvil_mi355x.compile(built)
    x = models.eval_inputs(built.spec, 2, models.config_tag(n))
    if built.spec.vocab:
        res = cm.run(x, "mi355x", batch=True, keep=keep, tokens=True)
    else:
        res = cm.run(x, "mi355x", batch=True, keep=keep)
    assert res.ints and any(c[0] in ("gemm", "gemm_add", "gemm_group") for c in dev.calls)


@pytest.mark.parametrize("keep", ["outputs", "all"])
def test_rmsnorm_after_a_fused_add_joins_its_epilogue(fake, cfg4, keep):
    """At C = 128 (config 4) each block's h2 = rmsnorm(r1), the second layer's h1 and the final norm hf run in the
    epilogue of the GEMM whose residual add makes their input (anvil_gemm_i8_add_norm): four such launches and one
    stand-alone rmsnorm (the first h1, whose input comes from outside). Every value against the oracle. At C = 256
    (config 3) the planner leaves the rmsnorm on its own."""
    cm = anvil_mi355x.compile(cfg4)
    x = models.eval_inputs(cfg4.spec, 2, 11)
    xf = models.to_float_input(cfg4.spec, cfg4.params, x)
    xq = cm.quantize_input(xf)
    fake.calls.clear()
    res = cm.run(xq, quantized=True, batch=True, keep=keep)
    kinds = [c[0] for c in fake.calls]
    assert kinds.count("gemm_add_norm") == 4 and kinds.count("rmsnorm") == 1, kinds
    assert all(c[1] % 128 == 0 and c[2] == 128 for c in fake.calls if c[0] == "gemm_add_norm")
    want = interp.run(cfg4.module, {"x": xq}, cfg4.consts, batch=True)
    names = want.values.keys() if keep == "all" else res.ints.keys()
    for k in names:
        if k in cfg4.consts:
            continue
        assert np.array_equal(res.ints[k], want.values[k]), k
    cm3 = anvil_mi355x.compile(models.config(3)[0])
    cm3._ensure_device()
    assert not any(lab.endswith("+h2") for lab, _, _ in cm3._plan(2, "outputs").steps)
