"""Pin the oracle to the known answers the reference's own tests hold for this path, and to its error contract.

Each test names the reference test it restates. None of them can run against the reference here (they import the
absent xf submodule), so the answers are checked against this repo's oracle and the product's quantize recipe.
"""
import numpy as np
import pytest

from anvil_mi355x import quantize as Q
from anvil_mi355x.ir import GraphBuilder
from oracle import interp
from oracle import semantics as sem

I16 = (-(1 << 15), (1 << 15) - 1)
RNG = np.random.default_rng(9)


def test_round_term_and_checked_int32():
    """tests/interp/test_semantics.py:48-62."""
    assert sem.round_term(0) == 0 and sem.round_term(5) == 16
    with pytest.raises(OverflowError):
        sem.requant([1 << 30], 4, 3)
    with pytest.raises(ValueError):
        sem.check_i8([128])
    with pytest.raises(ValueError):
        sem.round_term(32)
    with pytest.raises(OverflowError):
        sem.check_i32([1 << 31])


def test_requant_dtype_clamps_at_int16():
    """tests/lower/test_wide_residual.py:35-41: (-5 + 8) >> 4 = 0, the i16 clamps, an i16 operand out of range."""
    acc = np.array([-(1 << 30), -5, 0, 5, 1 << 30])
    assert list(sem.requant_dtype(acc, 1, 4, "i16")) == [I16[0], 0, 0, 0, I16[1]]
    a = np.array([I16[1], I16[0]])
    assert list(sem.add_requant(a, np.array([127, -128]), 1 << 14, 1 << 20, 14, "i16")) == [I16[1], I16[0]]
    with pytest.raises(ValueError):
        sem.add_requant(np.array([1 << 15]), np.array([0]), 1, 1, 0, "i16")


def test_add_requant_i16_operands_saturate_at_i8():
    """tests/frontend/test_quantize.py:108-112 (audit B1, mutant B11)."""
    a, b = np.array([30000, -30000, 200, -129, 5]), np.zeros(5, dtype=np.int64)
    assert list(sem.add_requant(a, b, 1, 1, 0, "i8")) == [127, -128, 127, -128, 5]


def test_wide_semantics_reduce_to_int8_forms():
    """tests/lower/test_wide_residual.py:24-33."""
    T, D = 4, 32
    x = RNG.integers(-128, 128, (5, T, D))
    w = RNG.integers(-128, 128, D)
    lut, s = Q.rsqrt_table(0.03, 0.01, 0.02, int(np.abs(w).max()), D, 1e-6)
    assert np.array_equal(sem.rmsnorm_wide(x, w, lut, 1, s), sem.rmsnorm_int(x, w, lut, 1, s))
    assert np.array_equal(sem.rmsnorm_wide(x, w, lut, 1, s, 0, 0, "i16"), sem.rmsnorm_int(x, w, lut, 1, s))
    a, b = RNG.integers(-128, 128, (2, 50))
    assert np.array_equal(sem.add_requant(a, b, 300, 500, 10), sem.residual_add(a, b, 300, 500, 10))
    assert np.array_equal(sem.requant_dtype(a * 1000, 7, 3, "i8"), sem.requant(a * 1000, 7, 3))


def _linear_graph(m, s, w=127):
    g = GraphBuilder("crafted")
    x = g.input("x", [4, 8], scale=0.03)
    y = g.qlinear("y", x, g.const("w", [8, 16], value=np.full((8, 16), w)), m, s, scale=0.05)
    g.output(y)
    return g.module()


def test_crafted_overflow_known_answer():
    """tests/frontend/test_quantize.py:82-95: acc <= 128 * 8 * 127; the largest safe M at s = 10 passes the proof and
    the interpreter, one more fails both on the all -128 input."""
    acc = 128 * 8 * 127
    m_ok = ((1 << 31) - 1 - (1 << 9)) // acc
    x = np.full((4, 8), -128)
    assert Q.prove_no_overflow(_linear_graph(m_ok, 10))["y"] == acc * m_ok + (1 << 9)
    interp.run(_linear_graph(m_ok, 10), {"x": x})
    with pytest.raises(OverflowError, match=r"y: requant numerator can reach"):
        Q.prove_no_overflow(_linear_graph(m_ok + 1, 10))
    with pytest.raises(OverflowError):
        interp.run(_linear_graph(m_ok + 1, 10), {"x": x})


def test_overflow_proof_names_every_bad_op():
    """tests/frontend/test_quantize.py:98-107."""
    g = GraphBuilder("crafted")
    x = g.input("x", [4, 8], scale=0.03)
    a = g.add_requant("res", x, x, 1 << 24, 1 << 24, 0, scale=0.05)
    sc = g.qmatmul("scores", a, g.transpose("aT", a, [1, 0]), 1 << 20, 3, scale=0.1)
    g.output(sc)
    with pytest.raises(OverflowError) as e:
        Q.prove_no_overflow(g.module())
    assert "res:" in str(e.value) and "scores:" in str(e.value)


def test_overflow_proof_wide_chain():
    """tests/frontend/test_quantize.py:~120-130: an i16 add chain overflows, the same chain at int8 magnitudes is
    provably safe."""
    b = GraphBuilder("p")
    x = b.input("x", [2, 4], "i16", 1.0)
    r = b.add_requant("r", x, x, 1, 1, 1, 1.0, dtype="i16")
    b.output(b.add_requant("r2", r, r, 1 << 15, 1 << 15, 16, 1.0, dtype="i16"))
    with pytest.raises(OverflowError):
        Q.prove_no_overflow(b.module(), {})
    b = GraphBuilder("p")
    x = b.input("x", [2, 4], "i8", 1.0)
    r = b.add_requant("r", x, x, 1, 1, 1, 1.0, dtype="i8")
    b.output(b.add_requant("r2", r, r, 1 << 15, 1 << 15, 16, 1.0, dtype="i16"))
    Q.prove_no_overflow(b.module(), {})


def test_choose_shift_known_answers():
    """tests/frontend/test_quantize.py:36-42."""
    with pytest.raises(OverflowError):
        Q.choose_shift([1.0], [1 << 31])
    with pytest.raises(ValueError):
        Q.choose_shift([1e-12, 1.0], [1 << 24, 1 << 24])
    (m,), s = Q.choose_shift([0.37], [1 << 20], top=12)
    assert s == 12 and m == round(0.37 * 4096)


def test_choose_shift_is_the_largest_admissible_shift():
    """The defining property (quantize.py:40-56): the chosen s admits its multipliers, s + 1 does not."""
    rng = np.random.default_rng(3)
    for _ in range(300):
        ms = list(rng.uniform(1e-5, 3.0, int(rng.integers(1, 4))))
        bounds = [int(b) for b in rng.integers(0, 1 << 24, len(ms))]
        k = int(rng.integers(0, 5))
        try:
            mi, s = Q.choose_shift(ms, bounds, k)
        except (ValueError, OverflowError):
            continue

        def fits(s_):
            m_ = [round(m * (1 << s_)) for m in ms]
            return sum(b * m for b, m in zip(bounds, m_)) + ((1 << (s_ + k - 1)) if s_ + k else 0) <= (1 << 31) - 1

        assert fits(s) and mi == [round(m * (1 << s)) for m in ms]
        assert s == 31 - k or not fits(s + 1)


def test_loudest_row_steps_and_exp_shift():
    """loudest_row_steps(8) for 8 entries of magnitude 128: 8 * 2^14 = 2^17 needs 4 shifts by 2 to drop below 1024;
    exp_shift is the largest E keeping (one + t//2) << E and t << E in int32 (quantize.py:155-157)."""
    assert Q.loudest_row_steps(8) == 4
    for t in range(1, 2049, 7):
        e = Q.exp_shift(t)
        ok = lambda e_: ((127 + t // 2) << e_) <= (1 << 31) - 1 and (t << e_) <= (1 << 31) - 1   # noqa: E731
        assert ok(e) and not ok(e + 1)


def test_planted_oracle_mistakes_are_caught(monkeypatch):
    """A dropped rounding term or a truncating (instead of flooring) shift in the oracle breaks the known answers
    above: the pins are sharp enough to catch those mistakes."""
    acc = np.array([-(1 << 30), -5, 0, 5, 1 << 30])
    monkeypatch.setattr(sem, "round_term", lambda s: 0)
    assert list(sem.requant_dtype(acc, 1, 4, "i16")) != [I16[0], 0, 0, 0, I16[1]]
    monkeypatch.undo()
    # the shift floors (arithmetic >>): (-17 + 8) >> 4 = -1, where a truncating division would give 0
    assert int(sem.requant_dtype(np.array([-17]), 1, 4, "i16")[0]) == -1
    assert int(np.trunc((-17 + 8) / 16)) == 0
