"""The evaluator's concatenation, RoPE of several axes and standardization,
pinned by the reference's known answers (test/Test/FuryKernel/ProgramTest.hs):

- ``evalConcat`` (:1511-1527): a concatenation's row is the first's then the
  second's, and a linear layer over it reads both;
- ``evalAxialRope`` (:1587-1611): a head of 8 in two parts of 4, part a
  turned by the row's a-th position as a head of 4 (pairs (0, 2) and (1, 3),
  angles p and p / 100);
- ``evalStandardize`` (:1638-1653): (f x_j - bias_j) scale_j;
- the gate's refusals beside them (:474-477): two axes over one position, a
  bias that is not a row wide, a factor that is not finite.

Each answer is checked against the exact evaluator and the vectorised one,
and the evaluator's bounds hold the same arithmetic done in binary32.
"""

import math

import numpy as np
import pytest

from furykernel_amd.program.build import program
from furykernel_amd.program.check import ProgramRefused, check_program, findings_of
from furykernel_amd.program.graph import RopeSpec, Shape, whole_row
from oracle import bounds as B
from oracle.eval import Bindings, evaluate, evaluate_fast


def joined_program():
    def body(b):
        x = b.input("x", whole_row(2))
        y = b.input("y", whole_row(2))
        w = b.weight("w", [1, 4])
        j = b.concatenate("joined", x, y)
        z = b.linear("z", w, 0, j)
        b.output("joined", j)
        b.output("z", z)
    return program("joined", body)


def axial_program(width):
    def body(b):
        x = b.input("x", Shape(8, 8))
        pos = b.row_ints("position", width, 64)
        b.output("turned", b.rope("turned", RopeSpec(10000.0, 2, 2), pos, x))
    return program("axial", body)


def standardized_program(width, factor=2.0):
    def body(b):
        x = b.input("x", whole_row(2))
        bias = b.weight("bias", [width])
        scale = b.weight("scale", [2])
        b.output("y", b.standardize("y", bias, scale, factor, x))
    return program("standardized", body)


@pytest.mark.parametrize("ev", [evaluate, evaluate_fast], ids=["exact", "fast"])
def test_a_concatenations_row_is_the_first_then_the_second(ev):
    b = Bindings(2, inputs={"x": [[1, 2], [3, 4]], "y": [[5, 6], [7, 8]]}, weights={"w": [1, 10, 100, 1000]})
    out = ev(check_program(joined_program()), b).outputs
    assert np.array_equal(np.asarray(out["joined"], np.float64), [[1, 2, 5, 6], [3, 4, 7, 8]])
    assert np.array_equal(np.asarray(out["z"], np.float64), [[6521], [8743]])


def turn(at, xs):
    """ProgramTest.hs:1601-1607: a part of 4, pairs (0, 2) and (1, 3) turned by p and p / 100."""
    a, c, e, g = xs
    s0, c0 = math.sin(at), math.cos(at)
    s1, c1 = math.sin(at / 100), math.cos(at / 100)
    return [a * c0 - e * s0, c * c1 - g * s1, e * c0 + a * s0, g * c1 + c * s1]


@pytest.mark.parametrize("ev", [evaluate, evaluate_fast], ids=["exact", "fast"])
def test_a_rotary_embedding_of_two_axes_turns_each_part_by_its_own_position(ev):
    x = [1, 2, 3, 4, 5, 6, 7, 8]
    b = Bindings(2, inputs={"x": [x, x]}, row_ints={"position": [[3, 0], [0, 5]]})
    got = np.asarray(ev(check_program(axial_program(2)), b).outputs["turned"], np.float64)
    want = np.array([turn(3, x[:4]) + x[4:], x[:4] + turn(5, x[4:])])
    assert np.max(np.abs(got - want)) < 1e-12
    # a dropped axis (both parts by the first position) is caught
    assert np.max(np.abs(got[1] - np.array(x[:4] + turn(0, x[4:])))) > 1


@pytest.mark.parametrize("ev", [evaluate, evaluate_fast], ids=["exact", "fast"])
def test_standardizing_scales_subtracts_the_bias_and_scales_again(ev):
    b = Bindings(2, inputs={"x": [[1, 2], [3, 4]]}, weights={"bias": [1, 1], "scale": [2, 3]})
    got = ev(check_program(standardized_program(2)), b).outputs["y"]
    assert np.array_equal(np.asarray(got, np.float64), [[2, 9], [10, 21]])


def test_the_gate_refuses_two_axes_over_one_position_and_weights_not_a_row_wide():
    with pytest.raises(ProgramRefused):
        check_program(axial_program(1))
    with pytest.raises(ProgramRefused):
        check_program(standardized_program(3))
    fs = findings_of(standardized_program(2, math.inf))
    assert [(f.rule, f.message) for f in fs] == [("Shapes", "y: its factor isn't finite.")], fs


def test_the_bounds_hold_the_binary32_arithmetic_of_standardize_and_axial_rope():
    """The bounds of each output hold the same arithmetic in binary32 (the
    operands rounded to it first): (f x - bias) scale, and each part's turn
    with binary32 sines and cosines."""
    rng = np.random.default_rng(11)
    xs = rng.standard_normal((1, 2))
    bias, scale = rng.standard_normal(2), rng.standard_normal(2)
    checked = check_program(standardized_program(2, 1.5))
    b = Bindings(1, inputs={"x": xs.tolist()}, weights={"bias": bias.tolist(), "scale": scale.tolist()})
    ev = evaluate(checked, b)
    bd = B.evaluate_bounds(checked, b, ev)
    f32 = np.float32
    y32 = (f32(1.5) * xs.astype(f32) - bias.astype(f32)) * scale.astype(f32)
    exact = np.asarray(ev.outputs["y"], np.float64)[0]
    assert np.all(np.abs(y32[0].astype(np.float64) - exact) <= np.asarray(bd.values["y"][0]))

    x = rng.standard_normal(8)
    pos = [37, 11]
    checked = check_program(axial_program(2))
    b = Bindings(1, inputs={"x": [x.tolist()]}, row_ints={"position": [pos]})
    ev = evaluate(checked, b)
    bd = np.asarray(B.evaluate_bounds(checked, b, ev).values["turned"][0])
    exact = np.asarray(ev.outputs["turned"], np.float64)[0]
    x32 = x.astype(f32)
    got = []
    for a in range(2):
        p = x32[4 * a:4 * a + 4]
        for j in range(4):
            i = j % 2
            t = f32(pos[a]) * f32(math.pow(10000.0, -(2 * i) / 4))
            c, s = f32(math.cos(t)), f32(math.sin(t))
            got.append(p[j] * c - p[j + 2] * s if j < 2 else p[j] * c + p[j - 2] * s)
    assert np.all(np.abs(np.asarray(got, np.float64) - exact) <= bd)
    assert np.all(bd > 0) and np.all(np.isfinite(bd))
