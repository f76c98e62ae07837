"""The f64 program evaluator (oracle/eval.py): pinned by the reference's
evaluator known answers (test/Test/FuryKernel/ProgramTest.hs:1066-1106) and by
closed forms; then the tiny f32 decode step, as the target's kernels compute it
(the oracle's CPU target, bit for bit what the GPU computes), against it.

Bars (the north star's): the f32 step within 1e-4 of the f64 evaluator; the
gfx950 order (SIMD width 64) within 1e-5 of the reference CPU target's order
(width 32).  Relative to the largest magnitude of the row, since logits pass
through zero.
"""

import dataclasses
import math

import numpy as np
import pytest

from furykernel_amd.kernels import PRO_COMBINE
from furykernel_amd.lower import lower_plan, rope_table
from furykernel_amd.program.build import program
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import TINY, TINY_GQA, decoder_step
from furykernel_amd.program.graph import AttnSpec, F32, Ring, RopeSpec, Shape, whole_row
from furykernel_amd.program.plan import PlanOptions, plan
from oracle import fkref
from oracle.cpu_target import CpuTarget
from oracle.eval import Bindings, EvalError, evaluate, round_bf16, rotate

TINY32 = dataclasses.replace(TINY, context=32)


def test_eval_small_known_answer():
    """ProgramTest.hs:1066-1083: y = (1, 3), mean square 5, normed by
    (5 + eps)^-1/2, softcapped at 30."""
    def body(b):
        x = b.input("x", whole_row(2), F32)
        w = b.weight("w", [2, 2])
        y = b.linear("y", w, 0, x)
        n = b.rmsnorm("n", 1e-6, None, 1, y)
        c = b.softcap("c", 30, n)
        b.output("c", c)

    ev = evaluate(check_program(program("small", body)),
                  Bindings(1, inputs={"x": [[1, 2]]}, weights={"w": [1, 0, 1, 1]}))
    s = (5 + 1e-6) ** -0.5
    assert np.array_equal(ev.outputs["c"][0], [30 * math.tanh(1 * s / 30), 30 * math.tanh(3 * s / 30)])


def attention_program(kv_shape=Shape(2, 2)):
    def body(b):
        q = b.input("q", Shape(4, 2), F32)
        pos = b.row_ints("position", 1, 4)
        slot = b.row_ints("slot", 1, 1)
        k = b.cache("k", Ring(1, 1, 4, 2))
        v = b.cache("v", Ring(1, 1, 4, 2))
        kv = b.input("kv", kv_shape, F32)
        b.kv_store("store_k", k, pos, slot, kv)
        b.kv_store("store_v", v, pos, slot, kv)
        o = b.attend("o", AttnSpec(2, 1, 2, None, 1), q, k, v, pos, slot)
        b.output("o", o)

    return program("attention", body)


def test_eval_attention_known_answer():
    """ProgramTest.hs:1085-1106: one position stored (rounded to the cache's
    bf16) and attended: every query head reads back the stored values."""
    ev = evaluate(check_program(attention_program()),
                  Bindings(1, inputs={"q": [[1, 2, 3, 4]], "kv": [[0.1, 0.2]]},
                           row_ints={"position": [[0]], "slot": [[0]]},
                           caches={"k": {0: [0.0] * 8}, "v": {0: [0.0] * 8}}))
    stored = [float(fkref.widen_bf16(fkref.narrow_bf16(0.1))), float(fkref.widen_bf16(fkref.narrow_bf16(0.2)))]
    assert ev.outputs["o"][0].tolist() == stored + stored


def test_eval_refuses_what_the_reference_refuses():
    with pytest.raises(EvalError):  # a position not below its bound
        evaluate(check_program(attention_program()),
                 Bindings(1, inputs={"q": [[1, 2, 3, 4]], "kv": [[0.1, 0.2]]},
                          row_ints={"position": [[4]], "slot": [[0]]},
                          caches={"k": {0: [0.0] * 8}, "v": {0: [0.0] * 8}}))
    with pytest.raises(EvalError):  # a missing weight
        evaluate(check_program(decoder_step(TINY, embed=False, layers=1)), Bindings(1))


def test_round_bf16_ties_to_even_and_agrees_with_narrowing():
    """roundBF16 (Eval.hs:669-684): the midpoint 1 + 2^-8 goes to the even 1
    (ProgramTest.hs:1124-1126); on binary32 values it is narrowBF16."""
    assert round_bf16(1 + 2.0**-8) == 1.0
    assert round_bf16(1 + 3 * 2.0**-8) == 1 + 2.0**-6
    rng = np.random.default_rng(3)
    for x in rng.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** rng.integers(-40, 38, 2000):
        want = float(fkref.widen_bf16(fkref.narrow_bf16(float(x))))
        assert round_bf16(float(x)) == want or (math.isinf(want) and math.isinf(round_bf16(float(x))))


def test_rotation_closed_forms():
    """RoPE at position 0 is the identity; a rotation keeps each pair's norm;
    pairs past `rotated` stay."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal(16)
    assert np.array_equal(rotate(10000.0, 8, 16, 0.0, x), x)
    y = rotate(10000.0, 6, 16, 7.0, x)
    for i in range(6):
        assert math.isclose(x[i] ** 2 + x[i + 8] ** 2, y[i] ** 2 + y[i + 8] ** 2, rel_tol=1e-12)
    assert np.array_equal(y[6:8], x[6:8]) and np.array_equal(y[14:16], x[14:16])
    # pair 0 turns by the position itself (frequency 1)
    assert math.isclose(y[0], x[0] * math.cos(7) - x[8] * math.sin(7), rel_tol=1e-12)


# The tiny decode step -------------------------------------------------------

def tiny_state(seed=2026, position=16, dims=None):
    """The tiny configuration: weights, caches and the input row N(0, 0.02)
    from one seed (norm gains 1), caches rounded to their f16, at a position
    whose ring holds 16 earlier tokens."""
    dims = TINY32 if dims is None else dims
    checked = check_program(decoder_step(dims, embed=False))
    rng = np.random.default_rng(seed)
    weights, caches = {}, {}
    for src in checked.program.sources:
        kind = type(src.kind).__name__
        if kind == "SWeight":
            n = int(np.prod(src.kind.dims))
            weights[src.name] = np.ones(n, np.float32) if len(src.kind.dims) == 1 else \
                (rng.standard_normal(n) * 0.02).astype(np.float32)
        elif kind == "SCache":
            lay = src.kind.layout
            n = lay.kv_heads * lay.length * lay.head_dim
            caches[src.name] = (rng.standard_normal(n) * 0.02).astype(np.float16)
    x = (rng.standard_normal(dims.d_model) * 0.02).astype(np.float32)
    return checked, weights, caches, x, position


def run_cpu_target(checked, weights, caches, x, position, width, options=PlanOptions(), wide=False):
    low = lower_plan(checked, plan(options, checked), wide=wide)
    cpu = CpuTarget(low, width)
    for name, w in weights.items():
        if f"weight:{name}" in low.buffers:
            cpu.write(f"weight:{name}", w)
    for name, c in caches.items():
        cpu.write(f"cache:{name}", c)
    for name, what in low.constants.items():
        if what[0] == "rope":
            cpu.write(name, rope_table(*what[1:]))
        elif what[0] == "ones":
            cpu.write(name, np.ones(low.buffers[name].count, np.float32))
    cpu.write("value:x", x)
    cpu.write("ints:position", [position])
    cpu.write("ints:slot", [0])
    cpu.run()
    return cpu


def run_evaluator(checked, weights, caches, x, position):
    return evaluate(checked, Bindings(
        1, inputs={"x": [x.astype(np.float64)]},
        weights={k: v.astype(np.float64) for k, v in weights.items()},
        row_ints={"position": [[position]], "slot": [[0]]},
        caches={k: {0: v.astype(np.float64)} for k, v in caches.items()}))


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("store_gelus", [False, True])
@pytest.mark.parametrize("position", [16, 31])
def test_tiny_decode_within_1e4_of_the_f64_evaluator(store_gelus, position):
    checked, w, c, x, _ = tiny_state(position=position)
    ev = run_evaluator(checked, w, c, x, position)
    cpu = run_cpu_target(checked, w, c, x, position, 64, PlanOptions(store_gelus=store_gelus))
    logits = cpu.read("value:logits")
    assert rel(logits, ev.outputs["logits"][0]) <= 1e-4
    # the caches' new rows: the f64 value rounded once to f16, or an f16
    # neighbour of it (the kernels round their binary32 value)
    for layer in range(TINY32.layers):
        for kv in ("k", "v"):
            name = f"l{layer}_{kv}_cache"
            got = cpu.read(f"cache:{name}").astype(np.float64)
            want = ev.caches[name][0]
            assert np.max(np.abs(got - want)) <= 2.0**-10 * np.max(np.abs(want))


def test_tiny_decode_width_64_within_1e5_of_width_32():
    """The gfx950 order (width 64) against the reference CPU target's (width
    32): the same f32 arithmetic summed in other orders."""
    checked, w, c, x, position = tiny_state()
    a = run_cpu_target(checked, w, c, x, position, 64).read("value:logits")
    b = run_cpu_target(checked, w, c, x, position, 32).read("value:logits")
    assert rel(a, b) <= 1e-5


def test_a_dropped_rope_term_is_caught():
    """The check has teeth: an evaluator whose RoPE forgets the partner term
    is far more than 1e-4 from the target."""
    import oracle.eval as E

    checked, w, c, x, position = tiny_state()
    cpu = run_cpu_target(checked, w, c, x, position, 64).read("value:logits")
    good = E.rotate

    def broken(theta, rotated, d, pos, xs):
        out = good(theta, rotated, d, pos, xs)
        half = d // 2
        for j in range(min(rotated, half)):
            t = pos * theta ** (-(2 * j) / d)
            out[j] = xs[j] * math.cos(t)
        return out

    E.rotate = broken
    try:
        bad = run_evaluator(checked, w, c, x, position).outputs["logits"][0]
    finally:
        E.rotate = good
    assert rel(cpu, bad) > 1e-3


@pytest.mark.parametrize("position", [130, 255])
@pytest.mark.parametrize("wide", [False, True], ids=["narrow", "wide"])
def test_tiny_gqa_decode_in_splits_within_1e4_of_the_f64_evaluator(position, wide):
    """Grouped queries (4 heads over 2 kv heads) over a ring of 256, at
    positions whose attention runs in splits (two of 128, or four wide
    splits of 64) combined in the O GEMV step's prologue: the CPU target's
    logits within 1e-4 of the f64 evaluator, and its new cache rows within
    f16 rounding."""
    checked, w, c, x, _ = tiny_state(position=position, dims=TINY_GQA)
    cpu = run_cpu_target(checked, w, c, x, position, 64, wide=wide)
    entry, splits = ("fk_step_attend_wide", 4) if wide else ("fk_step_attend", 2)
    attend = [L for L in cpu.lowered.launches if L.entry == entry]
    assert attend and all(L.params["splits"] == splits and L.params["heads"] // L.params["kv_heads"] == 2
                          for L in attend)
    combined = [L for L in cpu.lowered.launches if L.params.get("pro_mode") == PRO_COMBINE]
    assert len(combined) == TINY_GQA.layers
    ev = run_evaluator(checked, w, c, x, position)
    assert rel(cpu.read("value:logits"), ev.outputs["logits"][0]) <= 1e-4
    for layer in range(TINY_GQA.layers):
        for kv in ("k", "v"):
            name = f"l{layer}_{kv}_cache"
            got = cpu.read(f"cache:{name}").astype(np.float64)
            want = ev.caches[name][0]
            assert np.max(np.abs(got - want)) <= 2.0**-10 * np.max(np.abs(want))


@pytest.mark.parametrize("wide", [False, True], ids=["narrow", "wide"])
def test_tiny_gqa_with_a_split_dropped_is_caught(wide):
    """The check has teeth for the combine: the CPU target run with its
    combines (the combine launches, or the O GEMV steps' combine prologues)
    told of one split fewer (the last split's positions left out) misses the
    evaluator by far more than 1e-4."""
    checked, w, c, x, position = tiny_state(position=255, dims=TINY_GQA)
    good = run_cpu_target(checked, w, c, x, position, 64, wide=wide)
    low = good.lowered
    for L in low.launches:
        if L.entry == "fk_step_combine" or L.params.get("pro_mode") == PRO_COMBINE:
            L.params["splits"] -= 1
    bad = CpuTarget(low, 64)
    for name in low.buffers:
        if not name.startswith(("partials:", "value:")) or name == "value:x":
            bad.buffers[name][:] = good.buffers[name]
    bad.write("value:x", x)
    for name in c:
        bad.write(f"cache:{name}", c[name])
    bad.run()
    ev = run_evaluator(checked, w, c, x, position)
    assert rel(good.read("value:logits"), ev.outputs["logits"][0]) <= 1e-4
    assert rel(bad.read("value:logits"), ev.outputs["logits"][0]) > 1e-3
