"""GELU-tanh, the softcap and bf16 weights on the CPU: the oracle's binary32
restatements against the evaluator's contract bounds (src/FuryKernel/
Program/Eval.hs:36-73, geluBounds :797-807, the softcap's :384-390), and the
reference's own head program (test/Test/FuryKernel/ProgramTest.hs:643-652:
bf16 weights, softcap 30 on the logits, the greedy token) and a GELU-tanh
decoder with bf16 weights lowered and run by the oracle's CPU target within
1e-4 of the binary64 evaluator.  Planted mistakes show the checks see a
dropped cubic term and a dropped cap."""

import dataclasses
import math

import numpy as np
import pytest

from furykernel_amd.lower import EPI_SOFTCAP, lower_plan, rope_table
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import TINY_GELU_BF16, decoder_step
from furykernel_amd.program.graph import GELU_TANH
from furykernel_amd.program.plan import PlanOptions, plan
from oracle import bounds as B
from oracle import fkref
from oracle.cpu_target import CpuTarget
from oracle.eval import Bindings, evaluate, gelu
from programs import head_program

RNG = np.random.default_rng(41)


def f32(x):
    return float(np.float32(x))


def samples(n=4000):
    xs = np.concatenate([RNG.standard_normal(n) * 3, RNG.uniform(-12, 12, n), [0.0, -0.0, 1e-30, -1e-30, 5.5, -5.5]])
    return [f32(x) for x in xs]


def test_tanh_is_binary64s_rounded_once():
    L = fkref.lib()
    for x in samples():
        assert L.fkref_tanh(x) == f32(math.tanh(x))


def test_gelu_tanh_within_its_contract_bound():
    L = fkref.lib()
    for x in samples():
        got = L.fkref_gelu_tanh(x)
        want = gelu(GELU_TANH, x)
        bound = B.gelu_a(GELU_TANH, B.exact_a(x)).bound
        assert abs(got - want) <= bound, (x, got, want, bound)


def test_gelu_without_its_cubic_term_is_caught():
    """0.5 a (1 + tanh(c0 a)) misses the bound wherever the cubic matters."""
    missed = 0
    for x in samples(500):
        wrong = f32(0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * x)))
        if abs(wrong - gelu(GELU_TANH, x)) > B.gelu_a(GELU_TANH, B.exact_a(x)).bound:
            missed += 1
    assert missed > 100


@pytest.mark.parametrize("cap", [30.0, 1.0, 0.25])
def test_softcap_within_its_contract_bound(cap):
    L = fkref.lib()
    for x in samples():
        x = x * cap
        got = L.fkref_softcap(f32(x), cap)
        want = cap * math.tanh(f32(x) / cap)
        a = B.product_a([B.const_a(cap), B.monotone_a(5, math.tanh, B.product_a([B.exact_a(f32(x)),
                                                                                 B.const_a(1 / cap)]))])
        assert abs(got - want) <= a.bound, (x, got, want, a.bound)


def test_act_mul_forms():
    L = fkref.lib()
    a = RNG.standard_normal(300).astype(np.float32) * 3
    b = RNG.standard_normal(300).astype(np.float32)
    for act, form in ((0, "silu"), (1, GELU_TANH)):
        y = np.zeros(300, np.float32)
        assert L.fkref_act_mul(a.ctypes.data, b.ctypes.data, y.ctypes.data, 300, act) == 0
        for i in range(300):
            want = gelu(form, float(a[i])) * float(b[i])
            bound = B.product_a([B.gelu_a(form, B.exact_a(float(a[i]))), B.exact_a(float(b[i]))]).bound
            assert abs(float(y[i]) - want) <= bound
    assert L.fkref_act_mul(a.ctypes.data, b.ctypes.data, y.ctypes.data, 300, 7) != 0


def bf16_bits(x):
    """Round-to-nearest-even bf16 bits of f32 values."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def widen(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def head_state(seed=5):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(32)).astype(np.float32)
    w = {"final_norm": bf16_bits(1 + 0.1 * rng.standard_normal(32)),
         "embed": bf16_bits(rng.standard_normal((64, 32)) * 2.0)}
    return x, w


def run_cpu(low, weights, inputs, width=64, ints=()):
    cpu = CpuTarget(low, width)
    for name, w in weights.items():
        if f"weight:{name}" in low.buffers:
            cpu.write(f"weight:{name}", w)
        if f"widen:{name}" in low.buffers:
            cpu.write(f"widen:{name}", widen(w))
    for name, what in low.constants.items():
        if what[0] == "rope":
            cpu.write(name, rope_table(*what[1:]))
        elif what[0] == "ones":
            cpu.write(name, np.ones(low.buffers[name].count, np.float32))
    for name, v in inputs.items():
        cpu.write(f"value:{name}", v)
    for name, v in ints:
        cpu.write(f"ints:{name}", v)
    cpu.run()
    return cpu


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_the_reference_head_program_lowers_to_a_softcap_epilogue_and_the_token():
    c = check_program(head_program())
    low = lower_plan(c, plan(PlanOptions(), c))
    entries = [L.entry for L in low.launches]
    assert entries == ["fk_step_gemv_bf16_k2048_r1_p1_e5", "fk_step_token"]
    g = low.launches[0]
    assert g.params["epi_mode"] == EPI_SOFTCAP and g.params["cap"] == 30.0 and g.params["arg_slots"] == g.groups
    assert g.bind["gamma"] == "widen:final_norm" and low.layouts["widen:final_norm"] == ("widen", ("final_norm",))


def test_the_reference_head_program_on_the_cpu_target_within_1e4_of_the_evaluator():
    c = check_program(head_program())
    low = lower_plan(c, plan(PlanOptions(), c))
    x, w = head_state()
    cpu = run_cpu(low, w, {"x": x})
    ev = evaluate(c, Bindings(1, inputs={"x": [x.astype(np.float64)]},
                              weights={k: widen(v).astype(np.float64) for k, v in w.items()}))
    capped = cpu.read("value:capped")
    want = np.array(ev.values["capped"][0])
    assert rel(capped, want) <= 1e-4
    assert np.max(np.abs(want)) > 10  # the cap bends these logits
    assert int(cpu.read("value:token")[0]) == int(np.argmax(capped)) == int(ev.outputs["token"][0][0])
    # the check has teeth for the cap: the uncapped logits are far outside the bar
    assert rel(np.array(ev.values["logits"][0]), capped) > 1e-2


def gelu_tiny_state(seed=2026, position=20):
    c = check_program(decoder_step(TINY_GELU_BF16, embed=False))
    rng = np.random.default_rng(seed)
    weights, caches = {}, {}
    for src in c.program.sources:
        kind = type(src.kind).__name__
        if kind == "SWeight":
            dims = src.kind.dims
            v = 1 + 0.1 * rng.standard_normal(dims[0]) if len(dims) == 1 else 0.05 * rng.standard_normal(dims)
            weights[src.name] = bf16_bits(v) if src.kind.type == "bf16" else v.astype(np.float32)
        elif kind == "SCache":
            lay = src.kind.layout
            caches[src.name] = (rng.standard_normal(lay.kv_heads * lay.length * lay.head_dim) * 0.5).astype(np.float16)
    x = (rng.standard_normal(TINY_GELU_BF16.d_model) * 0.5).astype(np.float32)
    return c, weights, caches, x, position


def gelu_tiny_cpu(c, weights, caches, x, position, width=64, options=PlanOptions()):
    low = lower_plan(c, plan(options, c))
    cpu = CpuTarget(low, width)
    for name, w in weights.items():
        if f"weight:{name}" in low.buffers:
            cpu.write(f"weight:{name}", w)
        if f"widen:{name}" in low.buffers:
            cpu.write(f"widen:{name}", widen(w))
    for name, cv in caches.items():
        cpu.write(f"cache:{name}", cv)
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


def exact(v):
    return widen(v).astype(np.float64) if v.dtype == np.uint16 else v.astype(np.float64)


def gelu_tiny_eval(c, weights, caches, x, position):
    return evaluate(c, Bindings(1, inputs={"x": [x.astype(np.float64)]},
                                weights={k: exact(v) for k, v in weights.items()},
                                row_ints={"position": [[position]], "slot": [[0]]},
                                caches={k: {0: v.astype(np.float64)} for k, v in caches.items()}))


@pytest.mark.parametrize("store_gelus", [False, True])
def test_gelu_bf16_decoder_lowers_and_runs_within_1e4_of_the_evaluator(store_gelus):
    c, w, caches, x, pos = gelu_tiny_state()
    low = lower_plan(c, plan(PlanOptions(store_gelus=store_gelus), c))
    acts = [L for L in low.launches if L.params.get("act") == 1]
    assert acts and all("bf16" in L.entry for L in low.launches if L.entry.startswith("fk_step_gemv"))
    cpu = gelu_tiny_cpu(c, w, caches, x, pos, options=PlanOptions(store_gelus=store_gelus))
    ev = gelu_tiny_eval(c, w, caches, x, pos)
    assert rel(cpu.read("value:logits"), ev.outputs["logits"][0]) <= 1e-4


def test_a_silu_evaluator_misses_the_gelu_decoder():
    """The check has teeth for the activation: the same weights evaluated
    with SiLU in place of GELU-tanh are far from the target."""
    c, w, caches, x, pos = gelu_tiny_state()
    cpu = gelu_tiny_cpu(c, w, caches, x, pos)
    silu = check_program(decoder_step(dataclasses.replace(TINY_GELU_BF16, act="silu"), embed=False))
    ev = gelu_tiny_eval(silu, w, caches, x, pos)
    assert rel(cpu.read("value:logits"), ev.outputs["logits"][0]) > 1e-3
