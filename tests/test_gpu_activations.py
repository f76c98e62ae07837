"""GELU-tanh, the softcap and bf16 weights on the GPU through the C ABI:
the reference's own head program (test/Test/FuryKernel/ProgramTest.hs:
643-652: bf16 weights and gains, softcap 30, the greedy token), a tiny
GELU-tanh decoder with bf16 weights, and two layers of the 1B-class step
with bf16 weights and GELU-tanh: every stored buffer the oracle's CPU
target's, bit for bit (tanh and exp are binary64's rounded once on both
sides, whose libraries may round a value within their error of a binary32
midpoint differently: such elements are held to 1 ulp and to being rare),
and the tiny programs within 1e-4 of the binary64 evaluator."""

import dataclasses

import numpy as np
import pytest

from furykernel_amd.decode import DecodeSession
from furykernel_amd.engine import Engine
from furykernel_amd.lower import lower_plan, rope_table
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import ONE_B, TINY_GELU_BF16
from furykernel_amd.program.plan import PlanOptions, plan
from oracle.eval import Bindings, evaluate
from programs import head_program
from test_activations import exact, gelu_tiny_cpu, gelu_tiny_eval, gelu_tiny_state, head_state, rel, run_cpu, widen

pytestmark = pytest.mark.gpu


def ulps(a, b):
    ia = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def same(g, c):
    """Bit for bit, but for rare 1-ulp differences of a binary64-rounded-once
    transcendental."""
    if g.dtype != np.float32:
        return np.array_equal(g, c)
    u = ulps(g, c)
    return int(u.max(initial=0)) <= 1 and int(np.sum(u > 0)) <= max(1, g.size // 1000)


def load(engine, low, weights, caches=None, inputs=None, ints=None):
    engine.write_weights(weights)
    for name, what in low.constants.items():
        pass  # the engine wrote its constants
    for name, v in (caches or {}).items():
        engine.write(f"cache:{name}", v)
    for name, v in (inputs or {}).items():
        engine.write(f"value:{name}", v)
    for name, v in (ints or {}).items():
        engine.write(f"ints:{name}", np.asarray(v, np.uint32))


def test_the_reference_head_program_on_the_gpu(device, kernels):
    c = check_program(head_program())
    low = lower_plan(c, plan(PlanOptions(), c))
    x, w = head_state()
    eng = Engine(device, kernels, low)
    try:
        load(eng, low, w, inputs={"x": x})
        print("the reference's head program (softcap 30, bf16)", flush=True)
        eng.enqueue()
        device.sync()
        cpu = run_cpu(low, w, {"x": x})
        capped = eng.read("value:capped")
        assert same(capped, cpu.read("value:capped"))
        assert int(eng.read("value:token")[0]) == int(cpu.read("value:token")[0])
        ev = evaluate(c, Bindings(1, inputs={"x": [x.astype(np.float64)]},
                                  weights={k: exact(v) for k, v in w.items()}))
        assert rel(capped, ev.values["capped"][0]) <= 1e-4
    finally:
        eng.close()


@pytest.mark.parametrize("store_gelus", [False, True])
def test_gelu_bf16_tiny_decode_on_the_gpu(device, kernels, store_gelus):
    cprog, w, caches, x, pos = gelu_tiny_state()
    options = PlanOptions(store_gelus=store_gelus)
    low = lower_plan(cprog, plan(options, cprog))
    eng = Engine(device, kernels, low)
    try:
        load(eng, low, w, caches, {"x": x}, {"position": [pos], "slot": [0]})
        print(f"tiny GELU-tanh bf16 decode (store_gelus {store_gelus})", flush=True)
        eng.enqueue()
        device.sync()
        cpu = gelu_tiny_cpu(cprog, w, caches, x, pos, options=options)
        bad = [n for n in low.buffers if not n.startswith(("weight:", "widen:"))
               and not same(eng.read(n), cpu.read(n))]
        assert bad == []
        ev = gelu_tiny_eval(cprog, w, caches, x, pos)
        assert rel(eng.read("value:logits"), ev.outputs["logits"][0]) <= 1e-4
    finally:
        eng.close()


def test_1b_shapes_gelu_bf16_decode_step(device, kernels):
    """Two layers of the 1B-class step with bf16 weights and a GELU-tanh MLP at
    position 4095: every stored buffer the CPU target's."""
    from test_gpu_decode import mirror

    dims = dataclasses.replace(ONE_B, weight_type="bf16", act="gelu_tanh")
    s = DecodeSession(device, kernels, dims, PlanOptions(store_gelus=True), embed=True, layers=2)
    try:
        s.init_synthetic()
        s.set_position(4095, token=123)
        cpu = mirror(s)
        print(f"1B shapes, bf16, GELU-tanh: {len(s.lowered.launches)} launches", flush=True)
        s.step()
        device.sync()
        cpu.run()
        bad = [n for n in s.lowered.buffers if not n.startswith(("weight:", "widen:"))
               and not same(s.engine.read(n), cpu.read(n))]
        assert bad == []
        assert s.token() == int(cpu.read("value:token")[0])
    finally:
        s.close()
