"""The tiny decode with its token's embedding row gathered and scaled by
5.65625, the reference embedding program's factor (ProgramTest.hs:785-789):
the layer-0 QKV step's prologue gathers the row times the factor
(Eval.hs:528-535) and the attention output's residual epilogue adds the same
scaled row.  On the oracle's CPU target (widths 64 and 32), within 1e-4 of
the f64 evaluator; a CPU target whose gathers drop the factor misses it by
far more, so the factor is pinned where it enters (the GEMV prologue and
the gathered residual)."""

import numpy as np
import pytest

from furykernel_amd.kernels import EPI_ADD_GATHER, PRO_GATHER_RMSNORM
from furykernel_amd.lower import lower_plan, rope_table
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import TINY_EMBED, decoder_step
from furykernel_amd.program.plan import PlanOptions, plan
from oracle.cpu_target import CpuTarget
from oracle.eval import Bindings, evaluate

TOKEN, POSITION = 201, 19


def embed_state(seed=2026, dims=TINY_EMBED):
    checked = check_program(decoder_step(dims, embed=True))
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
            caches[src.name] = (rng.standard_normal(lay.kv_heads * lay.length * lay.head_dim) * 0.02).astype(np.float16)
    return checked, weights, caches


def run_cpu(checked, weights, caches, width=64, options=PlanOptions(), tamper=None):
    low = lower_plan(checked, plan(options, checked))
    if tamper is not None:
        tamper(low)
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
    cpu.write("ints:position", [POSITION])
    cpu.write("ints:slot", [0])
    cpu.write("ints:tokens", [TOKEN])
    cpu.run()
    return cpu


def run_eval(checked, weights, caches):
    return evaluate(checked, Bindings(
        1, weights={k: v.astype(np.float64) for k, v in weights.items()},
        row_ints={"position": [[POSITION]], "slot": [[0]], "tokens": [[TOKEN]]},
        caches={k: {0: v.astype(np.float64)} for k, v in caches.items()}))


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_the_factor_reaches_the_gathering_launches():
    checked, _, _ = embed_state()
    low = lower_plan(checked, plan(PlanOptions(), checked))
    gathering = [L for L in low.launches if L.params.get("pro_mode") == PRO_GATHER_RMSNORM
                 or L.params.get("epi_mode") == EPI_ADD_GATHER]
    assert len(gathering) == 2, [L.entry for L in low.launches]
    assert all(L.params["gfactor"] == 5.65625 for L in gathering)


@pytest.mark.parametrize("width", [64, 32])
@pytest.mark.parametrize("store_gelus", [False, True])
def test_embed_decode_within_1e4_of_the_f64_evaluator(width, store_gelus):
    checked, w, c = embed_state()
    ev = run_eval(checked, w, c)
    np.testing.assert_array_equal(ev.values["x0"][0], w["embed"].reshape(256, 64)[TOKEN].astype(np.float64) * 5.65625)
    cpu = run_cpu(checked, w, c, width, PlanOptions(store_gelus=store_gelus))
    assert rel(cpu.read("value:logits"), ev.outputs["logits"][0]) <= 1e-4
    assert int(cpu.read("value:token")[0]) == int(ev.outputs["token"][0][0])


def test_a_dropped_gather_factor_is_caught():
    """The check has teeth: the CPU target with its gathers' factor planted
    as 1 (prologue and residual both) misses the evaluator by far more
    than 1e-4, as does one with only the residual's factor dropped."""
    checked, w, c = embed_state()
    ev = run_eval(checked, w, c)

    def drop(which):
        def tamper(low):
            for L in low.launches:
                if L.params.get("pro_mode") == PRO_GATHER_RMSNORM and "pro" in which:
                    L.params["gfactor"] = 1.0
                if L.params.get("epi_mode") == EPI_ADD_GATHER and "epi" in which:
                    L.params["gfactor"] = 1.0
        return tamper

    for which in (("pro", "epi"), ("epi",)):
        bad = run_cpu(checked, w, c, tamper=drop(which)).read("value:logits")
        assert rel(bad, ev.outputs["logits"][0]) > 1e-3, which
