"""The reference's own program-layer test programs (test/Test/FuryKernel/
ProgramTest.hs, restated in tests/programs.py) lowered and run by the
oracle's CPU target against the f64 evaluator on seeded state: every output
within 1e-4 of the evaluator (relative to its largest magnitude), and the
token an argmax the evaluator decides the same.

- ``layer`` (:488-557, planned as ``layerPlan`` :559-640) and its k = v form:
  per-head RMSNorm in segments of 8 before RoPE in the store and attention
  steps (each norm a launch of its own), an Add and norms between anchors,
  gate/up and the router over different rows (two GEMV launches), a step of
  a linear and a routed anchor, bf16 expert tables, the MoE combine, and a
  closing chain of norms, adds and a ScaleBy;
- ``two_tiles`` (:655-663): an Add of two anchors as its own step;
- ``embed`` (:785-789): a gather scaled by 5.65625, stored;
- ``pooled`` (:1614-1621): three rows of a table summed and divided by 3
  (a repeated row among them), then a linear layer over rows of 4 (packs of
  4 elements, a wavefront a row);
- ``predicting`` (:769-784), planned ungated and gated (``optGated``,
  Plan.hs:246-251: the route's ids a stored step before the routed anchor).

Planted mistakes fail the bar: an Add that subtracts, a gather without its
factor, a route that swaps its ranks' weights."""

import numpy as np
import pytest

from furykernel_amd.lower import ELT_ADD
from furykernel_amd.program.check import check_program
from program_state import State, lowered, output_buffers, rel, widen
import programs as P

CASES = {
    "layer": (lambda: P.layer(False), {"position": [9], "slot": [1]}),
    "layer_kv": (lambda: P.layer(True), {"position": [30], "slot": [0]}),
    "two_tiles": (P.two_tiles, {}),
    "embed": (P.embed_program, {"tokens": [37]}),
    "pooled": (P.pooled, {"rows": [5, 0, 5]}),
    "predicting": (P.predicting, {}),
}


def run(name, gated=False, seed=7, tamper=None):
    make, ints = CASES[name]
    checked = check_program(make())
    low = lowered(checked, gated=gated)
    if tamper is not None:
        tamper(low)
    st = State(checked, seed=seed, ints=ints)
    cpu = st.cpu(low)
    cpu.run()
    return checked, low, st, cpu


def check_outputs(checked, st, read) -> dict:
    """Each output's error against the evaluator (relative to its largest
    magnitude; integers 0 if equal, else 1), and each cache's: the stored
    elements within a step of the cache's type of the evaluator's own
    rounding (bf16: 2^-7 of the cache's largest magnitude)."""
    ev = st.evaluate()
    out = {}
    for name, (t, v) in st.caches.items():
        got = widen(t, read(f"cache:{name}")).astype(np.float64)
        want = np.concatenate([ev.caches[name][s] for s in sorted(ev.caches[name])])
        # in units where one bf16 step (2^-7 relative) is the 1e-4 bar
        out[f"cache:{name}"] = rel(got, want) / 2.0 ** -7 * 1e-4 if t == "bf16" else rel(got, want)
    for o, buf in output_buffers(checked).items():
        got = read(buf)
        want = np.asarray(ev.outputs[o][0], np.float64)
        if checked.program.value(next(x.value for x in checked.program.outputs if x.name == o)).type == "u32":
            out[o] = 0.0 if np.array_equal(got[:want.size], want.astype(np.uint32)) else 1.0
        else:
            out[o] = rel(got[:want.size], want)
    return out


@pytest.mark.parametrize("gated", [False, True], ids=["ungated", "gated"])
@pytest.mark.parametrize("name", sorted(CASES))
def test_reference_program_on_the_cpu_target_within_1e4_of_the_evaluator(name, gated):
    checked, low, st, cpu = run(name, gated)
    errs = check_outputs(checked, st, cpu.read)
    assert errs and max(errs.values()) <= 1e-4, errs


def test_the_layer_lowers_its_norms_adds_and_mixed_anchors_to_launches_of_their_own():
    checked, low, _, _ = run("layer")
    entries = [(L.step, L.entry) for L in low.launches]
    # the per-head norms before RoPE, each its own launch, then the store and attention taking RoPE
    assert ("s1_store:k_normed", "fk_rmsnorm_f32") in entries and ("s2_attend:q_normed", "fk_rmsnorm_f32") in entries
    norm = [L for L in low.launches if L.step == "s1_store:k_normed"][0]
    assert norm.params["seg"] == 8
    # gate/up and the router read different rows: two GEMV launches of one step
    assert sum(1 for s, e in entries if s == "s5_gemv" and e.startswith("fk_step_gemv")) == 2
    # a step of a linear and a routed anchor
    assert {e for s, e in entries if s == "s6_gemv"} == {"fk_step_gemv_bf16_k2048_r1_p0_e0", "fk_gemv_routed_bf16_r1"}
    assert any(e == "fk_step_elementwise" for _, e in entries)


def test_the_gated_plan_stores_the_routes_first():
    checked, low, _, _ = run("predicting", gated=True)
    steps = [(L.step, L.entry) for L in low.launches]
    assert steps[1:3] == [("s1_route_ids:route", "fk_step_route")] * 2
    assert steps[3] == ("s2_gemv", "fk_gemv_routed_bf16_r1")


def test_planted_mistakes_miss_the_bar():
    """An Add that subtracts (two_tiles), a gather without its factor
    (embed), and a route whose ranks' weights are swapped (predicting) each
    miss the evaluator by far more than 1e-4."""
    checked, low, st, cpu = run("two_tiles")
    add = [L for L in low.launches if L.entry == "fk_step_elementwise" and L.params["op"] == ELT_ADD][0]
    cpu.buffers[add.bind["y"]][:] = cpu.read(add.bind["a"]) - cpu.read(add.bind["b"])
    assert rel(cpu.read("value:c"), st.evaluate().outputs["c"][0]) > 1e-3

    def unscaled(low):
        for L in low.launches:
            if L.entry.startswith("fk_step_gather_"):
                L.params["factor"] = 1.0
    checked, low, st, cpu = run("embed", tamper=unscaled)
    assert max(check_outputs(checked, st, cpu.read).values()) > 1e-3

    checked, low, st, cpu = run("predicting")
    ws = [L for L in low.launches if L.entry == "fk_step_route"][0].bind["ws"]
    cpu.buffers[ws][:2] = cpu.buffers[ws][:2][::-1].copy()
    for L in low.launches[[i for i, L in enumerate(low.launches) if L.entry == "fk_step_combine_ranks"][0]:]:
        cpu.run_launch(L)
    assert max(check_outputs(checked, st, cpu.read).values()) > 1e-3
