"""Routed experts on the CPU: the evaluator's Route, LinearRouted and
CombineRanks (Eval.hs:291-321,391-414) pinned by the reference's evalRoute
known answer (test/Test/FuryKernel/ProgramTest.hs:1500-1509) and closed
forms; the oracle's route against the evaluator's; and the lowered MoE step
(route, routed GEMVs, the gated GELU, the combine and its residual) run by
the oracle's CPU target within 1e-4 of the binary64 evaluator."""

import math

import numpy as np
import pytest

from furykernel_amd.program.build import program
from furykernel_amd.program.check import check_program
from furykernel_amd.program.graph import F32, Shape, whole_row
from moe_cases import CASES, case_id, lowered, moe_program, run_cpu, state
from oracle import fkref
from oracle.eval import Bindings, EvalError, evaluate


def routing(n, k, scaled=False):
    def body(b):
        x = b.input("x", whole_row(n), F32)
        s = b.weight("s", [n], F32) if scaled else None
        ids, ws = b.route("r", k, s, x)
        b.output("ids", ids)
        b.output("ws", ws)
    return check_program(program("routing", body))


def test_eval_route_known_answer():
    e = evaluate(routing(4, 2), Bindings(1, inputs={"x": [[1, 3, 3, 2]]}))
    assert e.outputs["ids"][0].tolist() == [1, 2] and e.outputs["ws"][0].tolist() == [0.5, 0.5]


def test_eval_linear_routed_and_combine_ranks_closed_forms():
    """Logits (5, -1, 9) route ranks to experts 2 and 0 of a table of three
    1 x 2 entries, over per-rank slices of (1, 2, 3, 4); the ranks combined
    by the route's weights, the softmax of (9, 5)."""
    def body(b):
        lg = b.input("logits", whole_row(3), F32)
        x = b.input("x", Shape(4, 2), F32)
        ids, ws = b.route("r", 2, None, lg)
        t = b.table("t", 3, [1, 2], F32)
        y = b.linear_routed("y", t, ids, x)
        b.output("y", y)
        b.output("c", b.combine_ranks("c", ws, y))
    c = check_program(program("routed", body))
    e = evaluate(c, Bindings(1, inputs={"logits": [[5, -1, 9]], "x": [[1, 2, 3, 4]]},
                             tables={"t": [[1, 1], [10, 100], [1000, 10000]]}))
    assert e.outputs["y"][0].tolist() == [1000 * 1 + 10000 * 2, 1 * 3 + 1 * 4]
    w0, w1 = 1 / (1 + math.exp(-4)), math.exp(-4) / (1 + math.exp(-4))
    assert abs(e.outputs["c"][0][0] - (w0 * 21000 + w1 * 7)) < 1e-9
    with pytest.raises(EvalError, match="has 2 entries bound, not 3"):
        evaluate(c, Bindings(1, inputs={"logits": [[5, -1, 9]], "x": [[1, 2, 3, 4]]}, tables={"t": [[1, 1], [2, 2]]}))


@pytest.mark.parametrize("n,k,scaled", [(16, 4, False), (64, 8, True), (8, 1, False), (128, 2, True)])
def test_the_oracles_route_is_the_evaluators(n, k, scaled):
    rng = np.random.default_rng(n + k)
    L = fkref.lib()
    for trial in range(50):
        x = rng.standard_normal(n).astype(np.float32)
        if trial % 5 == 0:
            x[rng.integers(n)] = x[rng.integers(n)]  # a tie, to the lower index
        s = (1 + 0.3 * rng.standard_normal(n)).astype(np.float32)
        ids = np.zeros(k, np.uint32)
        ws = np.zeros(k, np.float32)
        assert L.fkref_route(x.ctypes.data, s.ctypes.data if scaled else None, ids.ctypes.data, ws.ctypes.data, n,
                             k, int(scaled)) == 0
        b = Bindings(1, inputs={"x": [x.astype(np.float64)]}, weights={"s": s.astype(np.float64)} if scaled else {})
        e = evaluate(routing(n, k, scaled), b)
        assert ids.tolist() == [int(i) for i in e.outputs["ids"][0]]
        want = np.array(e.outputs["ws"][0])
        assert np.all(np.abs(ws - want) <= 1e-6 * np.abs(want) + 1e-30)
    assert L.fkref_route(x.ctypes.data, None, ids.ctypes.data, ws.ctypes.data, n, 9, 0) != 0


def test_the_moe_step_lowers_to_the_routed_launches():
    low = lowered(moe_program(CASES[0]))
    assert [L.entry for L in low.launches] == [
        "fk_rmsnorm_f32", "fk_step_gemv_f16_k2048_r1_p0_e0", "fk_step_route", "fk_gemv_routed_f16_r1",
        "fk_step_act_mul", "fk_gemv_routed_f16_r1", "fk_step_combine_ranks"]
    gu, down = low.launches[3], low.launches[5]
    assert gu.params["shared"] == 1 and down.params["shared"] == 0
    assert gu.bind["ids"] == down.bind["ids"] == "value:route_ids"
    assert low.constants["tableaddr:experts_gate_up"] == ("addresses", "table:experts_gate_up", 2 * 128 * 256 * 2)
    comb = low.launches[-1]
    assert comb.params == {"seg": 256, "ranks": 4, "residual": 1} and comb.bind["res"] == "value:x"


def eval_moe(checked, w, x):
    weights = {k: v.astype(np.float64).ravel() for k, v in w.items() if not k.startswith("experts_")}
    tables = {k: [e.astype(np.float64).ravel() for e in v] for k, v in w.items() if k.startswith("experts_")}
    return evaluate(checked, Bindings(1, inputs={"x": [x.astype(np.float64)]}, weights=weights, tables=tables))


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_the_moe_step_within_1e4_of_the_evaluator(case):
    checked = moe_program(case)
    w, x = state(case)
    cpu = run_cpu(lowered(checked), w, x)
    ev = eval_moe(checked, w, x)
    assert cpu.read("value:route_ids").tolist() == [int(i) for i in ev.values["route_ids"][0]]
    y, want = cpu.read("value:y"), np.array(ev.outputs["y"][0])
    assert float(np.max(np.abs(y - want)) / np.max(np.abs(want))) <= 1e-4
    # the experts' part alone (y - x), so the residual does not hide it
    part, want_part = y.astype(np.float64) - x, want - x
    assert float(np.max(np.abs(part - want_part)) / np.max(np.abs(want_part))) <= 1e-4


def test_a_wrong_expert_is_caught():
    """The check has teeth for the routed rows: the CPU target with the
    route's second id pointing at another expert misses by far more."""
    case = CASES[0]
    checked = moe_program(case)
    w, x = state(case)
    low = lowered(checked)
    cpu = run_cpu(low, w, x)
    ev = eval_moe(checked, w, x)
    ids = cpu.read("value:route_ids")
    ids[1] = (ids[1] + 1) % case[1] if (ids[1] + 1) % case[1] not in ids else (ids[1] + 2) % case[1]
    cpu.write("value:route_ids", ids)
    for L in low.launches[3:]:
        cpu.run_launch(L)
    want = np.array(ev.outputs["y"][0])
    assert float(np.max(np.abs(cpu.read("value:y") - want)) / np.max(np.abs(want - x))) > 1e-3


def host_checked(low):
    """Every launch through the engine's checks and the launch table's, on
    the host, over fake addresses of the buffers' sizes."""
    from furykernel_amd import kernels as K, runtime
    from furykernel_amd.engine import check_launch, params_struct
    at = 1 << 40
    addr = {}
    for name, spec in low.buffers.items():
        addr[name] = at
        at += (spec.nbytes + 4095) // 4096 * 4096
    for L in low.launches:
        check_launch(L, low.buffers)
        spans = [(0, 0) if L.bind.get(b) is None else (addr[L.bind[b]], low.buffers[L.bind[b]].nbytes)
                 for b in K.ABIS[L.entry].buffers]
        runtime.launch_check(L.entry, L.groups, L.threads, L.lds_bytes, spans, params_struct(L))


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_every_moe_launch_passes_the_launch_checks(case):
    host_checked(lowered(moe_program(case)))
