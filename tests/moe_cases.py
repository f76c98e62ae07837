"""A routed-experts decode step (the reference's MoE half of its layer,
test/Test/FuryKernel/ProgramTest.hs:533-547 of `layer`, :488-557, on its own): the row normed,
the router's logits, the k experts routed, their gate/up rows from a table,
the gated GELU of each rank's rows, their down rows, the ranks combined by
the route's weights and added to the row.  Seeded state, and the step's runs
on the oracle's CPU target."""

from __future__ import annotations

import numpy as np

from furykernel_amd.lower import lower_plan
from furykernel_amd.program.build import program
from furykernel_amd.program.check import check_program
from furykernel_amd.program.graph import F16, F32, whole_row
from furykernel_amd.program.plan import PlanOptions, plan
from oracle.cpu_target import CpuTarget

# hidden, experts, expert ffn, k, expert scale
CASES = [(256, 16, 128, 4, False), (512, 8, 256, 2, True)]
ONE_B_MOE = (2048, 16, 1024, 2, True)


def case_id(c) -> str:
    return "h{}_e{}_f{}_k{}_s{}".format(*[int(x) for x in c])


def moe_program(c):
    hidden, experts, ffn, k, scaled = c

    def body(b):
        x = b.input("x", whole_row(hidden), F32)
        g = b.weight("moe_norm", [hidden], F32)
        router = b.weight("router", [experts, hidden], F16)
        scale = b.weight("expert_scale", [experts], F32) if scaled else None
        gu = b.table("experts_gate_up", experts, [2 * ffn, hidden], F16)
        dn = b.table("experts_down", experts, [hidden, ffn], F16)
        cn = b.rmsnorm("moe_in", 1e-6, g, 1.0, x)
        logits = b.linear("router_logits", router, 0, cn)
        ids, ws = b.route("route", k, scale, logits)
        gue = b.linear_routed("experts_gate_up_out", gu, ids, cn)
        act = b.gated_gelu("experts_act", gue)
        de = b.linear_routed("experts_out", dn, ids, act)
        s = b.combine_ranks("experts_sum", ws, de)
        b.output("y", b.add("y", x, s))
    return check_program(program("moe", body))


def state(c, seed=11):
    hidden, experts, ffn, k, scaled = c
    rng = np.random.default_rng(seed)
    w = {"moe_norm": (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32),
         "router": (rng.standard_normal((experts, hidden)) * 0.2).astype(np.float16),
         "experts_gate_up": (rng.standard_normal((experts, 2 * ffn, hidden)) * 0.05).astype(np.float16),
         "experts_down": (rng.standard_normal((experts, hidden, ffn)) * 0.05).astype(np.float16)}
    if scaled:
        w["expert_scale"] = (1 + 0.2 * rng.standard_normal(experts)).astype(np.float32)
    x = rng.standard_normal(hidden).astype(np.float32)
    return w, x


def lowered(checked):
    return lower_plan(checked, plan(PlanOptions(), checked))


def run_cpu(low, w, x):
    cpu = CpuTarget(low, 64)
    for name, v in w.items():
        if f"weight:{name}" in low.buffers:
            cpu.write(f"weight:{name}", v.ravel())
        if f"table:{name}" in low.buffers:
            cpu.write(f"table:{name}", v.ravel())
    cpu.write("value:x", x)
    cpu.run()
    return cpu
