"""The program layer's gate and planner against the reference's goldens
(test/Test/FuryKernel/ProgramTest.hs:43-400) and its plan checker."""

import dataclasses
import math

import pytest

from furykernel_amd.program.check import BOUNDS, NAMES, SHAPES, STRUCTURE, ProgramRefused, check_program, findings_of
from furykernel_amd.program.graph import Paged, Ring, render_program
from furykernel_amd.program.plan import (
    DEFAULT_OPTIONS, EXPENSIVE, LAND, STAGE, PlanOptions, node_cost, plan, render_plan)

import programs as P
from plancheck import plan_issues


def lines_of(pl):
    return render_plan(pl).rstrip("\n").split("\n")


def names_of(prog, opts=DEFAULT_OPTIONS):
    return [s.name for s in plan(opts, check_program(prog)).steps]


def unplaced(prog):
    return [f.unplaced() for f in findings_of(prog)]


def test_a_layer_passes_the_gate():
    check_program(P.layer(False))


@pytest.mark.parametrize("name,prog,opts", [
    ("layer", P.layer(False), DEFAULT_OPTIONS),
    ("head", P.head_program(), DEFAULT_OPTIONS),
    ("embed", P.embed_program(), DEFAULT_OPTIONS),
    ("two_tiles", P.two_tiles(), DEFAULT_OPTIONS),
    ("attn_out", P.attn_out(), DEFAULT_OPTIONS),
    ("attn_capped", P.attn_capped(), DEFAULT_OPTIONS),
    ("attn_stored", P.attn_stored(), DEFAULT_OPTIONS),
    ("attn_normed", P.attn_normed(), DEFAULT_OPTIONS),
    ("attn_mixed", P.attn_mixed(), DEFAULT_OPTIONS),
    ("attn_kept", P.attn_kept(), DEFAULT_OPTIONS),
    ("predicting_gated", P.predicting(), PlanOptions(gated=True)),
    ("ring_staged", P.ring_program(), PlanOptions(sequence_rows=4)),
])
def test_plan_goldens(golden, name, prog, opts):
    assert lines_of(plan(opts, check_program(prog))) == golden("plans.json")[name]["lines"]


def test_step_names_under_options(golden):
    g = golden("plans.json")["step_names"]
    assert names_of(P.layer(True)) == g["layer_kv_default"]
    assert names_of(P.layer(False), PlanOptions(store_gelus=True)) == g["layer_store_gelus"]
    assert names_of(P.layer(False), PlanOptions(gated=True, store_gelus=True)) == g["layer_gated_store_gelus"]
    assert names_of(P.layer(False), PlanOptions(gated=True)) == g["layer_gated"]
    assert names_of(P.pooled()) == g["pooled"]
    assert names_of(P.embed_program()) == g["embed"]


def test_a_program_renders(golden):
    assert render_program(P.small()).rstrip("\n").split("\n") == golden("plans.json")["small_render"]["lines"]


def test_a_chain_reached_by_many_paths_is_planned_over_each_node_once():
    """ProgramTest.hs:103-110: 40 doublings."""
    from furykernel_amd.program.build import program
    from furykernel_amd.program.graph import whole_row

    def body(b):
        x = b.input("x", whole_row(4))
        w = b.weight("w", [4, 4])
        y = x
        for k in range(1, 41):
            y = b.add(f"d{k}", y, y)
        b.output("y", b.linear("y", w, 0, y))

    pl = plan(DEFAULT_OPTIONS, check_program(program("doubled", body)))
    assert [(s.name, len(s.work)) for s in pl.steps] == [("s0_gemv", 41)]


def test_every_test_programs_plans_pass_the_plan_checker():
    """ProgramTest.hs:262-268: under every set of options."""
    bad = []
    for prog in P.planned():
        for h in (True, False):
            for gd in (False, True):
                for s in (False, True):
                    for r in (1, 64):
                        opts = PlanOptions(h, gd, s, r)
                        found = plan_issues(opts, plan(opts, check_program(prog)))
                        if found:
                            bad.append((prog.name, opts, found))
    assert bad == []


def test_ring_with_room_lands_before_the_attention():
    opts = PlanOptions(sequence_rows=3)
    pl = plan(opts, check_program(P.ring_program()))
    assert [w for s in pl.steps for w in s.work if w.kind in (STAGE, LAND)] == []
    assert plan_issues(opts, pl) == []


def test_combine_step_names_the_caches_it_lands_in():
    def caches(rows):
        return [s.caches for s in plan(PlanOptions(sequence_rows=rows), check_program(P.ring_program())).steps
                if s.name == "s2_combine"]
    assert caches(3) == [[]]
    assert [len(c) for c in caches(4)] == [2]


def test_plan_checker_refuses_misplaced_lands_and_stagings():
    """ProgramTest.hs:300-318."""
    opts = PlanOptions(sequence_rows=4)
    pl = plan(opts, check_program(P.ring_program()))
    first = plan(DEFAULT_OPTIONS, check_program(P.ring_program()))
    lands = [w for s in pl.steps for w in s.work if w.kind == LAND]
    early_steps = [dataclasses.replace(s, work=[w for w in s.work if w.kind != LAND] +
                                       (lands if s.name == "s1_attend" else [])) for s in pl.steps]
    early = dataclasses.replace(pl, steps=early_steps)
    assert any("lands in a step no later than o's" in i for i in plan_issues(opts, early))
    assert plan_issues(opts, first) == [
        "store_k: stored first, though its ring hasn't room for a step's rows of one sequence",
        "store_v: stored first, though its ring hasn't room for a step's rows of one sequence"]
    assert plan_issues(DEFAULT_OPTIONS, pl) == [
        "store_k: staged, though its ring has room for a step's rows of one sequence",
        "store_v: staged, though its ring has room for a step's rows of one sequence"]


def test_a_gather_of_several_rows_is_expensive():
    pooled = P.pooled()
    from furykernel_amd.program.graph import Gather
    assert [node_cost(pooled, n.op) for n in pooled.nodes if isinstance(n.op, Gather)] == [EXPENSIVE]


# The gate ---------------------------------------------------------------------

def test_gate_bounds_routed_ids_by_the_tables_entries():
    F = lambda r, m: (r, m)
    assert [F(f.rule, f.message) for f in unplaced(P.routed_over(8, 8))] == []
    assert [F(f.rule, f.message) for f in unplaced(P.routed_over(16, 8))] == [
        (BOUNDS, "experts_out: the bound of its ids, 16, is more than the 8 entries of experts.")]


def test_gate_bounds_slots_blocks_and_positions():
    def msgs(p):
        return [(f.rule, f.message) for f in unplaced(p)]
    assert msgs(P.stored_into(Ring(2, 1, 4, 2), 2, 64)) == []
    assert msgs(P.stored_into(Ring(2, 1, 4, 2), 3, 64)) == [
        (BOUNDS, "store_k: the bound of slot, 3, is more than the 2 slots of k.")]
    assert msgs(P.stored_into(Paged(4, 2, 1, 2), 4, 4)) == []
    assert msgs(P.stored_into(Paged(4, 2, 1, 2), 5, 4)) == [
        (BOUNDS, "store_k: the bound of blocks, 5, is more than the 4 blocks of k.")]
    assert msgs(P.stored_into(Paged(4, 2, 1, 2), 4, 5)) == [
        (BOUNDS, "store_k: the bound of position, 5, is more than the 4 positions of its block table.")]
    assert msgs(P.paged_attention(4, 4, True)) == []
    assert msgs(P.paged_attention(4, 5, True)) == [
        (BOUNDS, "o: the bound of position, 5, is more than the 4 positions of its block table."),
        (BOUNDS, "o: the bound of reach, 5, is more than the 4 positions of its block table.")]


def test_gate_holds_attention_over_a_ring_to_what_it_holds():
    def msgs(p):
        return [f.message for f in unplaced(p)]
    assert msgs(P.over_ring(2, 2, 64)) == []
    assert msgs(P.over_ring(2, 3, 64)) == ["o: its window of 3 positions is longer than the 2 that k's ring holds."]
    assert msgs(P.over_ring(4, None, 4)) == []
    assert msgs(P.over_ring(4, None, 5)) == [
        "o: with no window it reads every position below the bound of position, 5, more than the 4 that k's ring holds."]
    assert msgs(P.reaching(4, 2, 2, 64, 64)) == []
    assert msgs(P.reaching(4, 2, 3, 64, 64)) == [
        "o: its window of 2 and its reach of up to 3 past a row's own position read 5 positions, more than the 4 "
        "that k's ring holds."]
    assert msgs(P.reaching(4, 2, 3, 64, 3)) == []
    assert msgs(P.reaching(4, None, 3, 2, 64)) == [
        "o: with no window, and a reach of up to 3 past a row's own position, it reads every position below 5, more "
        "than the 4 that k's ring holds."]


def test_gate_refuses_structure_and_shapes():
    small = P.small()
    rev = dataclasses.replace(small, sources=list(reversed(small.sources)))
    assert [(f.rule, f.message) for f in unplaced(rev)] == [
        (STRUCTURE, "The source ids don't increase in program order: 1, then 0.")]
    assert [(f.rule, f.message) for f in unplaced(P.stored_into(Ring(1, 1, 0, 2), 1, 1))] == [
        (SHAPES, "The cache k has a length of 0.")]
    renamed = dataclasses.replace(small, outputs=[dataclasses.replace(o, name="float") for o in small.outputs])
    assert [(f.rule, f.message) for f in unplaced(renamed)] == [(NAMES, "The name float is reserved in a target language.")]
    joined = dataclasses.replace(small, name="small_x_one")
    assert [(f.rule, f.message) for f in unplaced(joined)] == [
        (NAMES, "The program's name small_x_one holds _x_, which joins it to its steps' names.")]
    with pytest.raises(ProgramRefused):
        check_program(joined)


def test_gate_places_findings_in_program_and_node():
    from furykernel_amd.program.graph import RmsNorm
    small = P.small()
    bad = dataclasses.replace(small, name="small_x_one", nodes=[
        dataclasses.replace(n, op=dataclasses.replace(n.op, eps=math.inf)) if isinstance(n.op, RmsNorm) else n
        for n in small.nodes])
    assert [(f.location.program, f.location.nodes) for f in findings_of(bad)] == [
        ("small_x_one", ()), ("small_x_one", ("n",))]
