"""Paged KV pools and attention with a reach, lowered and run by the oracle's
CPU target (the kernels' arithmetic), on the CPU: the lowering's launches;
the paged step's partials and rows bit for bit the ring step's over the same
keys and values (the layout changes where rows live, not the order of any
sum); both within 1e-4 of the binary64 evaluator (Eval.hs:415-527 with
cacheIndex :592-602); a reach reading the rows past its position; and a
scrambled block table caught."""

import numpy as np
import pytest

from oracle.eval import Bindings, evaluate
from paged_cases import CASES, case_id, lowered, paged_program, ring_program, run_cpu, state


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def widen(bits, bf16):
    bits = np.ascontiguousarray(bits).view(np.uint16)
    if bf16:
        return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return bits.view(np.float16).astype(np.float64)


def eval_paged(checked, c, x, position, table, pool, reach=None):
    heads, kv, d, bs, blocks, tl, window, bf16 = c
    caches = {name: {int(b): widen(pool[j][b], bf16).ravel() for b in range(blocks)}
              for j, name in enumerate(("kc", "vc"))}
    ints = {"position": [[position]], "blocks": [list(map(int, table))]}
    if reach is not None:
        ints["reach"] = [[reach]]
    return evaluate(checked, Bindings(1, inputs={k: [v.astype(np.float64)] for k, v in x.items()}, row_ints=ints,
                                      caches=caches))


def test_a_paged_step_lowers_to_the_paged_attention_with_its_store():
    c = CASES[0]
    low = lowered(paged_program(c))
    entries = [L.entry for L in low.launches]
    assert entries == ["fk_step_attend_paged", "fk_step_combine"]
    att = low.launches[0]
    assert (att.params["store"], att.params["krope"], att.params["rope"]) == (1, 1, 1)
    assert (att.params["block_size"], att.params["table_len"], att.params["blocks"]) == (16, 16, 64)
    assert att.bind["kpool"] == "addr:kc" and att.bind["table"] == "ints:blocks"
    assert low.constants["addr:kc"] == ("addresses", "cache:kc", 16 * 2 * 64 * 2)
    from furykernel_amd.lower import lower_plan
    from furykernel_amd.program.plan import PlanOptions, plan
    ch = paged_program(c)
    apart = lower_plan(ch, plan(PlanOptions(), ch), fuse=False)
    assert [L.entry for L in apart.launches] == ["fk_step_store_paged", "fk_step_attend_paged", "fk_step_combine"]


@pytest.mark.parametrize("position", [0, 17, 200, 255])
@pytest.mark.parametrize("case", CASES[:1] + CASES[2:], ids=case_id)
def test_paged_is_the_ring_bit_for_bit_and_within_1e4_of_the_evaluator(case, position):
    heads, kv, d, bs, blocks, tl, window, bf16 = case
    position = min(position, bs * tl - 1)
    x, table, pool, ring = state(case, position)
    pg = run_cpu(lowered(paged_program(case)), x, position, table=table, pool=pool)
    rg = run_cpu(lowered(ring_program(case)), x, position, ring=ring)
    assert np.array_equal(pg.read("value:o").view(np.uint32), rg.read("value:o").view(np.uint32))
    assert np.array_equal(pg.read("partials:o").view(np.uint32), rg.read("partials:o").view(np.uint32))
    # the stored rows: the pool's block table[position // bs] row, the ring's position row
    blk, row = table[position // bs], position % bs
    stored = pg.read("cache:kc").reshape(blocks, kv, bs, d)[blk, :, row]
    assert np.array_equal(stored, rg.read("cache:kc").reshape(kv, bs * tl, d)[:, position])
    ev = eval_paged(paged_program(case), case, x, position, table, pool)
    assert rel(pg.read("value:o"), ev.outputs["o"][0]) <= 1e-4
    # the pool the evaluator left: every element the step did not store as it
    # was; the stored rows within a rounding of the cache's type (the key's
    # RoPE here takes the binary32 table's cosines, the evaluator exact ones)
    ulp = 2.0 ** (-7 if bf16 else -10)
    for j, name in enumerate(("kc", "vc")):
        got = widen(pg.read(f"cache:{name}"), bf16).reshape(blocks, kv, bs, d)
        want = np.stack([ev.caches[name][b] for b in range(blocks)]).reshape(blocks, kv, bs, d)
        mask = np.ones(got.shape, bool)
        mask[blk, :, row] = False
        assert np.array_equal(got[mask], want[mask]), name
        assert np.all(np.abs(got[blk, :, row] - want[blk, :, row]) <= ulp * np.abs(want[blk, :, row]) + 1e-30), name


def test_a_scrambled_block_table_is_caught():
    """The check has teeth for the table: the CPU target reading through a
    table whose first entry names another block of the pool misses the
    evaluator by far more than 1e-4.  (Swapping two entries would not: the
    cached keys are rotated already, and attention over a set of positions
    does not see their order.)"""
    case = CASES[0]
    position = 200
    x, table, pool, ring = state(case, position)
    bad = table.copy()
    bad[0] = next(b for b in range(case[4]) if b not in set(table.tolist()))
    pg = run_cpu(lowered(paged_program(case)), x, position, table=bad, pool=pool)
    ev = eval_paged(paged_program(case), case, x, position, table, pool)
    assert rel(pg.read("value:o"), ev.outputs["o"][0]) > 1e-3


@pytest.mark.parametrize("paged", [False, True], ids=["ring", "paged"])
def test_a_reach_reads_past_the_rows_position(paged):
    """A row at position 100 with a reach of 180: positions 0 to 180 of the
    caches as they stand (its own row stored first), within 1e-4 of the
    evaluator; and not what the row without its reach computes."""
    case = CASES[0]
    heads, kv, d, bs, blocks, tl, window, bf16 = case
    position, reach = 100, 180
    x, table, pool, ring = state(case, position)
    checked = (paged_program if paged else ring_program)(case, reach_bound=bs * tl)
    low = lowered(checked)
    att = low.launches[0]
    assert att.params["has_reach"] == 1 and att.bind["reach"] == "ints:reach"
    if paged:
        cpu = run_cpu(low, x, position, table=table, pool=pool, reach=reach)
        ev = eval_paged(checked, case, x, position, table, pool, reach=reach)
    else:
        cpu = run_cpu(low, x, position, ring=ring, reach=reach)
        ev = evaluate(checked, Bindings(1, inputs={k: [v.astype(np.float64)] for k, v in x.items()},
                                        row_ints={"position": [[position]], "slot": [[0]], "reach": [[reach]]},
                                        caches={n: {0: widen(ring[j], bf16).ravel()}
                                                for j, n in enumerate(("kc", "vc"))}))
    assert rel(cpu.read("value:o"), ev.outputs["o"][0]) <= 1e-4
    own = run_cpu(low, x, position, **({"table": table, "pool": pool} if paged else {"ring": ring}),
                  reach=position)
    assert rel(own.read("value:o"), ev.outputs["o"][0]) > 1e-3


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_every_paged_launch_passes_the_launch_checks(case):
    from test_moe import host_checked
    from furykernel_amd.lower import lower_plan
    from furykernel_amd.program.plan import PlanOptions, plan
    for checked in (paged_program(case), paged_program(case, reach_bound=case[3] * case[5]), ring_program(case)):
        for fuse in (True, False):
            host_checked(lower_plan(checked, plan(PlanOptions(), checked), fuse=fuse))


def test_the_planner_stages_ring_stores_only():
    """Plan.hs:335-345 stages a store only into a ring (``SCache (Ring ..)``)
    whose room is short of a step's rows; a paged pool's store is never
    staged, whatever the rows: the same prefill program over a ring of 256
    positions with positions bound by the whole ring stages its stores, and
    over a paged pool of the same positions does not (so no lowering of a
    staged store into a pool is asked for)."""
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import SMALL_PREFILL, decoder_step
    from furykernel_amd.program.plan import LAND, STAGE, PlanOptions, plan

    def kinds(paging):
        c = check_program(decoder_step(SMALL_PREFILL, name="prefill", layers=1, paging=paging))
        return {w.kind for s in plan(PlanOptions(sequence_rows=128), c).steps for w in s.work}

    assert {STAGE, LAND} <= kinds(None)
    assert not {STAGE, LAND} & kinds((64, 16))
