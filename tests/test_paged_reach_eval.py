"""Paged KV caches and attention with a reach in the binary64 evaluator
(oracle/eval.py, following src/FuryKernel/Program/Eval.hs:415-527,563-602)
and the gate: the reference's known answers evalSparse
(test/Test/FuryKernel/ProgramTest.hs:1453-1498), evalReach (:1541-1566) and
the gate's bounds of blocks, positions and reach (:359-372)."""

import numpy as np
import pytest

from furykernel_amd.program.build import program
from furykernel_amd.program.check import check_program, findings_of
from furykernel_amd.program.graph import AttnSpec, F32, Paged, Reach, Ring, Shape
from oracle.eval import Bindings, EvalError, evaluate


def huge_pool():
    """ProgramTest.hs:1436-1451: attention over a pool of 2^30 blocks of 4
    positions, its keys and values stored first."""
    def body(b):
        q = b.input("q", Shape(2, 2), F32)
        pos = b.row_ints("position", 1, 8)
        blocks = b.row_ints("blocks", 2, 2 ** 30)
        k = b.cache("k", Paged(2 ** 30, 4, 1, 2))
        v = b.cache("v", Paged(2 ** 30, 4, 1, 2))
        kv = b.input("kv", Shape(2, 2), F32)
        b.kv_store("store_k", k, pos, blocks, kv)
        b.kv_store("store_v", v, pos, blocks, kv)
        b.output("o", b.attend("o", AttnSpec(1, 1, 2, None, 1.0), q, k, v, pos, blocks))
    return program("huge_pool", body)


B1, B2 = 123456789, 987654321


def sparse(pool):
    return Bindings(1, inputs={"q": [[0, 0]], "kv": [[0.5, 0.25]]},
                    row_ints={"position": [[5]], "blocks": [[B1, B2]]},
                    caches={"k": {u: list(x) for u, x in pool.items()}, "v": {u: list(x) for u, x in pool.items()}})


def test_eval_sparse_known_answer():
    """Blocks 123456789 and 987654321 of the 2^30, a row at position 5: the
    second block's element 2 on; positions 0 to 3 hold ones, 4 zeros.  A
    query of zeros weighs the six positions alike."""
    c = check_program(huge_pool())
    e = evaluate(c, sparse({B1: [1.0] * 8, B2: [0.0] * 8}))
    want = [sum(x / 6 for x in (1, 1, 1, 1, 0, 0.5)), sum(x / 6 for x in (1, 1, 1, 1, 0, 0.25))]
    assert np.max(np.abs(np.array(e.outputs["o"][0]) - want)) < 1e-12
    assert e.caches["k"][B1].tolist() == [1.0] * 8
    assert e.caches["k"][B2].tolist() == [0, 0, 0.5, 0.25, 0, 0, 0, 0]
    with pytest.raises(EvalError, match="A store to k at block 987654321, element 2, which isn't bound."):
        evaluate(c, sparse({B1: [1.0] * 8}))
    with pytest.raises(EvalError, match="k: block 123456789, element 0, isn't bound."):
        evaluate(c, sparse({B2: [0.0] * 8}))


def test_a_ring_bound_by_its_steps_slot():
    """ProgramTest.hs:1480-1498: a ring of two slots read through slot 1
    only; a store to an unbound slot is refused."""
    def body(b):
        q = b.input("q", Shape(4, 2), F32)
        pos = b.row_ints("position", 1, 4)
        slot = b.row_ints("slot", 1, 2)
        k = b.cache("k", Ring(2, 1, 4, 2))
        v = b.cache("v", Ring(2, 1, 4, 2))
        kv = b.input("kv", Shape(2, 2), F32)
        b.kv_store("store_k", k, pos, slot, kv)
        b.kv_store("store_v", v, pos, slot, kv)
        b.output("o", b.attend("o", AttnSpec(2, 1, 2, None, 1.0), q, k, v, pos, slot))
    c = check_program(program("ring_slots", body))

    def out(caches):
        return evaluate(c, Bindings(1, inputs={"q": [[1, 2, 3, 4]], "kv": [[0.5, 0.25]]},
                                    row_ints={"position": [[2]], "slot": [[1]]},
                                    caches={"k": caches, "v": caches})).outputs["o"]
    both = {0: [float(x) for x in range(1, 9)], 1: [float(x) for x in range(9, 17)]}
    assert np.array_equal(out(both)[0], out({1: [float(x) for x in range(9, 17)]})[0])
    with pytest.raises(EvalError, match="A store to k at slot 1, element 4, which isn't bound."):
        out({0: [float(x) for x in range(1, 9)]})


def reaching(length, window, ahead, position_bound, reach_bound):
    """ProgramTest.hs:1568-1582: a ring of `length`, the window and reach
    given, keys and values stored first."""
    def body(b):
        q = b.input("q", Shape(4, 2), F32)
        pos = b.row_ints("position", 1, position_bound)
        slot = b.row_ints("slot", 1, 1)
        reach = None if ahead is None else Reach(b.row_ints("reach", 1, reach_bound).id, ahead)
        k = b.cache("k", Ring(1, 1, length, 2))
        v = b.cache("v", Ring(1, 1, length, 2))
        kv = b.input("kv", Shape(2, 2), F32)
        b.kv_store("store_k", k, pos, slot, kv)
        b.kv_store("store_v", v, pos, slot, kv)
        b.output("o", b.attend("o", AttnSpec(2, 1, 2, window, 1.0, reach), q, k, v, pos, slot))
    return check_program(program("reach", body))


def test_eval_reach_known_answers():
    b = Bindings(2, inputs={"q": [[0, 0, 0, 0]] * 2, "kv": [[0.5, 0.25], [0.75, 1]]},
                 row_ints={"position": [[0], [1]], "slot": [[0], [0]], "reach": [[1], [1]]},
                 caches={"k": {0: [0.0] * 8}, "v": {0: [0.0] * 8}})
    # with a reach, row 0 sees position 1 too; without, only its own
    got = evaluate(reaching(4, None, 3, 4, 4), b).outputs["o"]
    assert [list(r) for r in got] == [[0.625] * 4] * 2
    got = evaluate(reaching(4, None, None, 4, 4), b).outputs["o"]
    assert [list(r) for r in got] == [[0.5, 0.25, 0.5, 0.25], [0.625] * 4]
    # A ring of four, a window of two and a reach of up to two ahead, rows 1
    # to 3 an image's: rows 4 and 5 store over positions 0 and 1, which row 1
    # reads as the step's own rows left them.
    kvs = [[0.5, 0.25], [0.75, 1], [0.25, 0.5], [0.5, 0.25], [1, 0.5], [0.25, 0.75]]
    image = Bindings(6, inputs={"q": [[0, 0, 0, 0]] * 6, "kv": kvs},
                     row_ints={"position": [[t] for t in range(6)], "slot": [[0]] * 6,
                               "reach": [[0], [3], [3], [3], [4], [5]]},
                     caches={"k": {0: [0.0] * 8}, "v": {0: [0.0] * 8}})
    got = evaluate(reaching(4, 2, 2, 8, 8), image).outputs["o"]
    assert [list(got[i][:2]) for i in (0, 1, 4, 5)] == [[0.5, 0.25], [0.5, 0.5], [0.75, 0.375], [0.625, 0.625]]
    with pytest.raises(EvalError, match="o: row 1 reaches 3, more than 1 past its position, 1."):
        evaluate(reaching(4, 2, 1, 8, 8), image)


def stored_into(layout, sequences, positions):
    def body(b):
        x = b.input("x", Shape(2, 2), F32)
        pos = b.row_ints("position", 1, positions)
        sq = b.row_ints("slot", 1, sequences) if isinstance(layout, Ring) else b.row_ints("blocks", 2, sequences)
        k = b.cache("k", layout)
        b.kv_store("store_k", k, pos, sq, x)
    return program("stored_into", body)


def messages(p):
    return [f.message for f in findings_of(p)]


def test_the_gate_bounds_a_stores_blocks_by_the_pool_and_its_positions_by_its_table():
    assert messages(stored_into(Ring(2, 1, 4, 2), 2, 64)) == []
    assert messages(stored_into(Ring(2, 1, 4, 2), 3, 64)) == [
        "store_k: the bound of slot, 3, is more than the 2 slots of k."]
    assert messages(stored_into(Paged(4, 2, 1, 2), 4, 4)) == []
    assert messages(stored_into(Paged(4, 2, 1, 2), 5, 4)) == [
        "store_k: the bound of blocks, 5, is more than the 4 blocks of k."]
    assert messages(stored_into(Paged(4, 2, 1, 2), 4, 5)) == [
        "store_k: the bound of position, 5, is more than the 4 positions of its block table."]
