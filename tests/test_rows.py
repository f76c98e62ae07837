"""Steps of any number of rows through the prefill kernels, on the CPU: the
placement of a ragged prefill's rows (sequences of any length) and of a
decode step of several rows (each its own sequence, position and slot) into
a step of whole tiles, and the lowering's scratch slot that the rows filling
the tiles out store into."""

import numpy as np
import pytest

from furykernel_amd.lower import LoweringError
from furykernel_amd.prefill import (QBLOCK, SLAB, check_rows, decode_placement, lower_prefill, prefill_placement,
                                    run_of)
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import SMALL_PREFILL, decoder_step
from furykernel_amd.program.plan import PlanOptions, plan


def test_runs_round_up_to_whole_query_blocks_and_tiles():
    assert [run_of(n) for n in (1, 31, 32, 33, 100, 128, 129, 256, 257, 2048)] == \
        [32, 32, 32, 64, 128, 128, 256, 256, 512, 2048]
    with pytest.raises(LoweringError):
        run_of(0)


@pytest.mark.parametrize("seqs,seq_rows", [(1, 100), (2, 100), (3, 70), (4, 2048), (2, 128)])
def test_a_ragged_prefill_places_each_sequence_first_in_its_run(seqs, seq_rows):
    n_slots = 4
    rows, run, pos, sl, real = prefill_placement(seqs, seq_rows, n_slots)
    assert rows % SLAB == 0 and rows % run == 0 and run % QBLOCK == 0
    assert real.size == seqs * seq_rows
    for i in range(seqs):
        r = real[i * seq_rows:(i + 1) * seq_rows]
        assert np.array_equal(pos[r], np.arange(seq_rows)) and np.all(sl[r] == i)
    fill = np.setdiff1d(np.arange(rows), real)
    assert np.all(sl[fill] == n_slots)
    check_rows(pos, np.where(np.isin(np.arange(rows), real), sl.astype(np.int64), -1), QBLOCK, first_rows=True)


def test_a_decode_step_places_each_row_first_in_its_block():
    rows, pos, sl, real = decode_placement([5, 40, 200, 255], [0, 3, 1, 2], 4)
    assert rows == SLAB and real.tolist() == [0, 32, 64, 96]
    assert pos[real].tolist() == [5, 40, 200, 255] and sl[real].tolist() == [0, 3, 1, 2]
    assert np.array_equal(pos[32:64], 40 + np.arange(32))  # the block continues the row's positions
    assert np.all(np.delete(sl, real) == 4)                  # in the scratch slot
    check_rows(pos, np.where(np.isin(np.arange(rows), real), sl.astype(np.int64), -1), QBLOCK, first_rows=True)
    with pytest.raises(LoweringError):
        decode_placement([5], [4], 4)


def test_the_attention_contract_refuses_real_rows_after_filling_ones():
    pos = np.arange(32)
    sl = np.full(32, -1)
    sl[5] = 0   # a real row after filling rows
    with pytest.raises(LoweringError):
        check_rows(pos, sl, QBLOCK, first_rows=True)
    sl = np.zeros(32)
    sl[31] = 1  # two sequences in a block
    with pytest.raises(LoweringError):
        check_rows(pos, sl, QBLOCK, first_rows=True)


def test_the_scratch_slot_is_one_past_the_programs():
    c = check_program(decoder_step(SMALL_PREFILL, "prefill", position_bound=128))
    pl = plan(PlanOptions(sequence_rows=100), c)
    plain = lower_prefill(c, pl, 256, 128)
    scratch = lower_prefill(c, pl, 256, 128, scratch_slot=True)
    for name, spec in plain.buffers.items():
        if name.startswith("cache:"):
            assert scratch.buffers[name].count == spec.count // SMALL_PREFILL.slots * (SMALL_PREFILL.slots + 1)
    for L, M in zip(plain.launches, scratch.launches):
        if "slots" in L.params and L.params["slots"]:
            assert M.params["slots"] == L.params["slots"] + 1, L.entry
