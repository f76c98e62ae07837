"""The GEMV step launches of the decode steps, checked on the CPU for accesses
out of bounds: at the grid the lowering gives them and at other grids (fewer
threadgroups than blocks, so wavefronts take several; more, so some take
none)."""

import dataclasses

import pytest

from furykernel_amd.lower import lower_plan
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import ONE_B, TINY, decoder_step
from furykernel_amd.program.plan import PlanOptions, plan
from gemv_bounds import Bad, check_launch

TINY32 = dataclasses.replace(TINY, context=32)


def gemv_launches(dims, options, layers=None):
    c = check_program(decoder_step(dims, embed=True, layers=layers))
    low = lower_plan(c, plan(options, c))
    return low, [L for L in low.launches if L.entry.startswith("fk_step_gemv")]


@pytest.mark.parametrize("dims,layers", [(ONE_B, 2), (TINY32, None)])
@pytest.mark.parametrize("store_gelus", [False, True])
def test_every_gemv_launch_in_bounds_at_any_grid(dims, layers, store_gelus):
    low, launches = gemv_launches(dims, PlanOptions(store_gelus=store_gelus), layers)
    for L in launches:
        grids = [L.groups] if L.params["epi_mode"] == 4 else [L.groups, 1, 7, 128, 256, 384, 512, 768, 1024, 1536]
        for g in grids:
            check_launch(L, low.buffers, g)


def test_the_checker_sees_a_grid_past_the_argmax_slots():
    low, launches = gemv_launches(ONE_B, PlanOptions(store_gelus=True), 1)
    head = launches[-1]
    assert head.params["epi_mode"] == 4
    bad = dataclasses.replace(head, params=dict(head.params, arg_slots=head.groups * 3))
    with pytest.raises(Bad):
        check_launch(bad, low.buffers)


def test_the_checker_sees_a_short_weight_buffer():
    low, launches = gemv_launches(ONE_B, PlanOptions(), 1)
    qkv = launches[0]
    bufs = dict(low.buffers)
    w = bufs[qkv.bind["w1"]]
    bufs[qkv.bind["w1"]] = dataclasses.replace(w, count=w.count - 8)
    with pytest.raises(Bad):
        check_launch(qkv, bufs)
