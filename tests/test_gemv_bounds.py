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


def probe_swaps(low, key: int, period: int):
    """The launches a grid sweep made when it put the first launch's entry of a
    class of the step (launch i with i mod period == key, one per layer, for
    layers of `period` launches) onto every launch of the class: its
    parameters and bindings stayed each launch's own."""
    idx = [i for i in range(16 * period) if i % period == key]
    first = low.launches[idx[0]].entry
    return [dataclasses.replace(low.launches[i], entry=first) for i in idx]


# Layers of six launches (attention in splits of 128, the combine a launch of
# its own) and of five (wide splits, the combine in the O step's prologue).
SWAPS = [(False, 6, 0, "token"), (False, 6, 3, "res_token"), (True, 5, 0, "token"), (True, 5, 2, "res_token")]


@pytest.mark.parametrize("wide,period,key,unbound", SWAPS)
def test_a_swapped_entry_reading_an_unbound_buffer_is_refused(wide, period, key, unbound):
    """Layer 0's QKV step gathers its row (_p3) and its O step adds a gathered
    residual (_e2); layers 1-15's do not, and leave token / res_token unbound.
    The layer-0 entry on a later layer's launch reads address 0: the CPU model
    of the kernel's accesses and the engine's launch check both refuse it."""
    from furykernel_amd.engine import check_launch as engine_check
    from furykernel_amd.kernels import LaunchError
    c = check_program(decoder_step(ONE_B, embed=True))
    low = lower_plan(c, plan(PlanOptions(store_gelus=True), c), wide=wide)
    assert len(low.launches) == 16 * period + 2
    swapped = probe_swaps(low, key, period)
    assert low.launches[key].bind[unbound] is not None
    refused = 0
    for L in swapped[1:]:
        assert L.bind[unbound] is None
        with pytest.raises(Bad, match=f"{unbound} is read or written but not bound"):
            check_launch(L, low.buffers)
        with pytest.raises(LaunchError):
            engine_check(L, low.buffers)
        refused += 1
    assert refused == 15
    # The launches as lowered pass both.
    for i in range(16 * period):
        if i % period == key:
            check_launch(low.launches[i], low.buffers)
            engine_check(low.launches[i], low.buffers)


def test_the_engine_refuses_modes_that_disagree_with_the_entry():
    from furykernel_amd.engine import check_launch as engine_check
    from furykernel_amd.kernels import LaunchError
    low, launches = gemv_launches(ONE_B, PlanOptions(), 1)
    qkv = launches[0]
    bad = dataclasses.replace(qkv, params=dict(qkv.params, pro_mode=1 if qkv.params["pro_mode"] != 1 else 0))
    with pytest.raises(LaunchError, match="its parameters say"):
        engine_check(bad, low.buffers)


def test_a_gathered_table_is_read_at_the_weights_element_size():
    """A table of f32 read by an f16 entry is the wrong type; an f16 table read
    by an f32 entry would read twice its bytes: both refused."""
    from furykernel_amd.engine import check_launch as engine_check
    from furykernel_amd.kernels import LaunchError
    c = check_program(decoder_step(ONE_B, embed=True, layers=1))
    low = lower_plan(c, plan(PlanOptions(), c))
    first = low.launches[0]
    assert first.params["pro_mode"] == 3
    bufs = dict(low.buffers)
    t = bufs[first.bind["table"]]
    bufs[first.bind["table"]] = dataclasses.replace(t, dtype="f32", count=t.count // 2)
    with pytest.raises(LaunchError, match="the kernel reads f16"):
        engine_check(first, bufs)
    with pytest.raises(Bad):
        check_launch(dataclasses.replace(first, entry=first.entry.replace("f16_k2048", "f32_k1024")), bufs)
