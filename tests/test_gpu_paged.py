"""Paged KV pools and attention with a reach on the GPU: the lowered step
(fk_step_attend_paged with the KV store folded in, or fk_step_store_paged
apart, then the combine) through the engine, every buffer it writes bit for
bit the oracle's CPU target's; the paged rows the ring rows' over the same
keys and values; and a reach over a ring and a pool."""

import numpy as np
import pytest

from furykernel_amd.engine import Engine, _NP
from furykernel_amd.lower import lower_plan
from furykernel_amd.program.plan import PlanOptions, plan
from paged_cases import CASES, case_id, lowered, paged_program, ring_program, run_cpu, state

pytestmark = pytest.mark.gpu


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view({4: np.uint32, 2: np.uint16, 8: np.uint64}[a.dtype.itemsize])


def run_gpu(device, kernels, low, x, position, table=None, pool=None, ring=None, reach=None):
    eng = Engine(device, kernels, low)

    def raw(name, a):
        eng.write(name, np.ascontiguousarray(a).ravel().view(_NP[low.buffers[name].dtype]))

    for name, val in x.items():
        eng.write(f"value:{name}", val)
    eng.write("ints:position", np.array([position], np.uint32))
    if table is not None:
        eng.write("ints:blocks", table)
        raw("cache:kc", pool[0])
        raw("cache:vc", pool[1])
    else:
        eng.write("ints:slot", np.array([0], np.uint32))
        raw("cache:kc", ring[0])
        raw("cache:vc", ring[1])
    if reach is not None:
        eng.write("ints:reach", np.array([reach], np.uint32))
    eng.enqueue()
    device.sync()
    return eng


def compare(eng, cpu, low):
    bad = []
    for name in low.buffers:
        if name.startswith("addr:"):
            continue  # device addresses; the CPU target's are its own
        if not np.array_equal(bits(eng.read(name)), bits(cpu.read(name))):
            bad.append(name)
    return bad


@pytest.mark.parametrize("fuse", [True, False], ids=["fused", "apart"])
@pytest.mark.parametrize("position", [0, 200, 1023])
@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_paged_step_bit_exact_and_the_rings(device, kernels, case, position, fuse):
    heads, kv, d, bs, blocks, tl, window, bf16 = case
    position = min(position, bs * tl - 1)
    x, table, pool, ring = state(case, position)
    checked = paged_program(case)
    low = lower_plan(checked, plan(PlanOptions(), checked), fuse=fuse)
    print(f"paged decode attention {case_id(case)} at {position}, fuse {fuse}: "
          f"{[L.entry for L in low.launches]}", flush=True)
    eng = run_gpu(device, kernels, low, x, position, table=table, pool=pool)
    try:
        cpu = run_cpu(low, x, position, table=table, pool=pool)
        assert compare(eng, cpu, low) == []
        if fuse:
            rlow = lowered(ring_program(case))
            reng = run_gpu(device, kernels, rlow, x, position, ring=ring)
            try:
                assert np.array_equal(bits(eng.read("value:o")), bits(reng.read("value:o")))
                assert np.array_equal(bits(eng.read("partials:o")), bits(reng.read("partials:o")))
            finally:
                reng.close()
    finally:
        eng.close()


@pytest.mark.parametrize("paged", [False, True], ids=["ring", "paged"])
def test_a_reach_on_the_gpu(device, kernels, paged):
    case = CASES[0]
    heads, kv, d, bs, blocks, tl, window, bf16 = case
    position, reach = 100, 180
    x, table, pool, ring = state(case, position)
    low = lowered((paged_program if paged else ring_program)(case, reach_bound=bs * tl))
    print(f"reach {reach} from {position}, paged {paged}", flush=True)
    kw = {"table": table, "pool": pool} if paged else {"ring": ring}
    eng = run_gpu(device, kernels, low, x, position, reach=reach, **kw)
    try:
        cpu = run_cpu(low, x, position, reach=reach, **kw)
        assert compare(eng, cpu, low) == []
    finally:
        eng.close()
