"""Reductions across a threadgroup (src/FuryKernel/Reduce.hs): from
SIMD-group reductions and a threadgroup array of partials, and split-K's
combine.  Their order depends only on the thread count, the SIMD width and
the splits, never on the data or the threadgroup."""

from __future__ import annotations

from ..program.graph import F32
from .build import DIVERGENT, E, KernelBuilder, Tg, f32, max_e, simd_lane, simd_group_index, u32


def _tg_reduce(k: KernelBuilder, combine, simd_op, neutral: E, name: str, scratch: Tg, x: E) -> E:
    """Reduce.hs:55-85: each SIMD group's reduction into its slot; the first
    group's lane l folds slots l, l + w, ... from the identity and reduces
    once more; every thread reads the total; a last barrier frees scratch."""
    groups = k.simd_groups()
    if scratch.count < groups:
        k.note("threadgroup_memory", f"The scratch of reduction {name} has {scratch.count} slots for {groups} SIMD groups.")
    count = k.simd_group_count()
    width = k.simd_width()
    s = simd_op(name + "_simd", x)
    with k.when_lane(simd_lane.eq(0)):
        k.tg_store(scratch, simd_group_index, s)
    k.barrier()
    with k.when_simd(simd_group_index.eq(0)):
        acc = k.var(name + "_lane", neutral)
        with k.for_step(name + "_slot", simd_lane, count, width) as slot:
            k.assign(acc, combine(acc.get, k.tg_load(scratch, slot)))
        t = simd_op(name + "_group", acc.get)
        with k.when_lane(simd_lane.eq(0)):
            k.tg_store(scratch, 0, t)
    k.barrier()
    total = k.let(name, k.tg_load(scratch, 0))
    k.barrier()
    return total


def tg_reduce_sum(k: KernelBuilder, name: str, scratch: Tg, x: E) -> E:
    """The sum of x over the threadgroup, in every thread; slots summed from -0."""
    return _tg_reduce(k, lambda a, b: a + b, k.simd_sum, f32(-0.0), name, scratch, x)


def tg_reduce_max(k: KernelBuilder, name: str, scratch: Tg, x: E) -> E:
    """The maximum (maximumNumber) over the threadgroup; -inf over NaNs alone."""
    return _tg_reduce(k, max_e, k.simd_max, f32(float("-inf")), name, scratch, x)


def combine_splits(k: KernelBuilder, name: str, partials: Tg, splits: int, outputs: int, body) -> None:
    """Reduce.hs:96-125: after a barrier the threads take turns over the
    outputs, each output's partials added in split order, ((p0 + p1) + p2)
    + ..., the total handed to body(o, total) in a divergent region."""
    if splits == 0:
        k.note("threadgroup_memory", f"The partials of {name} come in no splits: a combine needs at least one.")
    if partials.count < splits * outputs:
        k.note("threadgroup_memory", f"The partials of {name} have {partials.count} slots for {outputs} outputs of {splits} splits.")
    k.barrier()
    with k.strided(name + "_output", outputs) as o:
        def part(q):
            return k.tg_load(partials, o * splits + q)
        acc = part(0)
        for q in range(1, max(1, splits)):
            acc = acc + part(q)
        total = k.let(name, acc)
        body(o, total)
