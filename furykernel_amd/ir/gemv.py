"""The reference's bf16 GEMV family (test/Test/FuryKernel/Gemv.hs:1-226) as
IR: y = W x for m rows of x, W [n, k] (out_in), all bf16, products
accumulated in f32, the shape and the variant (rows a SIMD group, threads,
pack width, split-K) baked into each kernel.

The order of each row's sum is fixed by the pack width and the split alone
(Gemv.hs:5-27): virtual lane q w + l of split q takes packs v, v + s w, ...;
each pack's elements go four at a time into one chain each as
((x0 w0 + x1 w1) + (x2 w2 + x3 w3)); a lane's chains are added in order,
then summed over the SIMD group; splits' partials are added in split order.
So every m, rows and thread count give a row the same bits."""

from __future__ import annotations

from dataclasses import dataclass

from ..program.graph import BF16, F32
from . import ir as I
from .build import KernelBuilder, TargetCaps, f32, group_index, narrow, quot, rem, simd_group_index, simd_lane, u32, widen
from .reduce import combine_splits

R, W = I.READ, I.WRITE


@dataclass(frozen=True)
class GemvShape:
    outputs: int
    inputs: int
    batch: int


@dataclass(frozen=True)
class GemvVariant:
    rows_per_simd: int
    threads: int
    pack: int
    split: int


def gemv(caps: TargetCaps, name: str, sh: "GemvShape", v: "GemvVariant"):
    """The kernel and the problems its builder noticed."""
    n, kk, m = sh.outputs, sh.inputs, sh.batch
    r, s = v.rows_per_simd, v.split
    width = caps.simd_width
    simds = v.threads // width
    row_groups = simds // s
    rows_per_group = row_groups * r
    per_group = rows_per_group * m
    packs = kk // v.pack
    chains = range(v.pack // 4)
    k = KernelBuilder(name, caps)
    x = k.buffer("x", R, BF16, m * kk)
    w = k.buffer("w", R, BF16, n * kk)
    y = k.buffer("y", W, BF16, m * n)
    k.threads(v.threads)
    k.groups(n // rows_per_group)
    partials = k.tg_array("partials", F32, s * per_group) if s > 1 else None
    if s == 1:
        split, row_group, lane = u32(0), simd_group_index, simd_lane
    else:
        split = k.let("split", rem(simd_group_index, s))
        row_group = k.let("row_group", quot(simd_group_index, s))
        lane = k.let("lane", split * width + simd_lane)
    row0 = k.let("row0", group_index * rows_per_group + row_group * r)
    accs = [[[k.var(f"acc{q}_{i}_{c}", f32(0.0)) for c in chains] for i in range(m)] for q in range(r)]
    with k.for_step("j", lane, packs, s * width) as j:
        xs = []
        for i in range(m):
            xp = k.load_pack(f"x{i}", v.pack, x, j if i == 0 else u32(i * packs) + j)
            xs.append([k.let(f"xf{i}_{e}", widen(F32, xe)) for e, xe in enumerate(xp)])
        for q in range(r):
            wp = k.load_pack(f"w{q}", v.pack, w, (row0 + q) * packs + j)
            ws = [k.let(f"wf{q}_{e}", widen(F32, we)) for e, we in enumerate(wp)]
            for xv, accs_i in zip(xs, accs[q]):
                for c, acc in zip(chains, accs_i):
                    def prod(o, c=c, xv=xv):
                        return xv[4 * c + o] * ws[4 * c + o]
                    k.assign(acc, acc.get + ((prod(0) + prod(1)) + (prod(2) + prod(3))))
    totals = []
    for q in range(r):
        row = []
        for i in range(m):
            terms = [a.get for a in accs[q][i]]
            e = terms[0]
            for t in terms[1:]:
                e = e + t
            row.append(k.simd_sum(f"total{q}_{i}", e))
        totals.append(row)
    if partials is None:
        with k.when_lane(simd_lane.eq(0)):
            for i in range(m):
                values = [narrow(BF16, totals[q][i]) for q in range(r)]
                if r == 1:
                    k.store(y, u32(i * n) + row0, values[0])
                else:
                    k.store_pack(y, u32(i * (n // r)) + group_index * row_groups + row_group, values)
    else:
        with k.when_lane(simd_lane.eq(0)):
            for q in range(r):
                for i in range(m):
                    k.tg_store(partials, ((row_group * r + q) * m + i) * s + split, totals[q][i])
        combine_splits(k, "total", partials, s, per_group,
                       lambda o, total: k.store(y, rem(o, m) * n + group_index * rows_per_group + quot(o, m),
                                                narrow(BF16, total)))
    return k.done()
