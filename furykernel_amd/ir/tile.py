"""A threadgroup's tile of C = A · Bᵀ (src/FuryKernel/Tile.hs:76-168): the
operands staged in threadgroup memory step by step, multiplied as 8×8 f32
fragments, each element summed over k in order, eight at a time; the results
handed back through a small threadgroup array, element by element."""

from __future__ import annotations

from dataclasses import dataclass

from ..program.graph import F32
from . import ir as I
from .build import E, KernelBuilder, Tg, quot, rem, simd_group_index, simd_lane, u32


@dataclass(frozen=True)
class GemmTile:
    rows: int
    cols: int
    step: int
    group_rows: int


def gemm_tile(k: KernelBuilder, name: str, t: GemmTile, a: Tg, b: Tg, c: Tg, kdim: E, a_run, b_run, element) -> None:
    """a_run(row, k) -> 4 f32 elements of A from k on; b_run(col, k) -> 8 of
    B; element(row, col, value) takes each result once, by some lane."""
    groups = k.simd_groups()
    k_multiple = k.known_multiple(kdim)
    width = k.simd_width()
    group_cols = groups // max(1, t.group_rows)
    sub_rows = t.rows // max(1, t.group_rows)
    sub_cols = t.cols // max(1, group_cols)
    frag_rows, frag_cols = sub_rows // 8, sub_cols // 8
    per_round = c.count // max(1, groups * 64)
    broken = []
    if not (t.step > 0 and t.step % 8 == 0):
        broken.append(f"its step, {t.step}, is not a positive multiple of 8")
    if not (t.group_rows > 0 and groups % t.group_rows == 0):
        broken.append(f"{groups} SIMD groups don't share {t.group_rows} rows of groups")
    if not (sub_rows > 0 and sub_cols > 0 and sub_rows * t.group_rows == t.rows and sub_cols * group_cols == t.cols
            and sub_rows % 8 == 0 and sub_cols % 8 == 0):
        broken.append(f"its {t.rows} × {t.cols} don't divide into the SIMD groups' blocks of 8×8 fragments")
    if not ((a.count, b.count) == (t.rows * t.step, t.cols * t.step) and per_round > 0 and c.count % (groups * 64) == 0):
        broken.append(f"its arrays hold ({a.count},{b.count},{c.count}) elements")
    if k_multiple is None or k_multiple % t.step:
        if isinstance(kdim.ir, I.EParam) and k_multiple is not None:
            what = f"the dimension {kdim.ir.name} declared a multiple of {k_multiple}"
        elif k_multiple is not None:
            what = str(k_multiple)
        else:
            what = I.render_expr(kdim.ir) + ", neither a literal nor a dimension"
        broken.append(f"k, {what}, is not known to be a multiple of its step, {t.step}")
    if broken:
        k.note("threadgroup_memory", f"The tile {name}: {broken[0]}.")
        return
    step = u32(t.step)
    group_row = k.let(name + "_group_row", quot(simd_group_index, group_cols))
    group_col = k.let(name + "_group_col", rem(simd_group_index, group_cols))
    accs = [((i, j), k.fragment(f"{name}_acc{i}_{j}", F32)) for i in range(frag_rows) for j in range(frag_cols)]
    as_ = [k.fragment(f"{name}_a{i}", F32) for i in range(frag_rows)]
    bs = [k.fragment(f"{name}_b{j}", F32) for j in range(frag_cols)]
    with k.for_u(name + "_step", 0, quot(kdim, step)) as s:
        with k.strided(name + "_stage_a", t.rows * t.step // 4) as e:
            row = quot(e, t.step // 4)
            at = s * step + rem(e, t.step // 4) * 4
            vs = a_run(row, at)
            _run_of(k, name, 4, vs, lambda: k.tg_store_pack(a, e, vs))
        with k.strided(name + "_stage_b", t.cols * t.step // 8) as e:
            col = quot(e, t.step // 8)
            at = s * step + rem(e, t.step // 8) * 8
            vs = b_run(col, at)

            def stage():
                k.tg_store_pack(b, e * 2, vs[:4])
                k.tg_store_pack(b, e * 2 + 1, vs[4:])
            _run_of(k, name, 8, vs, stage)
        k.barrier()
        for kk in range(0, t.step, 8):
            for i, fa in enumerate(as_):
                k.frag_load_tg(fa, a, (group_row * sub_rows + 8 * i) * step + kk, step)
            for j, fb in enumerate(bs):
                k.frag_load_tg_t(fb, b, (group_col * sub_cols + 8 * j) * step + kk, step)
            for (i, j), acc in accs:
                k.frag_mma(acc, as_[i], bs[j], acc)
        k.barrier()
    rounds = [accs[x:x + max(1, per_round)] for x in range(0, len(accs), max(1, per_round))]
    for these in rounds:
        for slot, (_, acc) in enumerate(these):
            k.frag_store_tg(c, (simd_group_index * per_round + slot) * 64, 8, acc)
        k.simd_barrier()
        for slot, ((i, j), _) in enumerate(these):
            with k.for_step(name + "_element", simd_lane, 64, width) as e:
                row = group_row * sub_rows + 8 * i + quot(e, 8)
                col = group_col * sub_cols + 8 * j + rem(e, 8)
                element(row, col, k.tg_load(c, (simd_group_index * per_round + slot) * 64 + e))
        k.simd_barrier()


def _run_of(k: KernelBuilder, name: str, n: int, vs: list, ok) -> None:
    if len(vs) == n:
        ok()
    else:
        k.note("typing", f"The tile {name}: a run of {len(vs)} elements, not {n}.")
