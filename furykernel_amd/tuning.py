"""Variant spaces of this target's GEMV families, their tuning on the GPU,
and the committed selections the lowering reads (src/FuryKernel/Variant.hs,
src/FuryKernel/Selection.hs; the GEMV axes of test/Test/FuryKernel/Gemv.hs:
93-99, rows a SIMD group, threads, pack, split-K).

Families:

* ``gemv_f32``, ``gemv_f16``, ``gemv_i8`` — the standalone matvec
  (``fk_gemv_<w>_<x>_r<R>``): axes rows a wavefront (r: 1, 2, 4) and
  threads (t: 64, 128, 256); classes n × k × m (m the batch, 1).  Pack and
  split-K, the reference's order axes, are fixed by these kernels (a pack of
  4 f32, 8 f16 or 16 i8 elements a lane load; no split), so no axis here
  decides a reduction's order: every variant of a class gives the same bits.
* ``step_gemv_f16``, ``step_gemv_bf16`` — the decode step's GEMV
  (``fk_step_gemv_<w>_k<K>_r<R>_p*_e*``): axes rows a block (r: 1, 2) and
  threadgroups a CU (g: 1 to 4, the grid's cap).  A class is a plain
  y = W x of n rows at input width k; its pick applies to every GEMV step
  launch of those rows and width whose prologue and epilogue take it.

Pruning keeps the reference's parallelism rule (at least twice as many
threadgroups as CUs), so the step family's classes are the ones whose rows
can fill 512 threadgroups of 8 wavefronts: the 1B model's gate/up pair
(16384 rows) and its logits (32000 rows).

Tuning times every kept variant of a class on the GPU over rotating copies of
its weights (past the 256 MB memory-side cache) and picks the fastest.  The
selections live in ``selections/<family>.json``; ``committed_chooser`` reads
and validates them, and a stale or invalid one is not used (the reason is
kept in ``chooser_problems``).
"""

from __future__ import annotations

import ctypes
import dataclasses
from pathlib import Path
from typing import Callable, Optional

from . import kernels as K
from .engine import _gemv_needs, params_struct
from .lower import (EPI_NONE, GEMV_THREADS, PRO_STORED, Launch as StepLaunch, LoweringError, _shape_gemv)
from .selection import Pick, Selection, SelectionError, TARGET, parse, render, validate
from .variant import Axis, Illegal, Launch, Profile, Space, point_value, shape_dim, shape_key, variants

SELECTIONS = Path(__file__).resolve().parent / "selections"
CORES = 256  # MI355X's CUs

GEMV_AXES = [Axis("rows_per_wave", "r", (1, 2, 4)), Axis("threads", "t", (64, 128, 256))]
STEP_AXES = [Axis("rows_per_block", "r", (1, 2)), Axis("groups_per_cu", "g", (1, 2, 3, 4))]

# The classes tuned: the standalone kernels' configurations, and the 1B
# decode step's GEMV shapes that pruning keeps.
GEMV_CLASSES = {"f32": [(4096, 4096)], "f16": [(4096, 4096)], "i8": [(8192, 8192)]}
STEP_CLASSES = {"f16": [(16384, 2048), (32000, 2048)], "bf16": [(16384, 2048), (32000, 2048)]}


def _cls(n: int, k: int) -> tuple:
    return (("n", n), ("k", k), ("m", 1))


# Standalone GEMV --------------------------------------------------------------

def gemv_space(wtype: str, classes: Optional[list] = None) -> Space:
    xtype = "f16" if wtype == "i8" else "f32"
    pack = K.GEMV_PACK[wtype]
    welt = {"f32": 4, "f16": 2, "i8": 1}[wtype]
    xelt = 2 if xtype == "f16" else 4

    def kernel(name, shape, point):
        n, k = shape_dim("n", shape), shape_dim("k", shape)
        r, t = point_value("r", point), point_value("t", point)
        entry = f"fk_gemv_{wtype}_{xtype}_r{r}"
        if entry not in K.ABIS:
            raise Illegal([f"{name}: no kernel {entry}."])
        per_group = t // 64 * r
        groups = -(-n // per_group)
        sizes = {"w": n * k * welt, "x": k * xelt, "y": n * 4, "scale": n * 4}
        return Launch(entry, groups, t, 0, bytes(K.GemvParams(n, k)),
                      tuple(sizes[b] for b in K.ABIS[entry].buffers))

    def divides(shape, point):
        n, k = shape_dim("n", shape), shape_dim("k", shape)
        per_group = point_value("t", point) // 64 * point_value("r", point)
        out = []
        if k % pack:
            out.append(f"k {k} is not a multiple of the pack width, {pack}.")
        if n % per_group:
            out.append(f"n {n} is not a multiple of the {per_group} rows of a threadgroup.")
        return out

    shapes = [_cls(n, k) for n, k in (GEMV_CLASSES[wtype] if classes is None else classes)]
    return Space(f"gemv_{wtype}", GEMV_AXES, shapes, ["m"], divides, kernel)


# Decode-step GEMV -------------------------------------------------------------

def _plain_step(wtype: str, n: int, k: int) -> StepLaunch:
    """y = W x as a GEMV step launch: one anchor of n rows, the row stored."""
    params = {"n_anchors": 1, "rows": [n, 0, 0], "first_row": [0, n, n, n], "k": k, "pro_mode": PRO_STORED,
              "seg": k, "eps": 0.0, "factor": 1.0, "gfactor": 1.0, "has_gamma": 0, "epi_mode": EPI_NONE,
              "store_tile": 1, "table_rows": 0, "blocks": 0, "arg_slots": 0}
    bind = {b: None for b in K.STEP_GEMV_BUFFERS}
    bind.update(w0="w0", y0="y0", src="src")
    return StepLaunch("plain", "", 0, GEMV_THREADS, bind, params, {"wtype": wtype}, 0)


def shape_step(launch: StepLaunch, compute_units: int, r: int, g: int) -> Optional[str]:
    """Reshapes a GEMV step launch (in place) to r rows a block and at most g
    threadgroups a CU; the reason it cannot take them, if so (the launch then
    keeps its shape)."""
    before = (launch.entry, launch.groups, launch.threads, launch.lds_bytes, dict(launch.params))
    try:
        _shape_gemv(launch, compute_units, rows=r, per_cu=g)
    except LoweringError as e:
        why = str(e)
    else:
        if K.gemv_entry(launch.entry)[3] == r:
            return None
        why = f"no GEMV step kernel of {r} rows a block at k = {launch.params['k']}"
    launch.entry, launch.groups, launch.threads, launch.lds_bytes = before[:4]
    launch.params.clear()
    launch.params.update(before[4])
    return why


def step_space(wtype: str, classes: Optional[list] = None, compute_units: int = CORES) -> Space:
    def kernel(name, shape, point):
        n, k = shape_dim("n", shape), shape_dim("k", shape)
        L = _plain_step(wtype, n, k)
        _shape_gemv(L, compute_units)
        why = shape_step(L, compute_units, point_value("r", point), point_value("g", point))
        if why:
            raise Illegal([f"{name}: {why}."])
        need = _gemv_needs(L)
        spans = tuple(need[b][0] if L.bind.get(b) else 0 for b in K.ABIS[L.entry].buffers)
        return Launch(L.entry, L.groups, L.threads, L.lds_bytes, bytes(params_struct(L)), spans)

    shapes = [_cls(n, k) for n, k in (STEP_CLASSES[wtype] if classes is None else classes)]
    return Space(f"step_gemv_{wtype}", STEP_AXES, shapes, ["m"], lambda s, p: [], kernel)


def step_class(launch: StepLaunch) -> tuple:
    """The class of a GEMV step launch: its rows, its input width, batch 1."""
    p = launch.params
    return _cls(p["first_row"][p["n_anchors"]], p["k"])


# Selections -------------------------------------------------------------------

def spaces(compute_units: int = CORES) -> list:
    return [gemv_space(w) for w in GEMV_CLASSES] + [step_space(w, compute_units=compute_units)
                                                     for w in STEP_CLASSES]


def load(family: str) -> Optional[Selection]:
    path = SELECTIONS / f"{family}.json"
    return parse(path.read_text()) if path.exists() else None


chooser_problems: dict = {}


def validated(compute_units: int = CORES) -> dict:
    """Every committed selection that validates, as family -> {class key:
    point}; the problems of those that don't in ``chooser_problems``."""
    out = {}
    chooser_problems.clear()
    profile = Profile(compute_units)
    for space in spaces(compute_units):
        try:
            sel = load(space.family)
        except SelectionError as e:
            chooser_problems[space.family] = e.problems
            continue
        if sel is None:
            continue
        try:
            picked = validate(profile, space, sel)
        except SelectionError as e:
            chooser_problems[space.family] = e.problems
            continue
        out[space.family] = {shape_key(v.shape): v.point for v in picked}
    return out


def committed_chooser(compute_units: int = CORES) -> Callable[[StepLaunch], Optional[tuple]]:
    """For the lowering: a GEMV step launch's (rows a block, threadgroups a CU)
    as the committed, valid selection of its family picks them, or None."""
    picks = validated(compute_units)

    def choose(launch: StepLaunch) -> Optional[tuple]:
        fam = picks.get(f"step_gemv_{launch.meta.get('wtype')}")
        point = fam.get(shape_key(step_class(launch))) if fam else None
        return None if point is None else (point_value("r", point), point_value("g", point))

    return choose


def gemv_pick(wtype: str, n: int, k: int, compute_units: int = CORES) -> Optional[tuple]:
    """The committed (rows a wavefront, threads) of a standalone GEMV class."""
    fam = validated(compute_units).get(f"gemv_{wtype}")
    point = fam.get(shape_key(_cls(n, k))) if fam else None
    return None if point is None else (point_value("r", point), point_value("t", point))


# Tuning (on the GPU) ----------------------------------------------------------

COPY_BYTES = 512 << 20  # past the memory-side cache


def _timer(device, ks: K.Kernels, space: Space, shape: tuple, reps: int = 20) -> Callable:
    """Times a variant's launch of the class over rotating copies of its
    largest buffer (its weights), the rest shared; microseconds a launch."""
    from . import runtime
    probe = space.kernel("probe", shape, variants(Profile(CORES), space, shape)[0].point)
    sizes = list(probe.spans)
    big = max(range(len(sizes)), key=lambda i: sizes[i])
    copies = max(2, -(-COPY_BYTES // sizes[big]))
    bufs = [device.alloc(max(s, 256)) if s else None for s in sizes]
    heavy = [device.alloc(sizes[big]) for _ in range(copies)]
    for i, h in enumerate(heavy):
        ks.fill_u32(h, 0x3c003c00 ^ (i * 0x00010001), sizes[big] // 4)
    for b, s in zip(bufs, sizes):
        if b is not None:
            ks.fill_u32(b, 0x3c003c00, max(s, 256) // 4)  # small finite values in every type read
    device.sync()

    def run(v) -> float:
        L = v.launch
        fn = ks.fn(L.entry)
        args = []
        for h in heavy:
            ptrs = [(h if i == big else b).ptr if s else 0 for i, (b, s) in enumerate(zip(bufs, sizes))]
            spans = [(p, s) for p, s in zip(ptrs, sizes)]
            params = (ctypes.c_uint8 * len(L.params)).from_buffer_copy(L.params)
            runtime.launch_check(L.entry, L.groups, L.threads, L.lds_bytes, spans, params)
            args.append(b"".join(p.to_bytes(8, "little") for p in ptrs) + L.params)
        for a in args:
            fn.launch(L.groups, L.threads, a, L.lds_bytes)
        device.sync()
        s, e = device.event(), device.event()
        s.record()
        for _ in range(reps):
            for a in args:
                fn.launch(L.groups, L.threads, a, L.lds_bytes)
        e.record()
        e.synchronize()
        return s.elapsed_ms(e) * 1e3 / (reps * len(args))

    def free():
        for b in bufs + heavy:
            if b is not None:
                b.free()

    run.free = free
    return run


def tune(device, ks: K.Kernels, space: Space, compute_units: int = CORES, log=print) -> Selection:
    """Times every kept variant of every class and picks the fastest."""
    profile = Profile(compute_units)
    sel = Selection(space.family, TARGET, profile, {})
    for shape in space.shapes:
        vs = variants(profile, space, shape)
        if not vs:
            raise SelectionError([f"The class {shape_key(shape)} of {space.family} keeps no variant."])
        timer = _timer(device, ks, space, shape)
        try:
            timed = []
            for v in vs:
                us = timer(v)
                timed.append((us, v))
                log(f"{space.family} {shape_key(shape)} {dataclasses.astuple(v.launch)[0]} "
                    f"x_{'_'.join(f'{p}{x}' for p, x in v.point)}: {us:.2f} us ({v.groups} groups)")
            us, best = min(timed, key=lambda t: t[0])
            sel.classes[shape_key(shape)] = Pick("_".join(f"{p}{x}" for p, x in best.point), best.ir_hash)
        finally:
            timer.free()
    return sel


def write(sel: Selection, directory: Path = SELECTIONS) -> Path:
    directory.mkdir(parents=True, exist_ok=True)
    path = directory / f"{sel.family}.json"
    path.write_text(render(sel))
    return path


def main(argv=None) -> int:
    """python -m furykernel_amd.tuning [family ...]: tunes the families (all
    by default) on GPU 0 and writes their selections."""
    import argparse
    import sys
    from . import runtime
    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("families", nargs="*")
    ap.add_argument("--dry-run", action="store_true", help="time and print, write nothing")
    ap.add_argument("--out", type=Path, default=SELECTIONS, help="where to write the selections")
    args = ap.parse_args(argv)
    device = runtime.Device(0)
    cus = device.info.compute_units
    ks = K.Kernels(device)
    for space in spaces(cus):
        if args.families and space.family not in args.families:
            continue
        sel = tune(device, ks, space, cus, log=lambda s: print(s, flush=True))
        print(render(sel), end="", flush=True)
        if not args.dry_run:
            print(f"wrote {write(sel, args.out)}", flush=True)
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
