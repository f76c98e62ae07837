"""The program gate (src/FuryKernel/Program/Check.hs).

``check_program`` returns a ``CheckedProgram`` or the findings: ids unique and
increasing in program order, every value made by one node and every cache
stored into by one; every operation's values and sources of the shapes and
types it takes; rows and caches of at least one element; weights of a float
type; finite parameters; every index below what it indexes; and names that
generated code can carry.  The planner and the engine take only checked
programs.
"""

from __future__ import annotations

import math
import re
from dataclasses import dataclass, field
from typing import Optional

from .graph import (
    BF16, F16, F32, U32, Add, ArgMax, Attend, CombineRanks, Concat, GatedGelu, Gather, GeluMul, Input, KvStore, Linear,
    LinearRouted, Paged, Program, Ring, RmsNorm, Rope, Route, SCache, ScaleBy, Shape, SInput, Softcap, SRowInts,
    STable, Standardize, SWeight, op_sources, op_values, segment_count, whole_row)

# Finding rules (src/FuryKernel/Finding.hs), the ones the program gate uses.
STRUCTURE, SHAPES, BOUNDS, NAMES = "Structure", "Shapes", "Bounds", "Names"


@dataclass(frozen=True)
class Location:
    program: str
    nodes: tuple = ()


@dataclass(frozen=True)
class Finding:
    rule: str
    message: str
    location: Optional[Location] = None

    def unplaced(self) -> "Finding":
        return Finding(self.rule, self.message, None)


class ProgramRefused(ValueError):
    def __init__(self, findings: list[Finding]):
        super().__init__("; ".join(f.message for f in findings))
        self.findings = findings


class CheckedProgram:
    """A program that passed the gate; only ``check_program`` makes one."""

    __slots__ = ("program",)

    def __init__(self, program: Program, _token=None):
        if _token is not _TOKEN:
            raise TypeError("a CheckedProgram comes from check_program")
        self.program = program


_TOKEN = object()

# Words the target languages reserve (C++, HIP's builtins, the shading
# languages' scalar and vector names) and prefixes generated code keeps.
_KEYWORDS = set("""
alignas alignof and and_eq asm auto bitand bitor bool break case catch char char8_t char16_t char32_t class compl
concept const consteval constexpr constinit const_cast continue co_await co_return co_yield decltype default delete do
double dynamic_cast else enum explicit export extern false float for friend goto if inline int long mutable namespace
new noexcept not not_eq nullptr operator or or_eq private protected public register reinterpret_cast requires return
short signed sizeof static static_assert static_cast struct switch template this thread_local throw true try typedef
typeid typename union unsigned using virtual void volatile wchar_t while xor xor_eq
threadIdx blockIdx blockDim gridDim warpSize half uint ushort uchar ulong size_t ptrdiff_t main kernel device
constant global local max min fma select self Self super crate None Some Ok Err NAN INFINITY
""".split())
_VECTOR_BASES = ("float", "half", "int", "uint", "short", "ushort", "char", "uchar", "bool", "long", "ulong",
                 "bfloat", "double")


def name_problem(n: str) -> Optional[str]:
    """What is wrong with a name in generated code (src/FuryKernel/Check.hs:288-311)."""
    if not n:
        return "An empty name."
    if not re.fullmatch(r"[A-Za-z_][A-Za-z0-9_]*", n):
        return f"The name {n} is not an identifier: use letters, digits and underscores."
    if n.startswith("_"):
        return f"The name {n} starts with an underscore, which C++ reserves."
    if "__" in n:
        return f"The name {n} holds two underscores in a row, which C++ reserves."
    if n.lower().startswith("fk_"):
        return f"The name {n} starts with fk_ in some case, which generated code reserves."
    vector = any(n.startswith(b) and re.fullmatch(r"[234](x[234])?", n[len(b):]) for b in _VECTOR_BASES)
    if n in _KEYWORDS or vector:
        return f"The name {n} is reserved in a target language."
    return None


def _finite(v: float) -> bool:
    return not (math.isnan(v) or math.isinf(v))


def check_program(p: Program) -> CheckedProgram:
    """The gate: a ``CheckedProgram``, or ``ProgramRefused`` with the findings."""
    fs = findings_of(p)
    if fs:
        raise ProgramRefused(fs)
    return CheckedProgram(p, _TOKEN)


def findings_of(p: Program) -> list[Finding]:
    out = _names(p) + _structure(p) + _row_bounds(p) + _layouts(p) + _element_types(p) + _Shapes(p).run()
    return [f if f.location is not None else Finding(f.rule, f.message, Location(p.name, ())) for f in out]


def _structure(p: Program) -> list[Finding]:
    out: list[Finding] = []

    def increasing(what: str, ids: list[int]):
        for a, b in zip(ids, ids[1:]):
            if a >= b:
                out.append(Finding(STRUCTURE, f"The {what} ids don't increase in program order: {a}, then {b}."))
                return

    increasing("source", [s.id for s in p.sources])
    increasing("value", [v.id for v in p.values])
    increasing("node", [n.id for n in p.nodes])
    for v in p.values:
        c = sum(1 for n in p.nodes if v.id in n.outputs)
        if c != 1:
            what = "no node" if c == 0 else "one node" if c == 1 else f"{c} nodes"
            out.append(Finding(STRUCTURE, f"The value {v.name} is made by {what}."))
    stores: dict[int, list] = {}
    for n in p.nodes:
        if isinstance(n.op, KvStore):
            stores.setdefault(n.op.at.cache, []).append(n)
    for c in sorted(stores):
        first, *others = stores[c]
        src = p.source(c)
        for again in others:
            out.append(Finding(STRUCTURE, f"{again.name} stores into {src.name if src else 'a cache'}, which "
                                          f"{first.name} already does: a program stores into a cache once."))
    return out


def _layouts(p: Program) -> list[Finding]:
    out = []
    for s in p.sources:
        if not isinstance(s.kind, SCache):
            continue
        lay = s.kind.layout
        if isinstance(lay, Ring):
            fields = [("0 slots", lay.slots), ("0 heads", lay.kv_heads), ("a length of 0", lay.length),
                      ("a head dimension of 0", lay.head_dim)]
        else:
            fields = [("0 blocks", lay.blocks), ("a block size of 0", lay.block_size), ("0 heads", lay.kv_heads),
                      ("a head dimension of 0", lay.head_dim)]
        out += [Finding(SHAPES, f"The cache {s.name} has {what}.") for what, v in fields if v == 0]
    return out


def _element_types(p: Program) -> list[Finding]:
    out = []
    for s in p.sources:
        k = s.kind
        if isinstance(k, (SWeight, STable)):
            what = "weight" if isinstance(k, SWeight) else "table"
            if k.type not in (BF16, F16, F32):
                out.append(Finding(SHAPES, f"The {what} {s.name} holds {k.type}, not bf16, f16 or f32."))
    for s in p.sources:
        k = s.kind
        if isinstance(k, (SWeight, STable)) and not k.layout:
            what = "weight" if isinstance(k, SWeight) else "table"
            out.append(Finding(SHAPES, f"The {what} {s.name} names no layout."))
    return out


def _names(p: Program) -> list[Finding]:
    input_values = {n.outputs[0] for n in p.nodes if isinstance(n.op, Input) and n.outputs}
    everything = ([s.name for s in p.sources] + [v.name for v in p.values if v.id not in input_values]
                  + [n.name for n in p.nodes if not n.outputs])
    out = []
    for n in [p.name] + everything + [o.name for o in p.outputs]:
        m = name_problem(n)
        if m:
            out.append(Finding(NAMES, m))
    if "_x_" in p.name:
        out.append(Finding(NAMES, f"The program's name {p.name} holds _x_, which joins it to its steps' names."))
    counts: dict[str, int] = {}
    for n in everything:
        counts[n] = counts.get(n, 0) + 1
    out += [Finding(NAMES, f"The name {n} is used {c} times.") for n, c in sorted(counts.items()) if c > 1]
    oc: dict[str, int] = {}
    for o in p.outputs:
        oc[o.name] = oc.get(o.name, 0) + 1
    out += [Finding(NAMES, f"The output {n} is named {c} times.") for n, c in sorted(oc.items()) if c > 1]
    return out


def _row_bounds(p: Program) -> list[Finding]:
    return [Finding(BOUNDS, f"The bound of {s.name}, 0, admits no value.")
            for s in p.sources if isinstance(s.kind, SRowInts) and s.kind.bound == 0]


def _weight2(s) -> Optional[tuple[int, int]]:
    if isinstance(s.kind, SWeight) and len(s.kind.dims) == 2:
        return s.kind.dims[0], s.kind.dims[1]
    return None


def _weight1(s) -> Optional[int]:
    if isinstance(s.kind, SWeight) and len(s.kind.dims) == 1:
        return s.kind.dims[0]
    return None


def _row_count(s) -> Optional[int]:
    return s.kind.count if isinstance(s.kind, SRowInts) else None


def _shape_text(sh: Shape) -> str:
    return f"[{sh.width}/{sh.segment}]"


@dataclass
class _Shapes:
    """Shapes, types and indices, node by node (Check.hs:180-421)."""

    p: Program
    made: dict = field(default_factory=dict)
    findings: list = field(default_factory=list)
    place: tuple = ()

    def run(self) -> list[Finding]:
        self.sources = {s.id: s for s in self.p.sources}
        self.values = {v.id: v for v in self.p.values}
        for n in self.p.nodes:
            self.node(n)
        self.place = ()
        for o in self.p.outputs:
            if o.value not in self.made:
                self.bad(f"The output {o.name} names no value of the program.")
        return self.findings

    def finding(self, rule: str, m: str) -> None:
        self.findings.append(Finding(rule, m, Location(self.p.name, self.place)))

    def bad(self, m: str) -> None:
        self.finding(SHAPES, m)

    def id_bound(self, v: int) -> Optional[int]:
        prod = self.p.producer(v)
        if prod is not None and isinstance(prod.op, (Route, ArgMax)):
            x = self.values.get(prod.op.x)
            return None if x is None else x.shape.width
        return None

    def node(self, n) -> None:
        self.place = (n.name,)
        ins = []
        for v in op_values(n.op):
            m = self.made.get(v)
            if m is None:
                self.bad(f"{n.name} reads a value no earlier node makes.")
            ins.append(m)
        srcs = []
        for s in op_sources(n.op):
            m = self.sources.get(s)
            if m is None:
                self.bad(f"{n.name} reads a source the program doesn't have.")
            srcs.append(m)
        outs = [self.values.get(v) for v in n.outputs]
        if any(o is None for o in outs):
            self.finding(STRUCTURE, f"{n.name} makes a value the program doesn't list.")
        if not (any(x is None for x in ins) or any(x is None for x in srcs) or any(o is None for o in outs)):
            self.op(n, ins, srcs, outs)
        for v in n.outputs:
            if v in self.values:
                self.made[v] = self.values[v]

    def op(self, n, ins, srcs, outs) -> None:
        op = n.op

        def expect(ok: bool, what: str) -> None:
            if not ok:
                self.bad(f"{n.name}: {what}.")

        def within(ok: bool, what: str) -> None:
            if not ok:
                self.finding(BOUNDS, f"{n.name}: {what}.")

        def f32(v) -> None:
            expect(v.type == F32, f"{v.name} is {v.type}, not f32")

        def u32(v) -> None:
            expect(v.type == U32, f"{v.name} is {v.type}, not u32")

        def whole(v) -> None:
            expect(v.shape.segment == v.shape.width, f"{v.name} is in segments")

        def shaped(o, sh: Shape, t: str) -> None:
            if o.shape != sh or o.type != t:
                self.bad(f"{n.name}: {o.name} should be {_shape_text(sh)} {t}.")
            elif sh.width == 0:
                self.bad(f"{n.name}: {o.name} is {_shape_text(sh)}, a row of no elements.")
            elif sh.segment == 0 or sh.width % sh.segment != 0:
                self.bad(f"{n.name}: {o.name} is {_shape_text(sh)}, its segments not dividing its row.")

        def row_ints1(s) -> None:
            expect(_row_count(s) == 1, f"{s.name} is not one u32 per row")

        def bounded(s, limit: int, what: str) -> None:
            if isinstance(s.kind, SRowInts):
                within(s.kind.bound <= limit, f"the bound of {s.name}, {s.kind.bound}, is more than {what}")

        def is_row_ints(k) -> bool:
            return isinstance(k, SRowInts) and k.count > 0

        def sequence_source(c, layout, s) -> None:
            if isinstance(layout, Ring):
                row_ints1(s)
                bounded(s, layout.slots, f"the {layout.slots} slots of {c.name}")
            else:
                expect(is_row_ints(s.kind), f"{s.name} is not a block table")
                bounded(s, layout.blocks, f"the {layout.blocks} blocks of {c.name}")

        def positions(layout, s, pos) -> None:
            k = _row_count(s)
            if isinstance(layout, Paged) and k is not None:
                bounded(pos, k * layout.block_size, f"the {k * layout.block_size} positions of its block table")

        if isinstance(op, Input):
            if len(ins) == 0 and len(srcs) == 1 and isinstance(srcs[0].kind, SInput) and len(outs) == 1:
                shaped(outs[0], srcs[0].kind.shape, srcs[0].kind.type)
            else:
                expect(False, "it reads a source that isn't an input")
        elif isinstance(op, Linear) and len(ins) == 1 and len(srcs) == 1 and len(outs) == 1:
            x, w, o = ins[0], srcs[0], outs[0]
            wd = _weight2(w)
            if wd is None:
                expect(False, f"{w.name} is not a two-dimensional weight")
            else:
                rows, cols = wd
                f32(x)
                expect(x.shape.width == cols,
                       f"its input has {x.shape.width} elements for a weight of {cols} columns")
                expect(op.segment > 0 and rows % op.segment == 0,
                       f"its segments of {op.segment} don't divide its {rows} outputs")
                shaped(o, Shape(rows, op.segment), F32)
        elif isinstance(op, LinearRouted) and len(ins) == 2 and len(srcs) == 1 and len(outs) == 1:
            ids, x = ins
            t, o = srcs[0], outs[0]
            if isinstance(t.kind, STable) and len(t.kind.dims) == 2:
                rows, cols = t.kind.dims
                u32(ids)
                f32(x)
                ranks = ids.shape.width
                expect(x.shape == whole_row(cols) or x.shape == Shape(ranks * cols, cols),
                       f"its input is neither one segment of {cols} nor one per rank")
                b = self.id_bound(ids.id)
                if b is not None:
                    within(b <= t.kind.entries,
                           f"the bound of its ids, {b}, is more than the {t.kind.entries} entries of {t.name}")
                else:
                    within(False, "nothing bounds its ids, which are neither a route's nor an argmax's")
                shaped(o, Shape(ranks * rows, rows), F32)
            else:
                expect(False, f"{t.name} is not a table of two-dimensional weights")
        elif isinstance(op, RmsNorm) and len(ins) == 1 and len(outs) == 1:
            x, o = ins[0], outs[0]
            f32(x)
            expect(op.eps > 0 and _finite(op.eps), "its epsilon isn't positive and finite")
            expect(_finite(op.factor), "its factor isn't finite")
            for gamma in srcs:
                expect(_weight1(gamma) == x.shape.segment, f"{gamma.name} is not a weight as wide as a segment")
            shaped(o, x.shape, F32)
        elif isinstance(op, Add) and len(ins) == 2 and not srcs and len(outs) == 1:
            a, b = ins
            f32(a)
            f32(b)
            expect(a.shape == b.shape, "its operands have different shapes")
            shaped(outs[0], a.shape, F32)
        elif isinstance(op, Concat) and len(ins) == 2 and not srcs and len(outs) == 1:
            a, b = ins
            f32(a)
            f32(b)
            expect(a.shape.segment == b.shape.segment, "its operands' segments differ")
            shaped(outs[0], Shape(a.shape.width + b.shape.width, a.shape.segment), F32)
        elif isinstance(op, ScaleBy) and len(ins) == 1 and len(srcs) == 1 and len(outs) == 1:
            f32(ins[0])
            expect(_weight1(srcs[0]) == 1, f"{srcs[0].name} is not a weight of one element")
            shaped(outs[0], ins[0].shape, F32)
        elif isinstance(op, GatedGelu) and len(ins) == 1 and not srcs and len(outs) == 1:
            x = ins[0]
            f32(x)
            expect(x.shape.segment % 2 == 0, "its segments have no halves")
            shaped(outs[0], Shape(x.shape.width // 2, x.shape.segment // 2), F32)
        elif isinstance(op, GeluMul) and len(ins) == 2 and not srcs and len(outs) == 1:
            a, b = ins
            f32(a)
            f32(b)
            expect(a.shape == b.shape, "its operands have different shapes")
            shaped(outs[0], a.shape, F32)
        elif isinstance(op, Rope) and len(ins) == 1 and len(srcs) == 1 and len(outs) == 1:
            x, pos, r = ins[0], srcs[0], op.spec
            f32(x)
            expect(r.axes > 0, "it has no axes")
            expect(_row_count(pos) == r.axes, f"{pos.name} is not {r.axes} u32 per row, a position an axis")
            expect(x.shape.segment % (2 * max(1, r.axes)) == 0, "its heads have no halves for each axis")
            expect(2 * r.axes * r.rotated <= x.shape.segment, "it rotates more pairs than a head has")
            expect(r.theta > 0 and _finite(r.theta), "its theta isn't positive and finite")
            shaped(outs[0], x.shape, F32)
        elif isinstance(op, Softcap) and len(ins) == 1 and not srcs and len(outs) == 1:
            f32(ins[0])
            expect(op.cap > 0 and _finite(op.cap), "its cap isn't positive and finite")
            shaped(outs[0], ins[0].shape, F32)
        elif isinstance(op, Route) and len(ins) == 1 and len(outs) == 2:
            x, (ids, ws) = ins[0], outs
            f32(x)
            whole(x)
            expect(0 < op.spec.k <= x.shape.width, f"it takes {op.spec.k} of {x.shape.width} logits")
            for s in srcs:
                expect(_weight1(s) == x.shape.width, f"{s.name} is not a weight with a scale per expert")
            shaped(ids, whole_row(op.spec.k), U32)
            shaped(ws, whole_row(op.spec.k), F32)
        elif isinstance(op, CombineRanks) and len(ins) == 2 and not srcs and len(outs) == 1:
            w, x = ins
            f32(w)
            f32(x)
            whole(w)
            expect(segment_count(x.shape) == w.shape.width, "its weights don't match its value's segments")
            shaped(outs[0], whole_row(x.shape.segment), F32)
        elif isinstance(op, KvStore) and len(ins) == 1 and len(srcs) == 3 and not outs:
            x, (c, pos, slot) = ins[0], srcs
            if isinstance(c.kind, SCache):
                lay = c.kind.layout
                f32(x)
                row_ints1(pos)
                sequence_source(c, lay, slot)
                positions(lay, slot, pos)
                expect(x.shape == Shape(lay.kv_heads * lay.head_dim, lay.head_dim),
                       f"its value isn't the {lay.kv_heads} heads of {lay.head_dim} of {c.name}")
            else:
                expect(False, f"{c.name} is not a cache")
        elif isinstance(op, Attend) and len(ins) == 1 and len(srcs) >= 4 and len(outs) == 1:
            q, o = ins[0], outs[0]
            k, v, pos, slot, *reach = srcs
            a = op.spec
            if isinstance(k.kind, SCache) and isinstance(v.kind, SCache):
                kl, vl = k.kind.layout, v.kind.layout
                f32(q)
                row_ints1(pos)
                for r in reach:
                    row_ints1(r)
                expect(len(reach) == (0 if a.reach is None else 1),
                       "its sources aren't a cache's, a position's, a sequence's and its reach's")
                sequence_source(k, kl, slot)
                for pr in [pos] + reach:
                    positions(kl, slot, pr)
                expect(kl == vl, "its key and value caches are laid out differently")
                expect(a.heads > 0, "it has no query heads")
                expect(a.kv_heads > 0 and a.heads % a.kv_heads == 0,
                       "its query heads don't share its key and value heads evenly")
                expect(kl.kv_heads == a.kv_heads and kl.head_dim == a.head_dim,
                       "its caches don't hold its key and value heads")
                expect(q.shape == Shape(a.heads * a.head_dim, a.head_dim), "its queries aren't its heads")
                expect(a.window is None or a.window > 0, "its window is empty")
                expect(a.scale > 0 and _finite(a.scale), "its scale isn't positive and finite")
                self.ring_fit(n, k, kl, a, pos, reach, within)
                shaped(o, q.shape, F32)
            else:
                expect(False, "it reads keys or values from something that isn't a cache")
        elif isinstance(op, Gather) and not ins and len(srcs) == 2 and len(outs) == 1:
            t, tok = srcs
            wd = _weight2(t)
            if wd is None:
                expect(False, f"{t.name} is not a two-dimensional weight")
            else:
                rows, cols = wd
                expect(_finite(op.factor), "its factor isn't finite")
                expect(is_row_ints(tok.kind), f"{tok.name} is not u32 per row")
                bounded(tok, rows, f"the {rows} rows of {t.name}")
                shaped(outs[0], whole_row(cols), F32)
        elif isinstance(op, Standardize) and len(ins) == 1 and len(srcs) == 2 and len(outs) == 1:
            x, (b, s) = ins[0], srcs
            f32(x)
            expect(_finite(op.factor), "its factor isn't finite")
            expect(_weight1(b) == x.shape.width, f"{b.name} is not a weight a row wide")
            expect(_weight1(s) == x.shape.width, f"{s.name} is not a weight a row wide")
            shaped(outs[0], x.shape, F32)
        elif isinstance(op, ArgMax) and len(ins) == 1 and not srcs and len(outs) == 1:
            f32(ins[0])
            whole(ins[0])
            shaped(outs[0], whole_row(1), U32)
        else:
            expect(False, "it has the wrong number of values or sources")

    @staticmethod
    def ring_fit(n, c, layout, a, pos, reach, within) -> None:
        """Attention over a ring reads no more positions than it holds (Check.hs:346-381)."""
        if not isinstance(layout, Ring):
            return
        length = layout.length
        holds = f", more than the {length} that {c.name}'s ring holds"

        def bound_of(s):
            return s.kind.bound if isinstance(s.kind, SRowInts) else None

        if a.window is not None and a.reach is None:
            within(a.window <= length, f"its window of {a.window} positions is longer than the {length} that "
                                       f"{c.name}'s ring holds")
        elif a.window is not None and a.reach is not None and len(reach) == 1 and bound_of(reach[0]) is not None:
            rb = bound_of(reach[0])
            spanned = min(a.window + a.reach.ahead, max(a.window, rb))
            within(spanned <= length, f"its window of {a.window} and its reach of up to {a.reach.ahead} past a "
                                      f"row's own position read {spanned} positions{holds}")
        elif a.window is None and a.reach is None and bound_of(pos) is not None:
            b = bound_of(pos)
            within(b <= length, f"with no window it reads every position below the bound of {pos.name}, {b}{holds}")
        elif (a.window is None and a.reach is not None and len(reach) == 1 and bound_of(pos) is not None
              and bound_of(reach[0]) is not None):
            b, rb = bound_of(pos), bound_of(reach[0])
            below = max(b, min(b + a.reach.ahead, rb))
            within(below <= length, f"with no window, and a reach of up to {a.reach.ahead} past a row's own "
                                    f"position, it reads every position below {below}{holds}")
