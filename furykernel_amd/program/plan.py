"""The planner (src/FuryKernel/Program/Plan.hs): a checked program as steps,
each one kernel launch, and the cut points where steps meet.

No threadgroup can wait for another inside a kernel, so a value is stored once
the step that writes it has finished.  Anchors (linear layers, attention) set
a step's grid; recomputed operations run in every threadgroup before them;
epilogues run on a linear layer's tile; light steps hold cache stores,
attention's combine and outputs no anchor computes; stores into a ring without
room for a step's rows of one sequence are staged and land after the last
attention reading the ring.

This module restates the reference's planner rule for rule (``plan`` below
follows ``plan`` at Plan.hs:314, ``anchor`` at :530, ``light`` at :614,
``effect`` at :672, ``closeOpen`` at :367, ``chain`` at :448), so that the
engine runs the launches the reference would plan.  One addition: a SiLU
``GeluMul`` is a GELU to the ``store_gelus`` option, the same trade-off.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

from .check import CheckedProgram
from .graph import (
    Attend, F32, Gather, GatedGelu, GeluMul, Input, KvStore, Linear, LinearRouted, Program, Ring, RmsNorm, Route,
    ArgMax, SCache, ScaleBy, Softcap, Add, SRowInts, op_sources, op_values)

# Work kinds (Plan.hs:124-139).
ANCHOR, RECOMPUTE, EPILOGUE, COMBINE, EFFECT, STAGE, LAND = (
    "anchor", "recompute", "epilogue", "combine", "effect", "stage", "land")
# Costs (Plan.hs:206-211), ordered.
CHEAP, PASS, EXPENSIVE = 0, 1, 2
# Families (Plan.hs:187-191).
GEMV, ATTENTION = "gemv", "attention"


@dataclass(frozen=True)
class Work:
    kind: str
    node: int


@dataclass(frozen=True)
class Stored:
    """A value in memory between steps: ``form`` is ("elements", type),
    ("partials",) or ("staged", cache source id) (Plan.hs:166-181)."""

    value: int
    form: tuple


def elements(t: str) -> tuple:
    return ("elements", t)


PARTIALS = ("partials",)


def staged_form(cache: int) -> tuple:
    return ("staged", cache)


@dataclass
class Step:
    index: int
    name: str
    work: list
    stores: list
    reads: list
    caches: list

    @property
    def anchors(self) -> list[int]:
        return [w.node for w in self.work if w.kind == ANCHOR]

    @property
    def is_light(self) -> bool:
        return not self.anchors


@dataclass
class Plan:
    program: Program
    steps: list


@dataclass(frozen=True)
class PlanOptions:
    """Plan.hs:243-268."""

    horizontal: bool = True
    gated: bool = False
    store_gelus: bool = False
    sequence_rows: int = 1


DEFAULT_OPTIONS = PlanOptions()


def anchor_family(op) -> Optional[str]:
    if isinstance(op, (Linear, LinearRouted)):
        return GEMV
    if isinstance(op, Attend):
        return ATTENTION
    return None


def node_cost(p: Program, op) -> int:
    """What recomputing an operation costs a threadgroup (Plan.hs:214-223)."""
    if isinstance(op, (RmsNorm, Route, ArgMax)):
        return PASS
    if isinstance(op, Gather):
        s = p.source(op.tokens)
        if s is not None and isinstance(s.kind, SRowInts) and s.kind.count > 1:
            return EXPENSIVE
    return CHEAP


def pointwise(op) -> bool:
    return isinstance(op, (Add, GeluMul, ScaleBy, Softcap, KvStore))


def is_effect(op) -> bool:
    return isinstance(op, KvStore)


def ring_room(length: int, window: Optional[int], bound: int) -> int:
    """Rows of one sequence a ring can store before an attention reads it (Plan.hs:276-281)."""
    seen = bound if window is None else window
    return 0 if seen > length else length - seen + 1


# Where a value is (Plan.hs:284-293): ("stored", step) with -1 for inputs,
# ("virtual", cost), ("tile", step, anchor node), ("partials", step).


@dataclass
class _StepB:
    index: int
    work: list = field(default_factory=list)
    stores: list = field(default_factory=list)
    family: Optional[str] = None
    writes: set = field(default_factory=set)


class _Planner:
    def __init__(self, opts: PlanOptions, checked: CheckedProgram):
        self.opts = opts
        p = self.p = checked.program
        self.nodes = {n.id: n for n in p.nodes}
        self.producer = {v: n for n in p.nodes for v in n.outputs}
        self.consumers: dict[int, list[int]] = {}
        for n in p.nodes:
            for v in op_values(n.op):
                self.consumers.setdefault(v, []).append(n.id)
        self.output_values = {o.value for o in p.outputs}
        self.avail: dict[int, tuple] = {}
        self.closed: list[_StepB] = []
        self.open: Optional[_StepB] = None
        self.next = 0
        self.landing: list[tuple] = []
        self.staged = self._staged()

    # What the rules see ---------------------------------------------------

    def op_of(self, n: int):
        node = self.nodes.get(n)
        return node.op if node else Input(0)

    def type_of(self, v: int) -> str:
        val = self.p.value(v)
        return val.type if val else F32

    def outs_of(self, n: int) -> list[int]:
        node = self.nodes.get(n)
        return list(node.outputs) if node else []

    def position_bound(self, s: int) -> int:
        src = self.p.source(s)
        return src.kind.bound if src is not None and isinstance(src.kind, SRowInts) else 0

    def _staged(self) -> set:
        out = set()
        for i, n in enumerate(self.p.nodes):
            if not isinstance(n.op, KvStore):
                continue
            c = n.op.at.cache
            src = self.p.source(c)
            if src is None or not isinstance(src.kind, SCache) or not isinstance(src.kind.layout, Ring):
                continue
            length = src.kind.layout.length
            if any(self.opts.sequence_rows > ring_room(length, r.op.spec.window, self.position_bound(r.op.to.positions))
                   for r in self.p.nodes[i + 1:]
                   if isinstance(r.op, Attend) and c in (r.op.to.keys, r.op.to.values)):
                out.add(n.id)
        return out

    def staged_into(self, c: int) -> Optional[int]:
        for n in self.p.nodes:
            if isinstance(n.op, KvStore) and n.op.at.cache == c and n.id in self.staged:
                return n.id
        return None

    def last_reader(self, c: int) -> Optional[int]:
        readers = [n.id for n in self.p.nodes if isinstance(n.op, Attend) and c in (n.op.to.keys, n.op.to.values)]
        return readers[-1] if readers else None

    def avail_of(self, v: int) -> tuple:
        return self.avail.get(v, ("stored", -1))

    def open_index(self) -> Optional[int]:
        return None if self.open is None else self.open.index

    # Steps ------------------------------------------------------------------

    def close_open(self) -> None:
        if self.open is None:
            return
        sb = self.open
        self.outputs_here()
        self.store_shared()
        sb1 = self.open if self.open is not None else sb
        in_step = {w.node for w in sb1.work}
        tiled = [v for w in sb1.work if w.kind in (ANCHOR, EPILOGUE) for v in self.outs_of(w.node)]
        stores = []
        for v in tiled:
            stores += self.store_tile(sb1, in_step, v)
        sb1.stores = sb1.stores + stores
        self.closed.append(sb1)
        self.open = None

    def store_tile(self, sb: _StepB, in_step: set, v: int) -> list:
        outside = any(c not in in_step for c in self.consumers.get(v, []))
        if not (outside or v in self.output_values):
            return []
        n = self.producer.get(v)
        if n is not None and isinstance(n.op, Attend):
            self.avail[v] = ("partials", sb.index)
            return [Stored(v, PARTIALS)]
        self.avail[v] = ("stored", sb.index)
        return [Stored(v, elements(self.type_of(v)))]

    def new_step(self, fam: Optional[str]) -> _StepB:
        self.close_open()
        sb = _StepB(self.next, family=fam)
        self.open = sb
        self.next += 1
        return sb

    def light_step(self) -> None:
        sb = self.open
        if not (sb is not None and sb.family is None and not any(w.kind == ANCHOR for w in sb.work)):
            self.new_step(None)
        i = self.open_index()
        due = [l for l in self.landing if i is not None and i > l[0]]
        for _, n, c in due:
            self.add_work(Work(LAND, n))
            if self.open is not None:
                self.open.writes.add(c)
        self.landing = [l for l in self.landing if l not in due]

    def land_rest(self) -> None:
        if self.landing:
            self.light_step()

    def add_work(self, w: Work) -> None:
        if self.open is not None and w.node not in [x.node for x in self.open.work]:
            self.open.work.append(w)

    def add_store(self, st: Stored) -> None:
        if self.open is not None and st not in self.open.stores:
            self.open.stores.append(st)

    # Chains -------------------------------------------------------------------

    def chain(self, v: int) -> None:
        a = self.avail_of(v)
        i = self.open_index()
        n = self.producer.get(v)
        if a[0] == "stored" and (i is None or a[1] != i):
            return
        if a[0] == "partials" and n is not None and (i is None or a[1] != i):
            self.add_work(Work(COMBINE, n.id))
            return
        if n is not None:
            planned = self.open is not None and n.id in [w.node for w in self.open.work]
            if not planned:
                for x in op_values(n.op):
                    self.chain(x)
                self.add_work(Work(RECOMPUTE, n.id))

    def outputs_here(self) -> None:
        st = self.open
        if st is None:
            return
        combined = {w.node for w in st.work if w.kind == COMBINE}

        def has(v: int) -> bool:
            a = self.avail_of(v)
            if a[0] == "stored":
                return True
            if a[0] == "partials":
                n = self.producer.get(v)
                return n is not None and n.id in combined
            if a[0] == "virtual" and v in self.producer:
                return all(has(x) for x in op_values(self.producer[v].op))
            return False

        if st.family is None and combined:
            for o in self.p.outputs:
                if self.avail_of(o.value)[0] == "virtual" and has(o.value):
                    self.materialize(o.value)

    def store_shared(self) -> None:
        st = self.open
        if st is None:
            return
        in_step = {w.node for w in st.work}

        def needed(v: int) -> bool:
            return any(c not in in_step for c in self.consumers.get(v, [])) or v in self.output_values

        def store(v: int) -> None:
            self.add_store(Stored(v, elements(self.type_of(v))))
            self.avail[v] = ("stored", st.index)

        work = list(st.work)
        for w in work:
            if w.kind == RECOMPUTE:
                for v in self.outs_of(w.node):
                    a = self.avail_of(v)
                    if a[0] == "virtual" and a[1] >= PASS and needed(v):
                        store(v)
        for w in work:
            if w.kind == COMBINE:
                for v in self.outs_of(w.node):
                    if self.avail_of(v)[0] == "partials" and needed(v):
                        store(v)

    def materialize(self, v: int) -> None:
        self.light_step()
        self.chain(v)
        i = self.open_index()
        if i is not None:
            self.add_store(Stored(v, elements(self.type_of(v))))
            self.avail[v] = ("stored", i)

    # Nodes ------------------------------------------------------------------

    def node(self, n) -> None:
        op = n.op
        if isinstance(op, Input):
            for v in n.outputs:
                self.avail[v] = ("stored", -1)
            return
        fam = anchor_family(op)
        if fam is not None:
            self.anchor(n, fam)
        elif is_effect(op):
            self.effect(n)
        else:
            self.light(n)

    def anchor(self, n, fam: str) -> None:
        ins = op_values(n.op)
        if any(self.touches_open(v) for v in ins):
            self.close_open()
        for v in ins:
            dear = self.expensive(v)
            gelu = self.stored_gelu(v)
            if dear or gelu:
                self.materialize(v)
        if isinstance(n.op, LinearRouted) and self.opts.gated:
            if self.avail_of(n.op.ids)[0] != "stored":
                self.materialize(n.op.ids)
        reads_caches = [c for c in op_sources(n.op) if self.open is not None and c in self.open.writes]
        gated_here = isinstance(n.op, LinearRouted) and self.opts.gated
        joins = (self.open is not None and self.opts.horizontal and self.open.family == fam and not reads_caches
                 and not gated_here)
        if not joins:
            self.new_step(fam)
        for v in ins:
            self.chain(v)
        self.add_work(Work(ANCHOR, n.id))
        s = self.open_index()
        if s is not None:
            for v in n.outputs:
                self.avail[v] = ("partials", s) if isinstance(n.op, Attend) else ("tile", s, n.id)
            if isinstance(n.op, Attend):
                for c in dict.fromkeys([n.op.to.keys, n.op.to.values]):
                    store = self.staged_into(c)
                    if self.last_reader(c) == n.id and store is not None:
                        self.landing.append((s, store, c))

    def touches_open(self, v0: int) -> bool:
        i = self.open_index()
        seen: set = set()
        todo = [v0]
        while todo:
            v = todo.pop(0)
            if v in seen:
                continue
            a = self.avail_of(v)
            if a[0] == "tile" and i is not None and a[1] == i:
                return True
            if a[0] == "partials" and i is not None and a[1] == i:
                return True
            seen.add(v)
            if a[0] == "virtual" and v in self.producer:
                todo = op_values(self.producer[v].op) + todo
        return False

    def stored_gelu(self, v: int) -> bool:
        n = self.producer.get(v)
        if self.opts.store_gelus and n is not None and isinstance(n.op, (GeluMul, GatedGelu)):
            return self.avail_of(v)[0] == "virtual"
        return False

    def expensive(self, v: int) -> bool:
        a = self.avail_of(v)
        if a[0] == "partials":
            return True
        if a[0] == "virtual":
            return a[1] >= EXPENSIVE
        return False

    def light(self, n) -> None:
        op = n.op
        ins = op_values(op)
        avails = [self.avail_of(v) for v in ins]
        i = self.open_index()
        on_tile = [(v, a[2]) for v, a in zip(ins, avails) if a[0] == "tile" and i is not None and a[1] == i]
        anchors = list(dict.fromkeys(a for _, a in on_tile))
        tiled_values = [v for v, _ in on_tile]

        def other(v, a) -> bool:
            if a[0] == "stored":
                return True
            if a[0] == "virtual" and a[1] == CHEAP:
                return not self.touches_open(v)
            return False

        others_ok = all(other(v, a) for v, a in zip(ins, avails) if v not in tiled_values)
        if len(anchors) == 1 and pointwise(op) and others_ok:
            for v, a in zip(ins, avails):
                if a[0] == "virtual":
                    self.chain(v)
            self.add_work(Work(EPILOGUE, n.id))
            if i is not None:
                for v in n.outputs:
                    self.avail[v] = ("tile", i, anchors[0])
        else:
            costs = [self.input_cost(v) for v in ins]
            c = max([node_cost(self.p, op)] + costs)
            for v in n.outputs:
                self.avail[v] = ("virtual", c)
            if self.opts.gated and (self.feeds_routed(n) or self.is_output_route(n)):
                if any(self.touches_open(v) for v in ins):
                    self.close_open()
                for v in list(n.outputs)[:1]:
                    self.materialize(v)

    def feeds_routed(self, r) -> bool:
        if not isinstance(r.op, Route) or not r.outputs:
            return False
        v = r.outputs[0]
        return any(isinstance(self.op_of(c), LinearRouted) and self.op_of(c).ids == v
                   for c in self.consumers.get(v, []))

    def is_output_route(self, r) -> bool:
        return isinstance(r.op, Route) and bool(r.outputs) and r.outputs[0] in self.output_values

    def input_cost(self, v: int) -> int:
        a = self.avail_of(v)
        if a[0] == "virtual":
            return a[1]
        if a[0] == "partials":
            return EXPENSIVE
        return CHEAP

    def effect(self, n) -> None:
        ins = op_values(n.op)
        if n.id in self.staged:
            self.light_step()
            for v in ins:
                self.chain(v)
            self.add_work(Work(STAGE, n.id))
            if isinstance(n.op, KvStore):
                self.add_store(Stored(n.op.x, staged_form(n.op.at.cache)))
        else:
            avails = [self.avail_of(v) for v in ins]
            i = self.open_index()
            on_tile = [v for v, a in zip(ins, avails) if a[0] == "tile" and i is not None and a[1] == i]
            if on_tile and pointwise(n.op) and len(on_tile) == len(ins):
                self.add_work(Work(EPILOGUE, n.id))
            else:
                self.light_step()
                for v in ins:
                    self.chain(v)
                self.add_work(Work(EFFECT, n.id))
            if self.open is not None:
                self.open.writes |= set(op_sources(n.op)[:1])

    def outputs(self) -> None:
        for o in self.p.outputs:
            if self.avail_of(o.value)[0] in ("virtual", "partials"):
                self.materialize(o.value)

    # Steps as the plan states them --------------------------------------------

    def run(self) -> Plan:
        for n in self.p.nodes:
            self.node(n)
        self.outputs()
        self.land_rest()
        self.close_open()
        return Plan(self.p, [self.finish(sb) for sb in self.closed])

    def finish(self, sb: _StepB) -> Step:
        order = {n.id: k for k, n in enumerate(self.p.nodes)}
        vorder = {v.id: k for k, v in enumerate(self.p.values)}
        caches = []
        for w in sb.work:
            for c in self.caches_of(w):
                if c not in caches:
                    caches.append(c)
        return Step(
            index=sb.index,
            name=self.name(sb),
            work=sorted(sb.work, key=lambda w: order.get(w.node, w.node)),
            stores=sorted(sb.stores, key=lambda st: vorder.get(st.value, st.value)),
            reads=sorted(self.reads_of(sb), key=lambda st: vorder.get(st.value, st.value)),
            caches=caches,
        )

    def caches_of(self, w: Work) -> list[int]:
        if w.kind in (STAGE, COMBINE):
            return []
        op = self.op_of(w.node)
        if isinstance(op, KvStore):
            return [op.at.cache]
        if isinstance(op, Attend):
            return [op.to.keys, op.to.values]
        return []

    def reads_of(self, sb: _StepB) -> list:
        in_step = {v for w in sb.work if w.kind in (COMBINE, ANCHOR, RECOMPUTE, EPILOGUE) for v in self.outs_of(w.node)}

        def reads_of_work(w: Work) -> list[int]:
            if w.kind == COMBINE:
                return self.outs_of(w.node)
            if w.kind == LAND:
                return []
            return [v for v in op_values(self.op_of(w.node)) if v not in in_step]

        def wanted(w: Work, form: tuple) -> bool:
            if w.kind == COMBINE:
                return form == PARTIALS
            return form[0] not in ("partials", "staged")

        def stages_read(w: Work) -> list[int]:
            op = self.op_of(w.node)
            if w.kind == ANCHOR and isinstance(op, Attend):
                return list(dict.fromkeys([op.to.keys, op.to.values]))
            if w.kind == LAND and isinstance(op, KvStore):
                return [op.at.cache]
            return []

        out: list = []
        for w in sb.work:
            for v in reads_of_work(w):
                for st in self.stored_before(sb.index, v):
                    if wanted(w, st.form) and st not in out:
                        out.append(st)
        for w in sb.work:
            for c in stages_read(w):
                for st in self.staged_before(sb.index, c):
                    if st not in out:
                        out.append(st)
        return out

    def stored_before(self, s: int, v: int) -> list:
        out = [st for sb in self.closed if sb.index < s for st in sb.stores if st.value == v]
        n = self.producer.get(v)
        if n is not None and isinstance(n.op, Input):
            out.append(Stored(v, elements(self.type_of(v))))
        return out

    def staged_before(self, s: int, c: int) -> list:
        return [st for sb in self.closed if sb.index < s for st in sb.stores if st.form == staged_form(c)]

    def name(self, sb: _StepB) -> str:
        anchors = [self.op_of(w.node) for w in sb.work if w.kind == ANCHOR]
        if anchors:
            words = list(dict.fromkeys("attend" if isinstance(a, Attend) else "gemv" for a in anchors))
            return f"s{sb.index}_" + "_".join(words)
        for w in sb.work:
            if w.kind in (EFFECT, STAGE):
                return f"s{sb.index}_store"
            if w.kind == COMBINE:
                return f"s{sb.index}_combine"
            if w.kind == RECOMPUTE:
                st = next((st for st in sb.stores if st.form[0] == "elements"), None)
                if st is not None:
                    return f"s{sb.index}_{self.p.value(st.value).name}"
        if any(w.kind == LAND for w in sb.work):
            return f"s{sb.index}_land"
        return f"s{sb.index}_light"


def plan(opts: PlanOptions, checked: CheckedProgram) -> Plan:
    """The program as steps, each one kernel launch (Plan.hs:314-318)."""
    return _Planner(opts, checked).run()


def render_plan(pl: Plan) -> str:
    """The deterministic text form (Plan.hs:816-843)."""
    p = pl.program

    def label(n: int) -> str:
        node = p.node(n)
        return node.name if node else "?"

    def stored(st: Stored) -> str:
        v = p.value(st.value)
        name = v.name if v else "?"
        if st.form[0] == "elements":
            return f"{name} {st.form[1]}"
        if st.form == PARTIALS:
            return f"{name} partials"
        src = p.source(st.form[1])
        return f"{name} staged for {src.name if src else '?'}"

    lines = [f"plan {p.name}"]
    for s in pl.steps:
        lines.append(f"  step {s.name}")
        lines += [f"    {w.kind} {label(w.node)}" for w in s.work]
        lines += [f"    reads {stored(st)}" for st in s.reads]
        lines += [f"    stores {stored(st)}" for st in s.stores]
    return "\n".join(lines) + "\n"
