"""The gate a kernel passes before a backend lowers it: a restatement of the
checks of src/FuryKernel/Check.hs that a lowering relies on.

Checked here, each failure a finding with the reference's rule: the kernel
was built for the target's SIMD width; its thread count is a positive
multiple of it within the target's limit; its bindings are at most the
target's; its threadgroup layout fits the target's memory; every name is
declared once and before use; every expression is well typed (the typed
surface's rules, Build.hs:310-595: arithmetic on compute types only,
operands of one type, bool conditions, u32 indices, the widenings and
narrowings there are); packs are two or more elements of a power-of-two
size the target loads at once from memory that aligned; barriers stand in
uniform control and SIMD-group operations and fragments where every lane of
the group is; fragment products take the target's fragment types; launch
sizes are u32 arithmetic over dimensions.

Not restated (the program-level gate and the dynamic interpreter stand for
them in this build's tests): the bounds proofs of Check/Bounds.hs and the
Omega test, the hazard check, and the verification of declared uniformity.
"""

from __future__ import annotations

from dataclasses import dataclass

from ..program.graph import BF16, BOOL, F16, F32, I8, I32, SCALAR_SIZE, U8, U32
from . import ir as I
from .build import FLOAT, INT, NARROW, NARROW_INT, NUM, WIDEN, Finding, TargetCaps


class GateError(Exception):
    def __init__(self, findings: list):
        super().__init__("; ".join(f.message for f in findings))
        self.findings = findings


@dataclass(frozen=True)
class Checked:
    """A kernel the gate took, for the target it took it for."""

    kernel: I.Kernel
    caps: TargetCaps


class _Env:
    def __init__(self, k: I.Kernel):
        self.params = {p.name: p.type for p in k.params}
        self.buffers = {b.name: b for b in k.buffers}
        self.tables = {t.name: t for t in k.tables}
        self.arrays = {a.name: a for a in k.tg_arrays}
        self.locals: dict = {}
        self.frags: dict = {}


def type_of(env: _Env, e) -> str:
    """The type of a well-typed expression (Cpu.hs:338-357's typeOf)."""
    if isinstance(e, I.ELit):
        return e.lit.type
    if isinstance(e, I.EVar):
        return env.locals[e.name]
    if isinstance(e, I.EParam):
        return env.params[e.name]
    if isinstance(e, I.EBuiltin):
        return U32
    if isinstance(e, I.EUn):
        return type_of(env, e.a)
    if isinstance(e, I.EBin):
        return BOOL if e.op in I.COMPARISONS or e.op in ("and", "or") else type_of(env, e.a)
    if isinstance(e, (I.ESelect,)):
        return type_of(env, e.a)
    if isinstance(e, I.EFma):
        return type_of(env, e.a)
    if isinstance(e, (I.EConvert, I.ENarrowInt)):
        return e.type
    if isinstance(e, I.ELoad):
        return env.buffers[e.buffer].type
    if isinstance(e, I.ELoadVia):
        return env.tables[e.table].type
    if isinstance(e, I.ETgLoad):
        return env.arrays[e.array].type
    raise TypeError(e)


class _Gate:
    def __init__(self, k: I.Kernel, caps: TargetCaps):
        self.k = k
        self.caps = caps
        self.env = _Env(k)
        self.findings: list = []

    def bad(self, rule: str, msg: str) -> None:
        self.findings.append(Finding(rule, msg))

    # -- expressions
    def expr(self, e) -> str | None:
        """The expression's type, or None after a finding."""
        env = self.env
        if isinstance(e, I.ELit):
            if not I.canonical_nan(e.lit):
                self.bad("typing", f"The NaN literal {I.render_literal(e.lit)} is not the canonical one.")
            return e.lit.type
        if isinstance(e, I.EVar):
            if e.name not in env.locals:
                self.bad("names", f"The local {e.name} is used before it is bound.")
                return None
            return env.locals[e.name]
        if isinstance(e, I.EParam):
            if e.name not in env.params:
                self.bad("names", f"The parameter {e.name} is not declared.")
                return None
            return env.params[e.name]
        if isinstance(e, I.EBuiltin):
            return U32
        if isinstance(e, I.EUn):
            t = self.expr(e.a)
            if t is None:
                return None
            ok = {"not": (BOOL,), "neg": NUM, "abs": NUM}.get(e.op, FLOAT)
            if t not in ok:
                self.bad("typing", f"{e.op} of {t}.")
                return None
            return t
        if isinstance(e, I.EBin):
            a, b = self.expr(e.a), self.expr(e.b)
            if a is None or b is None:
                return None
            if a != b:
                self.bad("typing", f"The operands of {I.BINOPS[e.op]} are {a} and {b}.")
                return None
            if e.op in ("and", "or"):
                ok = (BOOL,)
            elif e.op in ("eq", "ne"):
                ok = NUM + (BOOL,)
            elif e.op in ("div",):
                ok = NUM
            elif e.op == "rem":
                ok = INT
            else:
                ok = NUM
            if a not in ok:
                self.bad("typing", f"{I.BINOPS[e.op]} of {a}.")
                return None
            return BOOL if e.op in I.COMPARISONS or e.op in ("and", "or") else a
        if isinstance(e, I.ESelect):
            c, a, b = self.expr(e.c), self.expr(e.a), self.expr(e.b)
            if c != BOOL or a is None or a != b:
                self.bad("typing", "A select of a bool over two values of one type.")
                return None
            return a
        if isinstance(e, I.EFma):
            ts = {self.expr(e.a), self.expr(e.b), self.expr(e.c)}
            if len(ts) != 1 or next(iter(ts)) not in FLOAT:
                self.bad("typing", "An fma of three f32 or three f16.")
                return None
            return ts.pop()
        if isinstance(e, I.EConvert):
            t = self.expr(e.a)
            if t is None:
                return None
            if (t, e.type) not in WIDEN | NARROW | {(U32, F32), (I32, F32)} and t != e.type:
                self.bad("typing", f"No conversion of {t} to {e.type}.")
                return None
            return e.type
        if isinstance(e, I.ENarrowInt):
            t = self.expr(e.a)
            if (t, e.type) not in NARROW_INT:
                self.bad("typing", f"No integer narrowing of {t} to {e.type}.")
                return None
            return e.type
        if isinstance(e, I.ELoad):
            self.index(e.index)
            b = self.env.buffers.get(e.buffer)
            if b is None or b.access == I.WRITE:
                self.bad("access", f"A load of {e.buffer}, which the kernel cannot read.")
                return None
            return b.type
        if isinstance(e, I.ELoadVia):
            self.index(e.entry)
            self.index(e.index)
            t = self.env.tables.get(e.table)
            if t is None or t.access == I.WRITE:
                self.bad("access", f"A load through {e.table}, which the kernel cannot read.")
                return None
            return t.type
        if isinstance(e, I.ETgLoad):
            self.index(e.index)
            a = self.env.arrays.get(e.array)
            if a is None:
                self.bad("names", f"The threadgroup array {e.array} is not declared.")
                return None
            return a.type
        self.bad("typing", f"Not an expression: {e!r}.")
        return None

    def index(self, e) -> None:
        t = self.expr(e)
        if t is not None and t != U32:
            self.bad("typing", f"An index of {t}: {I.render_expr(e)}.")

    def value(self, e, want: str, where: str) -> None:
        t = self.expr(e)
        if t is not None and t != want:
            self.bad("typing", f"A value of {t} stored to {where}, of {want}.")

    def declare(self, name: str, t: str) -> None:
        if name in self.env.locals or name in self.env.params or name in self.env.buffers \
                or name in self.env.tables or name in self.env.arrays or name in self.env.frags:
            self.bad("names", f"The name {name} is declared twice.")
        self.env.locals[name] = t

    def pack(self, n: int, t: str, align: int, where: str) -> None:
        size = n * SCALAR_SIZE[t]
        if n < 2 or t == BOOL or size & (size - 1) or size > self.caps.lane_load_max or size > align:
            self.bad("packs", f"A pack of {n} {t} at {where}: {size} bytes, from memory aligned to {align}.")

    # -- statements
    def stmts(self, ss, region: str) -> None:
        for s in ss:
            self.stmt(s, region)

    def stmt(self, s, region: str) -> None:
        env = self.env
        if isinstance(s, (I.SLet, I.SVar)):
            t = self.expr(s.e)
            if t is not None and t != s.type:
                self.bad("typing", f"The local {s.name} of {s.type} bound to a value of {t}.")
            self.declare(s.name, s.type)
        elif isinstance(s, I.SAssign):
            if s.name not in env.locals:
                self.bad("names", f"An assignment to {s.name}, which is not bound.")
            else:
                self.value(s.e, env.locals[s.name], s.name)
        elif isinstance(s, I.SStore):
            self.index(s.index)
            b = env.buffers.get(s.buffer)
            if b is None or b.access == I.READ:
                self.bad("access", f"A store to {s.buffer}, which the kernel cannot write.")
            else:
                self.value(s.value, b.type, s.buffer)
        elif isinstance(s, I.SStoreVia):
            self.index(s.entry)
            self.index(s.index)
            t = env.tables.get(s.table)
            if t is None or t.access == I.READ:
                self.bad("access", f"A store through {s.table}, which the kernel cannot write.")
            else:
                self.value(s.value, t.type, s.table)
        elif isinstance(s, I.STgStore):
            self.index(s.index)
            a = env.arrays.get(s.array)
            if a is None:
                self.bad("names", f"The threadgroup array {s.array} is not declared.")
            else:
                self.value(s.value, a.type, s.array)
        elif isinstance(s, I.SLoadPack):
            self.index(s.index)
            b = env.buffers.get(s.buffer)
            if b is None or b.access == I.WRITE or b.type != s.type:
                self.bad("access", f"A pack loaded from {s.buffer}.")
            else:
                self.pack(len(s.names), b.type, b.align, s.buffer)
            for n in s.names:
                self.declare(n, s.type)
        elif isinstance(s, I.SLoadPackVia):
            self.index(s.entry)
            self.index(s.index)
            t = env.tables.get(s.table)
            if t is None or t.access == I.WRITE or t.type != s.type:
                self.bad("access", f"A pack loaded through {s.table}.")
            else:
                self.pack(len(s.names), t.type, t.align, s.table)
            for n in s.names:
                self.declare(n, s.type)
        elif isinstance(s, I.SStorePack):
            self.index(s.index)
            b = env.buffers.get(s.buffer)
            if b is None or b.access == I.READ:
                self.bad("access", f"A pack stored to {s.buffer}.")
            else:
                self.pack(len(s.values), b.type, b.align, s.buffer)
                for v in s.values:
                    self.value(v, b.type, s.buffer)
        elif isinstance(s, I.STgStorePack):
            self.index(s.index)
            a = env.arrays.get(s.array)
            if a is None:
                self.bad("names", f"The threadgroup array {s.array} is not declared.")
            else:
                self.pack(len(s.values), a.type, I.least_align(a.type), s.array)
                for v in s.values:
                    self.value(v, a.type, s.array)
        elif isinstance(s, I.SIf):
            if self.expr(s.cond) not in (BOOL, None):
                self.bad("typing", "A condition that is not a bool.")
            inner = _meet(region, s.region)
            self.stmts(s.then, inner)
            self.stmts(s.orelse, inner)
        elif isinstance(s, I.SFor):
            self.index(s.start)
            self.declare(s.var, U32)
            self.index(s.end)
            self.index(s.step)
            self.stmts(s.body, _meet(region, s.region))
        elif isinstance(s, I.SBarrier):
            if region != "uniform":
                self.bad("uniformity", "A barrier where not every thread of the threadgroup is.")
        elif isinstance(s, I.SSimdBarrier):
            self.converged(region, "A SIMD-group barrier")
        elif isinstance(s, I.SSimd):
            self.converged(region, "A SIMD-group reduction")
            t = self.expr(s.e)
            if t is not None and (t != s.type or t not in NUM):
                self.bad("typing", f"A SIMD-group reduction of {t} as {s.type}.")
            self.declare(s.name, s.type)
        else:
            self.fragment(s, region)

    def converged(self, region: str, what: str) -> None:
        if region == "divergent":
            self.bad("uniformity", f"{what} where the lanes of a SIMD group may diverge.")

    def fragment(self, s, region: str) -> None:
        env = self.env
        self.converged(region, "A fragment operation")
        if isinstance(s, I.SFragVar):
            if s.name in env.frags or s.name in env.locals:
                self.bad("names", f"The name {s.name} is declared twice.")
            env.frags[s.name] = s.type
            return
        names = {I.SFragLoad: ("name",), I.SFragStore: ("name",), I.SFragMma: ("d", "a", "b", "c"),
                 I.SFragConvert: ("d", "s"), I.SFragScaleRows: ("frag",)}.get(type(s))
        if names is None:
            self.bad("typing", f"Not a statement: {s!r}.")
            return
        for n in names:
            if getattr(s, n) not in env.frags:
                self.bad("names", f"The fragment {getattr(s, n)} is not declared.")
                return
        if isinstance(s, (I.SFragLoad, I.SFragStore)):
            self.index(s.index)
            self.index(s.stride)
            m = s.mem
            if m.kind == "device":
                t = env.buffers[m.name].type if m.name in env.buffers else None
            elif m.kind == "threadgroup":
                t = env.arrays[m.name].type if m.name in env.arrays else None
            else:
                self.index(m.entry)
                t = env.tables[m.name].type if m.name in env.tables else None
            if t != env.frags[s.name]:
                self.bad("typing", f"The fragment {s.name} of {env.frags[s.name]} against memory of {t}.")
        elif isinstance(s, I.SFragMma):
            ta, tb = env.frags[s.a], env.frags[s.b]
            if env.frags[s.d] != F32 or env.frags[s.c] != F32 or ta != tb or ta not in self.caps.fragments:
                self.bad("fragments", f"A product of {ta} and {tb} fragments into f32 on {self.caps.name}.")
        elif isinstance(s, I.SFragConvert):
            if env.frags[s.d] != F32:
                self.bad("fragments", "A fragment widens into f32.")
        elif isinstance(s, I.SFragScaleRows):
            self.index(s.index)
            a = env.arrays.get(s.array)
            if env.frags[s.frag] != F32 or a is None or a.type != F32:
                self.bad("fragments", "Rows of an f32 fragment scaled by an f32 threadgroup array.")

    # -- the kernel
    def launch_size(self, e, what: str) -> None:
        ok = (isinstance(e, I.ELit) and e.lit.type == U32) or (
            isinstance(e, I.EParam) and any(p.name == e.name and p.dim is not None for p in self.k.params)) or (
            isinstance(e, I.EBin) and e.op in ("add", "sub", "mul", "div", "rem"))
        if not ok:
            self.bad("launch", f"The {what}, {I.render_expr(e)}, is not u32 arithmetic over dimensions.")
        elif isinstance(e, I.EBin):
            self.launch_size(e.a, what)
            self.launch_size(e.b, what)

    def run(self) -> None:
        k, caps = self.k, self.caps
        if k.simd_width != caps.simd_width:
            self.bad("target", f"The kernel {k.name} was built for SIMD groups of {k.simd_width} lanes; "
                               f"{caps.name}'s have {caps.simd_width}.")
        if not (0 < k.threads <= caps.max_threads and k.threads % caps.simd_width == 0):
            self.bad("threads", f"{k.threads} threads a threadgroup: {caps.name} takes a multiple of "
                                f"{caps.simd_width} up to {caps.max_threads}.")
        if len(k.buffers) + len(k.tables) > caps.max_buffers:
            self.bad("buffers", f"{len(k.buffers) + len(k.tables)} bindings: {caps.name} takes {caps.max_buffers}.")
        total = I.tg_layout(k.tg_arrays)[1]
        if total > caps.tg_mem_bytes:
            self.bad("threadgroup_memory", f"{total} bytes of threadgroup memory: {caps.name} has {caps.tg_mem_bytes}.")
        seen = set()
        for n in [k.name] + [p.name for p in k.params] + [b.name for b in k.buffers] + [t.name for t in k.tables] \
                + [a.name for a in k.tg_arrays]:
            if n in seen:
                self.bad("names", f"The name {n} is declared twice.")
            seen.add(n)
        self.launch_size(k.groups, "grid")
        for b in k.buffers:
            self.launch_size(b.extent, f"extent of {b.name}")
        for t in k.tables:
            self.launch_size(t.entries, f"number of entries of {t.name}")
            self.launch_size(t.extent, f"extent of {t.name}")
        self.stmts(k.body, "uniform")


def _meet(a: str, b: str) -> str:
    order = {"uniform": 0, "simd_uniform": 1, "divergent": 2}
    return a if order[a] >= order[b] else b


def check(k: I.Kernel, caps: TargetCaps) -> Checked:
    """The kernel, checked for the target, or GateError with the findings."""
    g = _Gate(k, caps)
    g.run()
    if g.findings:
        raise GateError(g.findings)
    return Checked(k, caps)
