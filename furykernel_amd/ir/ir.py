"""The kernel IR (src/FuryKernel/IR.hs): untyped, first-order, structured.

Expressions and statements are frozen dataclasses, one per constructor of
the reference's ``Expr`` and ``Stmt`` (IR.hs:206-383); a kernel holds its
interface (parameters, buffers, tables, threadgroup arrays), its thread
count, the SIMD width it was built for, its grid over the parameters and its
body.  ``render_kernel`` is the deterministic text form (IR.hs:463-639),
first line ``ir 1``, which the IR hash is FNV-1a of (Abi.hs:255-262).

Scalar types are the short names of src/FuryKernel/Type.hs:43-52.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Optional, Union

from ..program.graph import BF16, BOOL, F16, F32, I8, I32, SCALAR_SIZE, U8, U32

STORAGE_ONLY = (BF16, I8, U8)  # Type.hs:74-75: no arithmetic


def least_align(t: str) -> int:
    """Type.hs:70-71: 16, or the type's size if larger."""
    return max(16, SCALAR_SIZE[t])


# ---------------------------------------------------------------------------
# Literals (IR.hs:64-124): floats by their bits, integers by their value.

@dataclass(frozen=True)
class Lit:
    type: str
    bits: int  # f32: the binary32 bits; f16/bf16: the 16 bits; ints: the value; bool: 0/1

    def __post_init__(self):
        lo, hi = {F32: (0, 0xFFFFFFFF), F16: (0, 0xFFFF), BF16: (0, 0xFFFF), I32: (-2**31, 2**31 - 1),
                  U32: (0, 2**32 - 1), I8: (-128, 127), U8: (0, 255), BOOL: (0, 1)}[self.type]
        if not lo <= self.bits <= hi:
            raise ValueError(f"the literal {self.bits} is outside {self.type}'s range, {lo} to {hi}.")


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def lit_f32(x: float) -> Lit:
    """A binary32 literal of a value binary32 holds (every NaN the canonical one, IR.hs:96-106)."""
    if x != x:
        return Lit(F32, 0x7FC00000)
    return Lit(F32, f32_bits(x))


def lit_u32(n: int) -> Lit:
    return Lit(U32, n)


def canonical_nan(l: Lit) -> bool:
    """IR.hs:96-106: no NaN, or the quiet NaN with no payload and no sign."""
    b = l.bits
    if l.type == F32:
        return (b & 0x7F800000) != 0x7F800000 or (b & 0x7FFFFF) == 0 or b == 0x7FC00000
    if l.type == F16:
        return (b & 0x7C00) != 0x7C00 or (b & 0x3FF) == 0 or b == 0x7E00
    if l.type == BF16:
        return (b & 0x7F80) != 0x7F80 or (b & 0x7F) == 0 or b == 0x7FC0
    return True


# ---------------------------------------------------------------------------
# Expressions (IR.hs:206-258)

UNOPS = ("neg", "not", "abs", "sqrt", "rsqrt", "exp", "log", "tanh")
BINOPS = {"add": "+", "sub": "-", "mul": "*", "div": "/", "rem": "%", "min": "min", "max": "max",
          "eq": "==", "ne": "!=", "lt": "<", "le": "<=", "gt": ">", "ge": ">=", "and": "&&", "or": "||"}
COMPARISONS = ("eq", "ne", "lt", "le", "gt", "ge")
BUILTINS = {"thread": "@thread", "group": "@group", "lane": "@lane", "simd_group": "@simd_group"}


@dataclass(frozen=True)
class ELit:
    lit: Lit


@dataclass(frozen=True)
class EVar:
    name: str


@dataclass(frozen=True)
class EParam:
    name: str


@dataclass(frozen=True)
class EBuiltin:
    which: str  # thread, group, lane, simd_group


@dataclass(frozen=True)
class EUn:
    op: str
    a: "Expr"


@dataclass(frozen=True)
class EBin:
    op: str
    a: "Expr"
    b: "Expr"


@dataclass(frozen=True)
class ESelect:
    c: "Expr"
    a: "Expr"
    b: "Expr"


@dataclass(frozen=True)
class EFma:
    a: "Expr"
    b: "Expr"
    c: "Expr"


@dataclass(frozen=True)
class EConvert:
    type: str
    a: "Expr"


@dataclass(frozen=True)
class ENarrowInt:
    overflow: str  # clamp | wrap
    type: str
    a: "Expr"


@dataclass(frozen=True)
class ELoad:
    buffer: str
    index: "Expr"


@dataclass(frozen=True)
class ELoadVia:
    table: str
    entry: "Expr"
    index: "Expr"


@dataclass(frozen=True)
class ETgLoad:
    array: str
    index: "Expr"


Expr = Union[ELit, EVar, EParam, EBuiltin, EUn, EBin, ESelect, EFma, EConvert, ENarrowInt, ELoad, ELoadVia, ETgLoad]

# ---------------------------------------------------------------------------
# Statements (IR.hs:260-383).  Regions: uniform, simd_uniform, divergent.

REGIONS = ("uniform", "simd_uniform", "divergent")
SIMD_OPS = ("simd_sum", "simd_max", "simd_min")


@dataclass(frozen=True)
class SLet:
    name: str
    type: str
    e: Expr


@dataclass(frozen=True)
class SVar:
    name: str
    type: str
    e: Expr


@dataclass(frozen=True)
class SAssign:
    name: str
    e: Expr


@dataclass(frozen=True)
class SStore:
    buffer: str
    index: Expr
    value: Expr


@dataclass(frozen=True)
class SStoreVia:
    table: str
    entry: Expr
    index: Expr
    value: Expr


@dataclass(frozen=True)
class STgStore:
    array: str
    index: Expr
    value: Expr


@dataclass(frozen=True)
class SLoadPack:
    names: tuple
    type: str
    buffer: str
    index: Expr


@dataclass(frozen=True)
class SStorePack:
    buffer: str
    index: Expr
    values: tuple


@dataclass(frozen=True)
class STgStorePack:
    array: str
    index: Expr
    values: tuple


@dataclass(frozen=True)
class SLoadPackVia:
    names: tuple
    type: str
    table: str
    entry: Expr
    index: Expr


@dataclass(frozen=True)
class SIf:
    region: str
    cond: Expr
    then: tuple
    orelse: tuple = ()


@dataclass(frozen=True)
class SFor:
    region: str
    var: str
    start: Expr
    end: Expr
    step: Expr
    body: tuple


@dataclass(frozen=True)
class SBarrier:
    pass


@dataclass(frozen=True)
class SSimdBarrier:
    pass


@dataclass(frozen=True)
class SSimd:
    name: str
    op: str
    type: str
    e: Expr


# Fragment memory: ("device", buffer) | ("threadgroup", array) | ("via", table, entry expr)
@dataclass(frozen=True)
class FragMem:
    kind: str
    name: str
    entry: Optional[Expr] = None


@dataclass(frozen=True)
class SFragVar:
    name: str
    type: str


@dataclass(frozen=True)
class SFragLoad:
    name: str
    mem: FragMem
    index: Expr
    stride: Expr
    transposed: bool


@dataclass(frozen=True)
class SFragMma:
    d: str
    a: str
    b: str
    c: str


@dataclass(frozen=True)
class SFragConvert:
    d: str
    s: str


@dataclass(frozen=True)
class SFragScaleRows:
    frag: str
    array: str
    index: Expr


@dataclass(frozen=True)
class SFragStore:
    mem: FragMem
    index: Expr
    stride: Expr
    name: str


Stmt = Union[SLet, SVar, SAssign, SStore, SStoreVia, STgStore, SLoadPack, SStorePack, STgStorePack, SLoadPackVia,
             SIf, SFor, SBarrier, SSimdBarrier, SSimd, SFragVar, SFragLoad, SFragMma, SFragConvert, SFragScaleRows,
             SFragStore]

# ---------------------------------------------------------------------------
# Kernels (IR.hs:385-461)

READ, WRITE, READ_WRITE = "read", "write", "read_write"


@dataclass(frozen=True)
class DimRange:
    min: int
    max: int
    multiple_of: int


@dataclass(frozen=True)
class Param:
    name: str
    type: str
    dim: Optional[DimRange] = None  # a dimension (u32 that sizes the launch), or a scalar


@dataclass(frozen=True)
class Buffer:
    name: str
    access: str
    type: str
    align: int
    extent: Expr
    apart: bool = False


@dataclass(frozen=True)
class Table:
    name: str
    access: str
    type: str
    align: int
    entries: Expr
    extent: Expr
    distinct: bool = False
    apart: bool = False


@dataclass(frozen=True)
class TgArray:
    name: str
    type: str
    count: int


def tg_align(a: TgArray) -> int:
    return least_align(a.type)


def tg_bytes(a: TgArray) -> int:
    al = tg_align(a)
    return (a.count * SCALAR_SIZE[a.type] + al - 1) // al * al


def tg_layout(arrays) -> tuple:
    """IR.hs:452-460: each array's offset, the more aligned first (a stable
    order otherwise), and the total."""
    placed = sorted(arrays, key=lambda a: -tg_align(a))
    offsets, at = [], 0
    for a in placed:
        offsets.append((a.name, at))
        at += tg_bytes(a)
    return offsets, sum(tg_bytes(a) for a in arrays)


@dataclass(frozen=True)
class Kernel:
    name: str
    threads: int
    simd_width: int
    groups: Expr
    params: tuple = ()
    buffers: tuple = ()
    tables: tuple = ()
    tg_arrays: tuple = ()
    body: tuple = ()


# ---------------------------------------------------------------------------
# Rendering (IR.hs:463-684)

def render_literal(l: Lit) -> str:
    if l.type == F32:
        return f"f32:0x{l.bits:x}"
    if l.type in (F16, BF16):
        return f"{l.type}:0x{l.bits:x}"
    if l.type == I32:
        return f"{l.bits}i"
    if l.type == U32:
        return f"{l.bits}u"
    if l.type == I8:
        return f"{l.bits}i8"
    if l.type == U8:
        return f"{l.bits}u8"
    return "true" if l.bits else "false"


def render_expr(e: Expr) -> str:
    """Fully parenthesised (IR.hs:617-665)."""
    if isinstance(e, ELit):
        return render_literal(e.lit)
    if isinstance(e, EVar):
        return e.name
    if isinstance(e, EParam):
        return "$" + e.name
    if isinstance(e, EBuiltin):
        return BUILTINS[e.which]
    if isinstance(e, EUn):
        return f"{e.op}({render_expr(e.a)})"
    if isinstance(e, EBin):
        return f"({render_expr(e.a)} {BINOPS[e.op]} {render_expr(e.b)})"
    if isinstance(e, ESelect):
        return f"select({render_expr(e.c)}, {render_expr(e.a)}, {render_expr(e.b)})"
    if isinstance(e, EFma):
        return f"fma({render_expr(e.a)}, {render_expr(e.b)}, {render_expr(e.c)})"
    if isinstance(e, EConvert):
        return f"{e.type}({render_expr(e.a)})"
    if isinstance(e, ENarrowInt):
        return f"{e.type}_{'clamped' if e.overflow == 'clamp' else 'wrapped'}({render_expr(e.a)})"
    if isinstance(e, ELoad):
        return f"{e.buffer}[{render_expr(e.index)}]"
    if isinstance(e, ELoadVia):
        return f"{e.table}[{render_expr(e.entry)}][{render_expr(e.index)}]"
    if isinstance(e, ETgLoad):
        return f"{e.array}[{render_expr(e.index)}]"
    raise TypeError(f"not an expression: {e!r}")


def _mem(m: FragMem) -> str:
    if m.kind == "device":
        return m.name
    if m.kind == "threadgroup":
        return "threadgroup " + m.name
    return f"{m.name}[{render_expr(m.entry)}]"


def render_stmt(s: Stmt, depth: int) -> list:
    pad = "  " * depth
    r = render_expr
    if isinstance(s, SLet):
        return [f"{pad}let {s.name} : {s.type} = {r(s.e)}"]
    if isinstance(s, SVar):
        return [f"{pad}var {s.name} : {s.type} = {r(s.e)}"]
    if isinstance(s, SAssign):
        return [f"{pad}{s.name} = {r(s.e)}"]
    if isinstance(s, SStore):
        return [f"{pad}{s.buffer}[{r(s.index)}] = {r(s.value)}"]
    if isinstance(s, SStoreVia):
        return [f"{pad}{s.table}[{r(s.entry)}][{r(s.index)}] = {r(s.value)}"]
    if isinstance(s, STgStore):
        return [f"{pad}{s.array}[{r(s.index)}] = {r(s.value)}"]
    if isinstance(s, SLoadPack):
        return [f"{pad}let ({', '.join(s.names)}) : {s.type} = {s.buffer}.pack{len(s.names)}[{r(s.index)}]"]
    if isinstance(s, (SStorePack, STgStorePack)):
        where = s.buffer if isinstance(s, SStorePack) else s.array
        return [f"{pad}{where}.pack{len(s.values)}[{r(s.index)}] = ({', '.join(r(v) for v in s.values)})"]
    if isinstance(s, SLoadPackVia):
        return [f"{pad}let ({', '.join(s.names)}) : {s.type} = {s.table}[{r(s.entry)}].pack{len(s.names)}[{r(s.index)}]"]
    if isinstance(s, SIf):
        out = [f"{pad}if {s.region} {r(s.cond)} {{"]
        for t in s.then:
            out += render_stmt(t, depth + 1)
        if s.orelse:
            out.append(f"{pad}}} else {{")
            for t in s.orelse:
                out += render_stmt(t, depth + 1)
        return out + [f"{pad}}}"]
    if isinstance(s, SFor):
        out = [f"{pad}for {s.region} {s.var} = {r(s.start)} until {r(s.end)} step {r(s.step)} {{"]
        for t in s.body:
            out += render_stmt(t, depth + 1)
        return out + [f"{pad}}}"]
    if isinstance(s, SBarrier):
        return [f"{pad}barrier"]
    if isinstance(s, SSimdBarrier):
        return [f"{pad}simd barrier"]
    if isinstance(s, SSimd):
        return [f"{pad}let {s.name} : {s.type} = {s.op}({r(s.e)})"]
    if isinstance(s, SFragVar):
        return [f"{pad}fragment {s.name} : {s.type}[8x8] = 0"]
    if isinstance(s, SFragLoad):
        t = "_t" if s.transposed else ""
        return [f"{pad}{s.name} = {_mem(s.mem)}.fragment{t}[{r(s.index)}, stride {r(s.stride)}]"]
    if isinstance(s, SFragMma):
        return [f"{pad}{s.d} = {s.a} * {s.b} + {s.c}"]
    if isinstance(s, SFragConvert):
        return [f"{pad}{s.d} = f32({s.s})"]
    if isinstance(s, SFragScaleRows):
        return [f"{pad}{s.frag} = rows({s.frag}) * {s.array}[{r(s.index)} + row]"]
    if isinstance(s, SFragStore):
        return [f"{pad}{_mem(s.mem)}.fragment[{r(s.index)}, stride {r(s.stride)}] = {s.name}"]
    raise TypeError(f"not a statement: {s!r}")


def render_kernel(k: Kernel) -> str:
    lines = ["ir 1", f"kernel {k.name} threads {k.threads} simd {k.simd_width} groups {render_expr(k.groups)}"]
    for p in k.params:
        role = "" if p.dim is None else f" dim {p.dim.min}..{p.dim.max} multiple of {p.dim.multiple_of}"
        lines.append(f"  param {p.name} : {p.type}{role}")
    for b in k.buffers:
        lines.append(f"  buffer {b.name} : {b.access} {b.type}[{render_expr(b.extent)}] align {b.align}"
                     + (" apart" if b.apart else ""))
    for t in k.tables:
        acc = "" if t.access == READ else t.access + " "
        lines.append(f"  table {t.name} : {acc}{render_expr(t.entries)} x {t.type}[{render_expr(t.extent)}] "
                     f"align {t.align}" + (" distinct" if t.distinct else "") + (" apart" if t.apart else ""))
    for a in k.tg_arrays:
        lines.append(f"  threadgroup {a.name} : {a.type}[{a.count}]")
    lines.append("{")
    for s in k.body:
        lines += render_stmt(s, 1)
    lines.append("}")
    return "\n".join(lines) + "\n"


def fnv1a64(data: bytes) -> int:
    """Abi.hs:258-262."""
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def ir_hash(k: Kernel) -> int:
    """FNV-1a over the kernel's text (Abi.hs:255-256)."""
    return fnv1a64(render_kernel(k).encode())


def hex64(w: int) -> str:
    return f"0x{w:016x}"
