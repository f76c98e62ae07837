"""Programs: what a model computes in one step, as dataflow
(src/FuryKernel/Program/Graph.hs).

A program is straight-line dataflow over row values: a step runs ``m`` rows
at once, one per token, and every value holds a row of elements for each.
Values are made by nodes, each one operation of a small vocabulary; what a
program reads comes from its sources (activations, row integers, weights,
tables, KV caches).  Ids are plain ints.

One addition to the reference's vocabulary: ``Gelu`` has a second form,
``SILU`` (x / (1 + e^-x)), next to ``GELU_TANH``, so that ``GeluMul`` states a
SiLU-gated FFN (the reference has GELU-tanh only: Graph.hs:283-291).
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Optional, Union

# Scalar types (src/FuryKernel/Type.hs:43-52), by their short names.
F32, F16, BF16, I32, U32, I8, U8, BOOL = "f32", "f16", "bf16", "i32", "u32", "i8", "u8", "bool"
SCALAR_SIZE = {F32: 4, F16: 2, BF16: 2, I32: 4, U32: 4, I8: 1, U8: 1, BOOL: 1}


@dataclass(frozen=True)
class Shape:
    """A row's elements: ``width`` of them in segments of ``segment`` (Graph.hs:89-93)."""

    width: int
    segment: int


def whole_row(n: int) -> Shape:
    return Shape(n, n)


def segment_count(s: Shape) -> int:
    return 0 if s.segment == 0 else s.width // s.segment


# Sources ----------------------------------------------------------------------


@dataclass(frozen=True)
class SInput:
    """A per-row activation from the engine, of this element type."""

    shape: Shape
    type: str


@dataclass(frozen=True)
class SRowInts:
    """Per row, ``count`` u32, each below ``bound``."""

    count: int
    bound: int


@dataclass(frozen=True)
class SWeight:
    """A weight: its shape (outputs first), element type and layout id."""

    dims: tuple
    type: str
    layout: str


@dataclass(frozen=True)
class STable:
    """A table of ``entries`` weights, each of this shape, type and layout."""

    entries: int
    dims: tuple
    type: str
    layout: str


@dataclass(frozen=True)
class Ring:
    """``Ring slots kvHeads length headDim`` (Graph.hs:137-143): position p of
    slot s, head h starts at ((s * kvHeads + h) * length + p mod length) * headDim."""

    slots: int
    kv_heads: int
    length: int
    head_dim: int


@dataclass(frozen=True)
class Paged:
    """``Paged blocks blockSize kvHeads headDim`` (Graph.hs:144-152): position p,
    head h at (h * blockSize + p mod blockSize) * headDim in block table[p / blockSize]."""

    blocks: int
    block_size: int
    kv_heads: int
    head_dim: int


CacheLayout = Union[Ring, Paged]

# CacheElem (Graph.hs:164-179): the type a cache rounds its stores to.
CACHE_BF16, CACHE_F16 = "bf16", "f16"


@dataclass(frozen=True)
class SCache:
    layout: CacheLayout
    elem: str


SourceKind = Union[SInput, SRowInts, SWeight, STable, SCache]


@dataclass(frozen=True)
class Source:
    id: int
    name: str
    kind: SourceKind


# Values, nodes and operations ----------------------------------------------


@dataclass(frozen=True)
class Value:
    id: int
    name: str
    shape: Shape
    type: str


ROPE_HALVES = "halves"
GELU_TANH = "gelu_tanh"
SILU = "silu"
SOFTMAX_OF_TOPK = "softmax_of_top_k"


@dataclass(frozen=True)
class RopeSpec:
    theta: float
    rotated: int
    axes: int = 1
    pairs: str = ROPE_HALVES


@dataclass(frozen=True)
class Reach:
    source: int
    ahead: int


@dataclass(frozen=True)
class AttnSpec:
    heads: int
    kv_heads: int
    head_dim: int
    window: Optional[int]
    scale: float
    reach: Optional[Reach] = None


@dataclass(frozen=True)
class RouteSpec:
    k: int
    expert_scale: Optional[int] = None
    weights: str = SOFTMAX_OF_TOPK


@dataclass(frozen=True)
class StoreAt:
    cache: int
    positions: int
    sequences: int


@dataclass(frozen=True)
class AttendTo:
    keys: int
    values: int
    positions: int
    sequences: int


# Operations (Graph.hs:299-360).
@dataclass(frozen=True)
class Input:
    source: int


@dataclass(frozen=True)
class Linear:
    weight: int
    segment: int
    x: int


@dataclass(frozen=True)
class LinearRouted:
    table: int
    ids: int
    x: int


@dataclass(frozen=True)
class RmsNorm:
    eps: float
    gamma: Optional[int]
    factor: float
    x: int


@dataclass(frozen=True)
class Add:
    a: int
    b: int


@dataclass(frozen=True)
class Concat:
    a: int
    b: int


@dataclass(frozen=True)
class ScaleBy:
    weight: int
    x: int


@dataclass(frozen=True)
class GatedGelu:
    form: str
    x: int


@dataclass(frozen=True)
class GeluMul:
    form: str
    a: int
    b: int


@dataclass(frozen=True)
class Rope:
    spec: RopeSpec
    positions: int
    x: int


@dataclass(frozen=True)
class Softcap:
    cap: float
    x: int


@dataclass(frozen=True)
class Route:
    spec: RouteSpec
    x: int


@dataclass(frozen=True)
class CombineRanks:
    weights: int
    x: int


@dataclass(frozen=True)
class KvStore:
    at: StoreAt
    x: int


@dataclass(frozen=True)
class Attend:
    spec: AttnSpec
    q: int
    to: AttendTo


@dataclass(frozen=True)
class Gather:
    table: int
    tokens: int
    factor: float


@dataclass(frozen=True)
class Standardize:
    bias: int
    scale: int
    factor: float
    x: int


@dataclass(frozen=True)
class ArgMax:
    x: int


Op = Union[Input, Linear, LinearRouted, RmsNorm, Add, Concat, ScaleBy, GatedGelu, GeluMul, Rope, Softcap, Route,
           CombineRanks, KvStore, Attend, Gather, Standardize, ArgMax]


def op_values(op: Op) -> list[int]:
    """The values an operation reads, in order (Graph.hs:363-382)."""
    if isinstance(op, (Input, Gather)):
        return []
    if isinstance(op, Linear):
        return [op.x]
    if isinstance(op, LinearRouted):
        return [op.ids, op.x]
    if isinstance(op, (RmsNorm, ScaleBy, GatedGelu, Rope, Softcap, Route, KvStore, Standardize, ArgMax)):
        return [op.x]
    if isinstance(op, (Add, Concat, GeluMul)):
        return [op.a, op.b]
    if isinstance(op, CombineRanks):
        return [op.weights, op.x]
    if isinstance(op, Attend):
        return [op.q]
    raise TypeError(op)


def op_sources(op: Op) -> list[int]:
    """The sources an operation reads or, for a cache, writes (Graph.hs:385-404)."""
    if isinstance(op, Input):
        return [op.source]
    if isinstance(op, Linear):
        return [op.weight]
    if isinstance(op, LinearRouted):
        return [op.table]
    if isinstance(op, RmsNorm):
        return [] if op.gamma is None else [op.gamma]
    if isinstance(op, ScaleBy):
        return [op.weight]
    if isinstance(op, Rope):
        return [op.positions]
    if isinstance(op, Route):
        return [] if op.spec.expert_scale is None else [op.spec.expert_scale]
    if isinstance(op, KvStore):
        return [op.at.cache, op.at.positions, op.at.sequences]
    if isinstance(op, Attend):
        extra = [] if op.spec.reach is None else [op.spec.reach.source]
        return [op.to.keys, op.to.values, op.to.positions, op.to.sequences] + extra
    if isinstance(op, Gather):
        return [op.table, op.tokens]
    if isinstance(op, Standardize):
        return [op.bias, op.scale]
    return []


@dataclass(frozen=True)
class Node:
    id: int
    name: str
    op: Op
    outputs: tuple


@dataclass(frozen=True)
class Output:
    name: str
    value: int


@dataclass
class Program:
    name: str
    sources: list = field(default_factory=list)
    values: list = field(default_factory=list)
    nodes: list = field(default_factory=list)
    outputs: list = field(default_factory=list)

    def value(self, v: int) -> Optional[Value]:
        return next((x for x in self.values if x.id == v), None)

    def source(self, s: int) -> Optional[Source]:
        return next((x for x in self.sources if x.id == s), None)

    def node(self, n: int) -> Optional[Node]:
        return next((x for x in self.nodes if x.id == n), None)

    def producer(self, v: int) -> Optional[Node]:
        return next((n for n in self.nodes if v in n.outputs), None)

    def source_named(self, name: str) -> Optional[Source]:
        return next((s for s in self.sources if s.name == name), None)

    def value_named(self, name: str) -> Optional[Value]:
        return next((v for v in self.values if v.name == name), None)


def cache_kv_heads(layout: CacheLayout) -> int:
    return layout.kv_heads


def cache_head_dim(layout: CacheLayout) -> int:
    return layout.head_dim


def double_text(d: float) -> str:
    """A double by its bits, as renderProgram writes it (Graph.hs:520)."""
    return "f64:0x" + format(struct.unpack("<Q", struct.pack("<d", d))[0], "x")


def render_program(p: Program) -> str:
    """The deterministic text form (Graph.hs:430-525)."""

    def shape(sh: Shape) -> str:
        return f"[{sh.width}/{sh.segment}]"

    def dims(ds) -> str:
        return "[" + ", ".join(str(d) for d in ds) + "]"

    def kind(k) -> str:
        if isinstance(k, SInput):
            return f"input {shape(k.shape)} {k.type}"
        if isinstance(k, SRowInts):
            return f"row_ints {k.count} below {k.bound}"
        if isinstance(k, SWeight):
            return f"weight {dims(k.dims)} {k.type} {k.layout}"
        if isinstance(k, STable):
            return f"table {k.entries} x {dims(k.dims)} {k.type} {k.layout}"
        lay = k.layout
        if isinstance(lay, Ring):
            lt = f"ring slots {lay.slots} heads {lay.kv_heads} length {lay.length} dim {lay.head_dim}"
        else:
            lt = f"paged blocks {lay.blocks} size {lay.block_size} heads {lay.kv_heads} dim {lay.head_dim}"
        return f"cache {lt} {k.elem}"

    def value(v: int) -> str:
        val = p.value(v)
        return val.name if val else f"%{v}"

    def src(s: int) -> str:
        x = p.source(s)
        return x.name if x else "?"

    def info(v: int) -> str:
        val = p.value(v)
        return f"{shape(val.shape)} {val.type}" if val else "?"

    def op(o) -> str:
        if isinstance(o, Input):
            return f"input({src(o.source)})"
        if isinstance(o, Linear):
            return f"linear({src(o.weight)}, {value(o.x)}) segment {o.segment}"
        if isinstance(o, LinearRouted):
            return f"linear_routed({src(o.table)}, {value(o.ids)}, {value(o.x)})"
        if isinstance(o, RmsNorm):
            g = "" if o.gamma is None else f", gamma {src(o.gamma)}"
            return f"rmsnorm({value(o.x)}, eps {double_text(o.eps)}{g}, factor {double_text(o.factor)})"
        if isinstance(o, Add):
            return f"add({value(o.a)}, {value(o.b)})"
        if isinstance(o, Concat):
            return f"concat({value(o.a)}, {value(o.b)})"
        if isinstance(o, ScaleBy):
            return f"scale_by({src(o.weight)}, {value(o.x)})"
        if isinstance(o, GatedGelu):
            return f"gated_{'gelu' if o.form == GELU_TANH else 'silu'}({value(o.x)})"
        if isinstance(o, GeluMul):
            return f"{'gelu' if o.form == GELU_TANH else 'silu'}_mul({value(o.a)}, {value(o.b)})"
        if isinstance(o, Rope):
            axes = "" if o.spec.axes == 1 else f", axes {o.spec.axes}"
            return (f"rope({value(o.x)}, {src(o.positions)}, theta {double_text(o.spec.theta)}, "
                    f"rotated {o.spec.rotated}{axes})")
        if isinstance(o, Softcap):
            return f"softcap({value(o.x)}, {double_text(o.cap)})"
        if isinstance(o, Route):
            sc = "" if o.spec.expert_scale is None else f", scale {src(o.spec.expert_scale)}"
            return f"route({value(o.x)}, k {o.spec.k}{sc})"
        if isinstance(o, CombineRanks):
            return f"combine_ranks({value(o.weights)}, {value(o.x)})"
        if isinstance(o, KvStore):
            return f"kv_store({src(o.at.cache)}, {src(o.at.positions)}, {src(o.at.sequences)}, {value(o.x)})"
        if isinstance(o, Attend):
            a = o.spec
            w = "" if a.window is None else f", window {a.window}"
            r = "" if a.reach is None else f", reach {src(a.reach.source)} ahead {a.reach.ahead}"
            parts = ", ".join([value(o.q), src(o.to.keys), src(o.to.values), src(o.to.positions), src(o.to.sequences)])
            return (f"attend({parts}, heads {a.heads}/{a.kv_heads}, dim {a.head_dim}{w}, "
                    f"scale {double_text(a.scale)}{r})")
        if isinstance(o, Gather):
            return f"gather({src(o.table)}, {src(o.tokens)}, factor {double_text(o.factor)})"
        if isinstance(o, Standardize):
            return f"standardize({value(o.x)}, {src(o.bias)}, {src(o.scale)}, factor {double_text(o.factor)})"
        if isinstance(o, ArgMax):
            return f"argmax({value(o.x)})"
        raise TypeError(o)

    lines = [f"program {p.name}"]
    lines += [f"  source {s.name} : {kind(s.kind)}" for s in p.sources]
    for n in p.nodes:
        outs = ", ".join(f"{value(v)} : {info(v)}" for v in n.outputs)
        lines.append("  " + outs + (" = " if n.outputs else "") + n.name + " " + op(n.op))
    lines += [f"  output {o.name} = {value(o.value)}" for o in p.outputs]
    return "\n".join(lines) + "\n"
