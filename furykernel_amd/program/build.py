"""Writing programs (src/FuryKernel/Program/Build.hs).

``ProgramBuilder`` is the ``P`` monad as an object: each method adds a source
or a node and returns its handle.  Sources keep their names exactly (the
engine binds them by name); a value or node named as an earlier one takes a
suffix ``_1``, ``_2``, ... (Build.hs:109-115).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional

from .graph import (
    BF16, F32, U32, Add, ArgMax, AttendTo, Attend, AttnSpec, CACHE_BF16, CombineRanks, Concat, GatedGelu, Gather,
    GELU_TANH, GeluMul, Input, KvStore, Linear, LinearRouted, Node, Output, Program, RmsNorm, Rope, RopeSpec, Route,
    RouteSpec, SCache, ScaleBy, Shape, SInput, Softcap, Source, SRowInts, STable, Standardize, StoreAt, SWeight, Value,
    whole_row)


@dataclass(frozen=True)
class Val:
    id: int
    shape: Shape


@dataclass(frozen=True)
class Src:
    id: int
    kind: object


class ProgramBuilder:
    def __init__(self, name: str):
        self.name = name
        self.names: set[str] = set()
        self.sources: list[Source] = []
        self.values: list[Value] = []
        self.nodes: list[Node] = []
        self.outputs: list[Output] = []

    def finish(self) -> Program:
        return Program(self.name, list(self.sources), list(self.values), list(self.nodes), list(self.outputs))

    # Names ----------------------------------------------------------------

    def _fresh(self, base: str) -> str:
        n, i = base, 0
        while n in self.names:
            i += 1
            n = f"{base}_{i}"
        self.names.add(n)
        return n

    def _add_source(self, name: str, kind) -> Src:
        s = Source(len(self.sources), name, kind)
        self.names.add(name)
        self.sources.append(s)
        return Src(s.id, kind)

    def _add_node(self, name: str, op, outs: list[tuple[str, Shape, str]]) -> list[Val]:
        vals = []
        for vname, sh, t in outs:
            vn = self._fresh(vname)
            v = Value(len(self.values), vn, sh, t)
            self.values.append(v)
            vals.append((Val(v.id, sh), vn))
        n = vals[0][1] if vals else self._fresh(name)
        self.nodes.append(Node(len(self.nodes), n, op, tuple(v.id for v, _ in vals)))
        return [v for v, _ in vals]

    def _one(self, name: str, op, sh: Shape, t: str) -> Val:
        return self._add_node(name, op, [(name, sh, t)])[0]

    # Sources --------------------------------------------------------------

    def input(self, name: str, sh: Shape, t: str = F32) -> Val:
        s = self._add_source(name, SInput(sh, t))
        v = Value(len(self.values), name, sh, t)
        self.values.append(v)
        self.nodes.append(Node(len(self.nodes), name, Input(s.id), (v.id,)))
        return Val(v.id, sh)

    def row_ints(self, name: str, n: int, bound: int) -> Src:
        return self._add_source(name, SRowInts(n, bound))

    def weight(self, name: str, dims: list[int], t: str = BF16) -> Src:
        """A weight in the model's ``out_in`` layout (two dimensions) or
        ``row_major``: bf16 as ``weight`` has it (Build.hs:170-176), or the
        element type given, which the gate allows (Check.hs:105-121)."""
        return self._add_source(name, SWeight(tuple(dims), t, "out_in" if len(dims) == 2 else "row_major"))

    def rows_f32(self, name: str, dims: list[int]) -> Src:
        return self._add_source(name, SWeight(tuple(dims), F32, "row_major"))

    def table(self, name: str, n: int, dims: list[int], t: str = BF16) -> Src:
        return self._add_source(name, STable(n, tuple(dims), t, "out_in"))

    def cache(self, name: str, layout, elem: str = CACHE_BF16) -> Src:
        return self._add_source(name, SCache(layout, elem))

    # Operations -------------------------------------------------------------

    @staticmethod
    def _weight_rows(s: Src) -> int:
        if isinstance(s.kind, SWeight):
            return s.kind.dims[0] if s.kind.dims else 0
        if isinstance(s.kind, STable):
            return s.kind.dims[0] if s.kind.dims else 0
        return 0

    def linear(self, name: str, w: Src, seg: int, x: Val) -> Val:
        n = self._weight_rows(w)
        seg2 = n if seg == 0 else seg
        return self._one(name, Linear(w.id, seg2, x.id), Shape(n, seg2), F32)

    def linear_routed(self, name: str, t: Src, ids: Val, x: Val) -> Val:
        n = self._weight_rows(t)
        ranks = ids.shape.width
        return self._one(name, LinearRouted(t.id, ids.id, x.id), Shape(ranks * n, n), F32)

    def rmsnorm(self, name: str, eps: float, gamma: Optional[Src], factor: float, x: Val) -> Val:
        return self._one(name, RmsNorm(eps, None if gamma is None else gamma.id, factor, x.id), x.shape, F32)

    def add(self, name: str, a: Val, b: Val) -> Val:
        return self._one(name, Add(a.id, b.id), a.shape, F32)

    def concatenate(self, name: str, a: Val, b: Val) -> Val:
        return self._one(name, Concat(a.id, b.id), Shape(a.shape.width + b.shape.width, a.shape.segment), F32)

    def scale_by(self, name: str, w: Src, x: Val) -> Val:
        return self._one(name, ScaleBy(w.id, x.id), x.shape, F32)

    def gated_gelu(self, name: str, x: Val, form: str = GELU_TANH) -> Val:
        return self._one(name, GatedGelu(form, x.id), Shape(x.shape.width // 2, x.shape.segment // 2), F32)

    def gelu_mul(self, name: str, a: Val, b: Val, form: str = GELU_TANH) -> Val:
        return self._one(name, GeluMul(form, a.id, b.id), a.shape, F32)

    def rope(self, name: str, spec: RopeSpec, pos: Src, x: Val) -> Val:
        return self._one(name, Rope(spec, pos.id, x.id), x.shape, F32)

    def softcap(self, name: str, cap: float, x: Val) -> Val:
        return self._one(name, Softcap(cap, x.id), x.shape, F32)

    def route(self, name: str, k: int, scale: Optional[Src], x: Val) -> tuple[Val, Val]:
        ids, ws = self._add_node(name, Route(RouteSpec(k, None if scale is None else scale.id), x.id),
                                 [(name + "_ids", whole_row(k), U32), (name + "_weights", whole_row(k), F32)])
        return ids, ws

    def combine_ranks(self, name: str, w: Val, x: Val) -> Val:
        return self._one(name, CombineRanks(w.id, x.id), whole_row(x.shape.segment), F32)

    def kv_store(self, name: str, cache: Src, positions: Src, sequences: Src, x: Val) -> None:
        self._add_node(name, KvStore(StoreAt(cache.id, positions.id, sequences.id), x.id), [])

    def attend(self, name: str, spec: AttnSpec, q: Val, keys: Src, values: Src, positions: Src,
               sequences: Src) -> Val:
        return self._one(name, Attend(spec, q.id, AttendTo(keys.id, values.id, positions.id, sequences.id)), q.shape,
                         F32)

    def gather(self, name: str, t: Src, tok: Src, factor: float) -> Val:
        width = t.kind.dims[1] if isinstance(t.kind, SWeight) and len(t.kind.dims) == 2 else 0
        return self._one(name, Gather(t.id, tok.id, factor), whole_row(width), F32)

    def standardize(self, name: str, bias: Src, scale: Src, factor: float, x: Val) -> Val:
        return self._one(name, Standardize(bias.id, scale.id, factor, x.id), x.shape, F32)

    def argmax(self, name: str, x: Val) -> Val:
        return self._one(name, ArgMax(x.id), whole_row(1), U32)

    def output(self, name: str, v: Val) -> None:
        self.outputs.append(Output(name, v.id))


def program(name: str, body: Callable[[ProgramBuilder], None]) -> Program:
    b = ProgramBuilder(name)
    body(b)
    return b.finish()


__all__ = ["ProgramBuilder", "program", "Val", "Src", "SCache", "AttnSpec", "RopeSpec", "RouteSpec", "Gather"]
