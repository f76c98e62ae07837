"""Writing kernels (src/FuryKernel/Build.hs): a builder that records the IR
a kernel's author states, with the typed surface's rules checked as the
kernel is built.

A kernel has the reference's three phases: its interface (dimensions,
parameters, buffers, tables, threads, grid), its threadgroup arrays, then its
body.  Here they are calls on one ``KernelBuilder``; the body's blocks are
``with`` statements::

    k = KernelBuilder("scale", ROCM)
    n = k.dim("n", DimRange(1, 65536, 1))
    s = k.param("s", F32)
    x = k.buffer("x", READ, BF16, n)
    y = k.buffer("y", WRITE, BF16, n)
    k.threads(64)
    k.groups(1)
    with k.strided("i", n) as i:
        v = k.let("v", widen(F32, k.load(x, i)))
        k.store(y, i, narrow(BF16, v * s))
    kernel, problems = k.done()

What Haskell's types refuse at compile time (arithmetic on a storage type,
operands of two types, a barrier under a branch, a SIMD-group operation
where lanes diverge, a pack wider than the target's lane loads) raises
``BuildError`` here as the kernel is built; what the reference's builder
notices itself (a name declared twice, no thread count or grid) is a
problem returned with the kernel, as ``kernelProblems`` (Build.hs:251-257).
"""

from __future__ import annotations

import contextlib
import struct
from dataclasses import dataclass
from fractions import Fraction
from typing import Optional

from ..program.graph import BF16, BOOL, F16, F32, I8, I32, SCALAR_SIZE, U8, U32
from . import ir as I


class BuildError(TypeError):
    """What the reference's types refuse: the kernel is not built."""


@dataclass(frozen=True)
class TargetCaps:
    """A target's limits (src/FuryKernel/Target.hs:73-97)."""

    name: str
    simd_width: int
    max_threads: int
    tg_mem_bytes: int
    max_buffers: int
    lane_load_max: int
    fragments: tuple = ()


# The MI355X (gfx950): 64-lane wavefronts, 1024 threads a workgroup, 64 KiB of
# LDS a kernel declares statically (the CU has 160 KiB), one 16-byte load a
# lane, fragments of bf16, f16 and f32.
ROCM = TargetCaps("MI355X", 64, 1024, 65536, 31, 16, (BF16, F16, F32))

NUM = (F32, F16, I32, U32)
FLOAT = (F32, F16)
INT = (I32, U32)
WIDEN = {(BF16, F32), (F16, F32), (I8, I32), (U8, U32)}
NARROW = {(F32, BF16), (F32, F16)}
NARROW_INT = {(I32, I8), (U32, U8)}


# ---------------------------------------------------------------------------
# Literals: rounded once from their exact value.

def _round_binary(q: Fraction, p: int, emin: int, emax: int, ebits: int) -> int:
    """The bits of the binary format (p significand bits, normal exponents
    emin..emax) nearest q, ties to even, overflow to infinity."""
    sign = 1 if q < 0 else 0
    a = abs(q)
    top = 1 << (ebits + p - 1)
    if a == 0:
        return sign * top
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    scaled = a / Fraction(2) ** (e - (p - 1))
    n = scaled.numerator // scaled.denominator
    r = scaled - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    if n == 1 << p:
        n >>= 1
        e += 1
    if e > emax:
        return sign * top | (((1 << ebits) - 1) << (p - 1))
    if n < 1 << (p - 1):
        return sign * top | n
    return sign * top | ((e + (1 << (ebits - 1)) - 1) << (p - 1)) | (n - (1 << (p - 1)))


def f32_rational(q: Fraction) -> int:
    return _round_binary(Fraction(q), 24, -126, 127, 8)


def f16_rational(q: Fraction) -> int:
    """rationalF16 (src/FuryKernel/Numerics.hs): the exact value rounded once."""
    return _round_binary(Fraction(q), 11, -14, 15, 5)


def _exact(x) -> Fraction:
    """A literal's exact value: a Python float taken as the decimal it was
    written as (its shortest repr), as Haskell reads a literal."""
    if isinstance(x, Fraction):
        return x
    if isinstance(x, int):
        return Fraction(x)
    return Fraction(repr(float(x)))


def literal(t: str, x) -> I.Lit:
    """A literal of type t from a Python number (Build.hs:324-432)."""
    if isinstance(x, bool) or t == BOOL:
        if t != BOOL:
            raise BuildError(f"a bool literal where {t} is wanted")
        return I.Lit(BOOL, int(bool(x)))
    if t == F32:
        if isinstance(x, float) and (x != x or x in (float("inf"), float("-inf"))):
            return I.lit_f32(x)
        if isinstance(x, float) and x == 0.0:
            return I.Lit(F32, I.f32_bits(x))
        return I.Lit(F32, f32_rational(_exact(x)))
    if t == F16:
        if isinstance(x, float) and x != x:
            return I.Lit(F16, 0x7E00)
        if isinstance(x, float) and x in (float("inf"), float("-inf")):
            return I.Lit(F16, 0x7C00 if x > 0 else 0xFC00)
        if isinstance(x, float) and x == 0.0:
            return I.Lit(F16, 0x8000 if str(x).startswith("-") else 0)
        return I.Lit(F16, f16_rational(_exact(x)))
    if t in (I32, U32):
        if not isinstance(x, int):
            raise BuildError(f"an integer literal of {t} from {x!r}")
        lo, hi = (-2**31, 2**31 - 1) if t == I32 else (0, 2**32 - 1)
        if not lo <= x <= hi:
            raise BuildError(f"FuryKernel.Build: the literal {x} is outside {t}'s range, {lo} to {hi}.")
        return I.Lit(t, x)
    raise BuildError(f"{t} is a storage type, with no literals of its own")


def f32(x: float) -> "E":
    """A binary32 literal of a value binary32 holds, every NaN the canonical
    one (Build.hs:1222-1228)."""
    return E(I.ELit(I.lit_f32(x)), F32)


# ---------------------------------------------------------------------------
# Typed expressions

class E:
    """An expression of a scalar type (Build.hs's ``Exp a``)."""

    __slots__ = ("ir", "type")

    def __init__(self, ir_expr, t: str):
        self.ir = ir_expr
        self.type = t

    def _other(self, o) -> "E":
        if isinstance(o, E):
            if o.type != self.type:
                raise BuildError(f"operands of {self.type} and {o.type}")
            return o
        return E(I.ELit(literal(self.type, o)), self.type)

    def _num(self, op, o, rev=False) -> "E":
        o = self._other(o)
        if self.type not in NUM:
            raise BuildError(f"{self.type} has no arithmetic: widen it first")
        a, b = (o, self) if rev else (self, o)
        return E(I.EBin(op, a.ir, b.ir), self.type)

    def __add__(self, o):
        return self._num("add", o)

    def __radd__(self, o):
        return self._num("add", o, rev=True)

    def __sub__(self, o):
        return self._num("sub", o)

    def __rsub__(self, o):
        return self._num("sub", o, rev=True)

    def __mul__(self, o):
        return self._num("mul", o)

    def __rmul__(self, o):
        return self._num("mul", o, rev=True)

    def __truediv__(self, o):
        if self.type not in FLOAT:
            raise BuildError(f"{self.type} divides with quot and rem")
        return self._num("div", o)

    def __rtruediv__(self, o):
        if self.type not in FLOAT:
            raise BuildError(f"{self.type} divides with quot and rem")
        return self._num("div", o, rev=True)

    def __neg__(self):
        if self.type not in NUM:
            raise BuildError(f"{self.type} has no arithmetic")
        return E(I.EUn("neg", self.ir), self.type)

    def __abs__(self):
        if self.type not in NUM:
            raise BuildError(f"{self.type} has no arithmetic")
        return E(I.EUn("abs", self.ir), self.type)

    def _cmp(self, op, o) -> "E":
        o = self._other(o)
        if self.type not in NUM:
            raise BuildError(f"{self.type} has no order")
        return E(I.EBin(op, self.ir, o.ir), BOOL)

    def __lt__(self, o):
        return self._cmp("lt", o)

    def __le__(self, o):
        return self._cmp("le", o)

    def __gt__(self, o):
        return self._cmp("gt", o)

    def __ge__(self, o):
        return self._cmp("ge", o)

    def eq(self, o):
        if self.type == BOOL:
            return E(I.EBin("eq", self.ir, self._other(o).ir), BOOL)
        return self._cmp("eq", o)

    def ne(self, o):
        if self.type == BOOL:
            return E(I.EBin("ne", self.ir, self._other(o).ir), BOOL)
        return self._cmp("ne", o)

    def __and__(self, o):
        if self.type != BOOL:
            raise BuildError("&& of bools only")
        return E(I.EBin("and", self.ir, self._other(o).ir), BOOL)

    def __or__(self, o):
        if self.type != BOOL:
            raise BuildError("|| of bools only")
        return E(I.EBin("or", self.ir, self._other(o).ir), BOOL)

    def __invert__(self):
        if self.type != BOOL:
            raise BuildError("not of bools only")
        return E(I.EUn("not", self.ir), BOOL)

    __hash__ = None  # expressions are not keys


def lit(t: str, x) -> E:
    return E(I.ELit(literal(t, x)), t)


def u32(n: int) -> E:
    return lit(U32, n)


def select(c: E, a, b) -> E:
    if c.type != BOOL:
        raise BuildError("a select's condition is a bool")
    if not isinstance(a, E):
        a = b._other(a) if isinstance(b, E) else None
    if not isinstance(b, E):
        b = a._other(b)
    a._other(b)
    return E(I.ESelect(c.ir, a.ir, b.ir), a.type)


def _bin(op, a: E, b, kinds, what) -> E:
    if not isinstance(a, E):
        a, b = b._other(a), b
    b = a._other(b)
    if a.type not in kinds:
        raise BuildError(f"{what} of {a.type}")
    return E(I.EBin(op, a.ir, b.ir), a.type)


def min_e(a, b) -> E:
    return _bin("min", a, b, NUM, "a minimum")


def max_e(a, b) -> E:
    return _bin("max", a, b, NUM, "a maximum")


def quot(a, b) -> E:
    return _bin("div", a, b, INT, "an integer quotient")


def rem(a, b) -> E:
    return _bin("rem", a, b, INT, "an integer remainder")


def _float_un(op, a: E) -> E:
    if a.type not in FLOAT:
        raise BuildError(f"{op} of {a.type}")
    return E(I.EUn(op, a.ir), a.type)


def sqrt_e(a):
    return _float_un("sqrt", a)


def rsqrt_e(a):
    return _float_un("rsqrt", a)


def exp_e(a):
    return _float_un("exp", a)


def log_e(a):
    return _float_un("log", a)


def tanh_e(a):
    return _float_un("tanh", a)


def fma_e(a: E, b, c) -> E:
    if a.type not in FLOAT:
        raise BuildError(f"an fma of {a.type}")
    b, c = a._other(b), a._other(c)
    return E(I.EFma(a.ir, b.ir, c.ir), a.type)


def widen(t: str, a: E) -> E:
    if (a.type, t) not in WIDEN:
        raise BuildError(f"{a.type} does not widen to {t}")
    return E(I.EConvert(t, a.ir), t)


def narrow(t: str, a: E) -> E:
    if (a.type, t) not in NARROW:
        raise BuildError(f"{a.type} does not narrow to {t}")
    return E(I.EConvert(t, a.ir), t)


def narrow_clamped(t: str, a: E) -> E:
    if (a.type, t) not in NARROW_INT:
        raise BuildError(f"{a.type} does not narrow to {t}")
    return E(I.ENarrowInt("clamp", t, a.ir), t)


def narrow_wrapped(t: str, a: E) -> E:
    if (a.type, t) not in NARROW_INT:
        raise BuildError(f"{a.type} does not narrow to {t}")
    return E(I.ENarrowInt("wrap", t, a.ir), t)


def to_f32(a: E) -> E:
    if a.type != U32:
        raise BuildError("toF32 of u32 only")
    return E(I.EConvert(F32, a.ir), F32)


thread_index = E(I.EBuiltin("thread"), U32)
group_index = E(I.EBuiltin("group"), U32)
simd_lane = E(I.EBuiltin("lane"), U32)
simd_group_index = E(I.EBuiltin("simd_group"), U32)
true_ = E(I.ELit(I.Lit(BOOL, 1)), BOOL)
false_ = E(I.ELit(I.Lit(BOOL, 0)), BOOL)


# ---------------------------------------------------------------------------
# Handles of the interface

@dataclass(frozen=True)
class Buf:
    name: str
    access: str
    type: str
    align: int


@dataclass(frozen=True)
class Tab:
    name: str
    access: str
    type: str
    align: int


@dataclass(frozen=True)
class Tg:
    name: str
    type: str
    count: int


@dataclass(frozen=True)
class Var:
    name: str
    type: str

    @property
    def get(self) -> E:
        return E(I.EVar(self.name), self.type)


@dataclass(frozen=True)
class Frag:
    name: str
    type: str


@dataclass(frozen=True)
class Finding:
    rule: str
    message: str


UNIFORM, SIMD_UNIFORM, DIVERGENT = "uniform", "simd_uniform", "divergent"


def _meet(a: str, b: str) -> str:
    order = {UNIFORM: 0, SIMD_UNIFORM: 1, DIVERGENT: 2}
    return a if order[a] >= order[b] else b


class KernelBuilder:
    def __init__(self, name: str, caps: TargetCaps):
        self.name = name
        self.caps = caps
        self._names: set = set()
        self._params: list = []
        self._buffers: list = []
        self._tables: list = []
        self._tg: list = []
        self._threads: Optional[int] = None
        self._groups = None
        self._blocks: list = [[]]
        self._regions: list = [UNIFORM]
        self.problems: list = []
        self._claim(name)

    # -- names (Build.hs:216-229)
    def _claim(self, n: str) -> None:
        if n in self._names:
            self.problems.append(Finding("names", f"The name {n} is declared twice."))
        self._names.add(n)

    def fresh(self, base: str) -> str:
        n, i = base, 0
        while n in self._names:
            i += 1
            n = f"{base}_{i}"
        self._names.add(n)
        return n

    def _emit(self, s) -> None:
        self._blocks[-1].append(s)

    @property
    def region(self) -> str:
        return self._regions[-1]

    # -- the interface (Build.hs:637-744)
    def dim(self, name: str, r: I.DimRange) -> E:
        self._claim(name)
        self._params.append(I.Param(name, U32, r))
        return E(I.EParam(name), U32)

    def param(self, name: str, t: str) -> E:
        self._claim(name)
        self._params.append(I.Param(name, t, None))
        return E(I.EParam(name), t)

    def buffer(self, name: str, access: str, t: str, extent, align: int = 16) -> Buf:
        if align < max(16, SCALAR_SIZE[t]) or align & (align - 1):
            raise BuildError(f"buffer {name}: alignment {align} is not a power of two of at least 16 and {t}'s size")
        self._claim(name)
        self._buffers.append(I.Buffer(name, access, t, align, _u32(extent).ir, False))
        return Buf(name, access, t, align)

    def apart(self, b: Buf) -> None:
        self._buffers = [I.Buffer(x.name, x.access, x.type, x.align, x.extent, True) if x.name == b.name else x
                         for x in self._buffers]

    def table(self, name: str, t: str, entries, extent, align: int = 16, access: str = I.READ) -> Tab:
        if align < max(16, SCALAR_SIZE[t]) or align & (align - 1):
            raise BuildError(f"table {name}: alignment {align} is not a power of two of at least 16 and {t}'s size")
        self._claim(name)
        self._tables.append(I.Table(name, access, t, align, _u32(entries).ir, _u32(extent).ir))
        return Tab(name, access, t, align)

    def _retable(self, tb: Tab, **kw) -> None:
        out = []
        for x in self._tables:
            if x.name == tb.name:
                d = dict(name=x.name, access=x.access, type=x.type, align=x.align, entries=x.entries,
                         extent=x.extent, distinct=x.distinct, apart=x.apart)
                d.update(kw)
                x = I.Table(**d)
            out.append(x)
        self._tables = out

    def distinct(self, tb: Tab) -> None:
        self._retable(tb, distinct=True)

    def apart_via(self, tb: Tab) -> None:
        self._retable(tb, apart=True)

    def threads(self, n: int) -> None:
        if self._threads is not None:
            self.problems.append(Finding("threads", "The thread count is declared twice."))
        if not (0 < n <= self.caps.max_threads and n % self.caps.simd_width == 0):
            raise BuildError(f"{n} threads on {self.caps.name}: at most {self.caps.max_threads}, "
                             f"a multiple of {self.caps.simd_width}")
        self._threads = n

    def groups(self, e) -> None:
        if self._groups is not None:
            self.problems.append(Finding("threads", "The grid size is declared twice."))
        self._groups = _u32(e).ir

    # -- threadgroup memory (Build.hs:746-760)
    def tg_array(self, name: str, t: str, count: int) -> Tg:
        if count <= 0:
            raise BuildError(f"threadgroup array {name} of no elements")
        self._claim(name)
        self._tg.append(I.TgArray(name, t, count))
        if I.tg_layout(self._tg)[1] > self.caps.tg_mem_bytes:
            raise BuildError(f"threadgroup memory over {self.caps.tg_mem_bytes} bytes")
        return Tg(name, t, count)

    # -- locals (Build.hs:828-862)
    def let(self, name: str, e: E) -> E:
        n = self.fresh(name)
        self._emit(I.SLet(n, e.type, e.ir))
        return E(I.EVar(n), e.type)

    def var(self, name: str, e: E) -> Var:
        n = self.fresh(name)
        self._emit(I.SVar(n, e.type, e.ir))
        return Var(n, e.type)

    def assign(self, v: Var, e) -> None:
        e = v.get._other(e)
        self._emit(I.SAssign(v.name, e.ir))

    # -- memory
    def load(self, b: Buf, i) -> E:
        if b.access == I.WRITE:
            raise BuildError(f"a load of the write-only {b.name}")
        return E(I.ELoad(b.name, _u32(i).ir), b.type)

    def store(self, b: Buf, i, v) -> None:
        if b.access == I.READ:
            raise BuildError(f"a store to the read-only {b.name}")
        self._emit(I.SStore(b.name, _u32(i).ir, _typed(b.type, v).ir))

    def load_via(self, t: Tab, e, i) -> E:
        if t.access == I.WRITE:
            raise BuildError(f"a load through the write-only {t.name}")
        return E(I.ELoadVia(t.name, _u32(e).ir, _u32(i).ir), t.type)

    def store_via(self, t: Tab, e, i, v) -> None:
        if t.access == I.READ:
            raise BuildError(f"a store through the read-only {t.name}")
        self._emit(I.SStoreVia(t.name, _u32(e).ir, _u32(i).ir, _typed(t.type, v).ir))

    def _pack_ok(self, n: int, t: str, align: int) -> None:
        size = n * SCALAR_SIZE[t]
        if n < 2 or t == BOOL or size & (size - 1) or size > self.caps.lane_load_max or size > align:
            raise BuildError(f"a pack of {n} {t} on {self.caps.name} from memory aligned to {align}")

    def load_pack(self, base: str, n: int, b: Buf, j) -> list:
        if b.access == I.WRITE:
            raise BuildError(f"a load of the write-only {b.name}")
        self._pack_ok(n, b.type, b.align)
        names = tuple(self.fresh(f"{base}_{i}") for i in range(n))
        self._emit(I.SLoadPack(names, b.type, b.name, _u32(j).ir))
        return [E(I.EVar(x), b.type) for x in names]

    def load_pack_via(self, base: str, n: int, t: Tab, e, j) -> list:
        if t.access == I.WRITE:
            raise BuildError(f"a load through the write-only {t.name}")
        self._pack_ok(n, t.type, t.align)
        names = tuple(self.fresh(f"{base}_{i}") for i in range(n))
        self._emit(I.SLoadPackVia(names, t.type, t.name, _u32(e).ir, _u32(j).ir))
        return [E(I.EVar(x), t.type) for x in names]

    def store_pack(self, b: Buf, j, values: list, n: Optional[int] = None) -> None:
        if b.access == I.READ:
            raise BuildError(f"a store to the read-only {b.name}")
        n = len(values) if n is None else n
        self._pack_ok(n, b.type, b.align)
        if len(values) != n:
            self.problems.append(Finding("typing", f"A pack of {n} stored to {b.name} with {len(values)} values."))
        self._emit(I.SStorePack(b.name, _u32(j).ir, tuple(_typed(b.type, v).ir for v in values)))

    def tg_load(self, a: Tg, i) -> E:
        return E(I.ETgLoad(a.name, _u32(i).ir), a.type)

    def tg_store(self, a: Tg, i, v) -> None:
        self._emit(I.STgStore(a.name, _u32(i).ir, _typed(a.type, v).ir))

    def tg_store_pack(self, a: Tg, j, values: list) -> None:
        self._pack_ok(len(values), a.type, I.least_align(a.type))
        self._emit(I.STgStorePack(a.name, _u32(j).ir, tuple(_typed(a.type, v).ir for v in values)))

    # -- synchronisation and SIMD groups (Build.hs:936-1016)
    def barrier(self) -> None:
        if self.region != UNIFORM:
            raise BuildError("a barrier needs every thread of the threadgroup: only in uniform control")
        self._emit(I.SBarrier())

    def simd_barrier(self) -> None:
        self._converged("a SIMD-group barrier")
        self._emit(I.SSimdBarrier())

    def _converged(self, what: str) -> None:
        if self.region == DIVERGENT:
            raise BuildError(f"{what} needs every lane of its SIMD group: not under a per-lane branch")

    def _simd(self, op: str, name: str, e: E) -> E:
        self._converged("a SIMD-group reduction")
        if e.type not in NUM:
            raise BuildError(f"a SIMD-group reduction of {e.type}")
        n = self.fresh(name)
        self._emit(I.SSimd(n, op, e.type, e.ir))
        return E(I.EVar(n), e.type)

    def simd_sum(self, name: str, e: E) -> E:
        return self._simd("simd_sum", name, e)

    def simd_max(self, name: str, e: E) -> E:
        return self._simd("simd_max", name, e)

    def simd_min(self, name: str, e: E) -> E:
        return self._simd("simd_min", name, e)

    # -- fragments (Build.hs:1044-1140)
    def fragment(self, name: str, t: str) -> Frag:
        self._converged("a fragment")
        n = self.fresh(name)
        self._emit(I.SFragVar(n, t))
        return Frag(n, t)

    def _frag_load(self, f: Frag, mem: I.FragMem, t: str, i, st, tr: bool) -> None:
        self._converged("a fragment load")
        if f.type != t:
            raise BuildError(f"a fragment of {f.type} loaded from {t}")
        self._emit(I.SFragLoad(f.name, mem, _u32(i).ir, _u32(st).ir, tr))

    def frag_load(self, f: Frag, b: Buf, i, st) -> None:
        self._frag_load(f, I.FragMem("device", b.name), b.type, i, st, False)

    def frag_load_t(self, f: Frag, b: Buf, i, st) -> None:
        self._frag_load(f, I.FragMem("device", b.name), b.type, i, st, True)

    def frag_load_via(self, f: Frag, t: Tab, e, i, st) -> None:
        self._frag_load(f, I.FragMem("via", t.name, _u32(e).ir), t.type, i, st, False)

    def frag_load_via_t(self, f: Frag, t: Tab, e, i, st) -> None:
        self._frag_load(f, I.FragMem("via", t.name, _u32(e).ir), t.type, i, st, True)

    def frag_load_tg(self, f: Frag, a: Tg, i, st) -> None:
        self._frag_load(f, I.FragMem("threadgroup", a.name), a.type, i, st, False)

    def frag_load_tg_t(self, f: Frag, a: Tg, i, st) -> None:
        self._frag_load(f, I.FragMem("threadgroup", a.name), a.type, i, st, True)

    def frag_mma(self, d: Frag, a: Frag, b: Frag, c: Frag) -> None:
        self._converged("a fragment product")
        if d.type != F32 or c.type != F32 or a.type != b.type or a.type not in self.caps.fragments:
            raise BuildError(f"a product of {a.type} fragments into f32 on {self.caps.name}")
        self._emit(I.SFragMma(d.name, a.name, b.name, c.name))

    def frag_convert(self, d: Frag, s: Frag) -> None:
        self._converged("a fragment conversion")
        if d.type != F32:
            raise BuildError("a fragment widens into f32")
        self._emit(I.SFragConvert(d.name, s.name))

    def frag_scale_rows(self, f: Frag, a: Tg, i) -> None:
        self._converged("a fragment's rows scaled")
        if f.type != F32 or a.type != F32:
            raise BuildError("rows of an f32 fragment by an f32 array")
        self._emit(I.SFragScaleRows(f.name, a.name, _u32(i).ir))

    def _frag_store(self, mem: I.FragMem, t: str, i, st, f: Frag) -> None:
        self._converged("a fragment store")
        if f.type != t:
            raise BuildError(f"a fragment of {f.type} stored to {t}")
        self._emit(I.SFragStore(mem, _u32(i).ir, _u32(st).ir, f.name))

    def frag_store(self, b: Buf, i, st, f: Frag) -> None:
        if b.access == I.READ:
            raise BuildError(f"a store to the read-only {b.name}")
        self._frag_store(I.FragMem("device", b.name), b.type, i, st, f)

    def frag_store_via(self, t: Tab, e, i, st, f: Frag) -> None:
        if t.access == I.READ:
            raise BuildError(f"a store through the read-only {t.name}")
        self._frag_store(I.FragMem("via", t.name, _u32(e).ir), t.type, i, st, f)

    def frag_store_tg(self, a: Tg, i, st, f: Frag) -> None:
        self._frag_store(I.FragMem("threadgroup", a.name), a.type, i, st, f)

    # -- control (Build.hs:1142-1191)
    @contextlib.contextmanager
    def _block(self, region: str):
        self._blocks.append([])
        self._regions.append(region)
        try:
            yield
        finally:
            self._regions.pop()
        return

    @contextlib.contextmanager
    def _when(self, cond: E, region: str, inner: str):
        if cond.type != BOOL:
            raise BuildError("a condition is a bool")
        self._blocks.append([])
        self._regions.append(inner)
        try:
            yield
        finally:
            self._regions.pop()
            body = self._blocks.pop()
        self._emit(I.SIf(region, cond.ir, tuple(body), ()))

    def when_u(self, cond: E):
        return self._when(cond, "uniform", self.region)

    def when_simd(self, cond: E):
        return self._when(cond, "simd_uniform", _meet(self.region, SIMD_UNIFORM))

    def when_lane(self, cond: E):
        return self._when(cond, "divergent", DIVERGENT)

    @contextlib.contextmanager
    def _for(self, name: str, region: str, inner: str, start, end, step):
        v = self.fresh(name)
        self._blocks.append([])
        self._regions.append(inner)
        try:
            yield E(I.EVar(v), U32)
        finally:
            self._regions.pop()
            body = self._blocks.pop()
        self._emit(I.SFor(region, v, _u32(start).ir, _u32(end).ir, _u32(step).ir, tuple(body)))

    def for_u(self, name: str, lo, hi):
        return self._for(name, "uniform", self.region, lo, hi, 1)

    def for_step(self, name: str, start, end, step):
        return self._for(name, "divergent", DIVERGENT, start, end, step)

    def strided(self, name: str, end):
        """The threads take turns over [0, end): thread i visits i, i +
        threads, ... (Build.hs:1171-1181)."""
        return self._for(name, "divergent", DIVERGENT, thread_index, end, self._threads or 0)

    # -- what the builder knows (Build.hs:1183-1220)
    def thread_count(self) -> E:
        return u32(self._threads or 0)

    def simd_group_count(self) -> E:
        return u32((self._threads or 0) // max(1, self.caps.simd_width))

    def simd_width(self) -> E:
        return u32(self.caps.simd_width)

    def simd_groups(self) -> int:
        return (self._threads or 0) // max(1, self.caps.simd_width)

    def known_multiple(self, e: E) -> Optional[int]:
        if isinstance(e.ir, I.ELit) and e.ir.lit.type == U32:
            return e.ir.lit.bits
        if isinstance(e.ir, I.EParam):
            for p in self._params:
                if p.name == e.ir.name and p.dim is not None:
                    return p.dim.multiple_of
        return None

    def note(self, rule: str, message: str) -> None:
        self.problems.append(Finding(rule, message))

    def done(self):
        if len(self._blocks) != 1:
            raise BuildError("a block left open")
        problems = list(self.problems)
        if self._threads is None:
            problems.append(Finding("threads", "No thread count: declare one with threads."))
        if self._groups is None:
            problems.append(Finding("threads", "No grid size: declare one with groups."))
        k = I.Kernel(self.name, self._threads or 0, self.caps.simd_width,
                     self._groups if self._groups is not None else I.ELit(I.lit_u32(0)),
                     tuple(self._params), tuple(self._buffers), tuple(self._tables), tuple(self._tg),
                     tuple(self._blocks[0]))
        return k, problems


def _u32(e) -> E:
    if isinstance(e, E):
        if e.type != U32:
            raise BuildError(f"an index or size of {e.type}, not u32")
        return e
    return u32(e)


def _typed(t: str, v) -> E:
    if isinstance(v, E):
        if v.type != t:
            raise BuildError(f"a value of {v.type} where {t} is wanted")
        return v
    return lit(t, v)
