"""The oracle's SIMT interpreter for the kernel IR: a restatement of
src/FuryKernel/Interp.hs, the reference that kernels and targets are checked
against.

TEST INFRASTRUCTURE: only tests/ load this, as the checker of the IR target
(furykernel_amd/ir/rocm.py's HIP on the GPU).  Nothing in the product path
imports it.

The model (Interp.hs:1-52): threadgroups run one after another; within one,
every thread runs each statement together, as lanes of numpy vectors with an
active set, a branch splitting it, a loop keeping the lanes whose condition
holds, the lanes reconverging after.  SIMD-group reductions combine each
group's lanes pairwise, neighbours first.  Arithmetic is the IR's: binary32
with IEEE rounding (numpy's, subnormals kept), binary16 rounded after every
operation, the conversions and transcendentals of the oracle's C library
(oracle/fkref.c: Numerics.hs's, and the platform libm's binary64 rsqrt, exp,
log and tanh rounded once), integers wrapping.

Errors instead of undefined behaviour, with the reference's names: accesses
past what the kernel declares, dimensions outside their range, reads of
threadgroup memory never written, integer division by zero and the quotient
that overflows, loops that never end, barriers and SIMD-group operations
reached by part of a group, launch sizes that leave u32, unbound table
entries.  Not restated: the race detector (Interp.hs:680-735) and the
seed-drawn order of threadgroups and stores, which change nothing for a
kernel free of races; here threadgroups run in order and a statement's
stores land in lane order.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from furykernel_amd.ir import ir as I
from furykernel_amd.program.graph import BF16, BOOL, F16, F32, I8, I32, U8, U32

from . import fkref

NP = {F32: np.float32, F16: np.uint16, BF16: np.uint16, I32: np.int32, U32: np.uint32, I8: np.int8, U8: np.uint8,
      BOOL: np.bool_}
MAX_ITERATIONS = 2 ** 24
QNAN32 = np.uint32(0x7FC00000).view(np.float32)


class RunError(Exception):
    """What stops a run (Interp.hs:160-205): ``kind`` is the constructor's
    name, ``args`` its fields."""

    def __init__(self, kind: str, *args):
        super().__init__(f"{kind} {args}")
        self.kind = kind
        self.args_ = args


# ---------------------------------------------------------------------------
# Numerics, element-wise, through the oracle's C library

def _c(fn, x, out_dtype, *extra):
    x = np.ascontiguousarray(x)
    y = np.empty(x.shape, out_dtype)
    if x.size:
        getattr(fkref.lib(), fn)(*extra, x.ctypes.data, y.ctypes.data, x.size)
    return y


def widen_f16(h):
    return _c("fkref_widen_f16_n", np.asarray(h, np.uint16), np.float32)


def widen_bf16(b):
    return _c("fkref_widen_bf16_n", np.asarray(b, np.uint16), np.float32)


def narrow_f16(x):
    return _c("fkref_narrow_f16_n", np.asarray(x, np.float32), np.uint16)


def narrow_bf16(x):
    return _c("fkref_narrow_bf16_n", np.asarray(x, np.float32), np.uint16)


def narrow_f16_f64(x):
    return _c("fkref_narrow_f16_f64_n", np.asarray(x, np.float64), np.uint16)


def unary_f64(op: int, x):
    return _c("fkref_unary_f64_n", np.asarray(x, np.float64), np.float64, op)


def fma_f32(a, b, c):
    a, b, c = (np.ascontiguousarray(v, np.float32) for v in (a, b, c))
    y = np.empty(a.shape, np.float32)
    if a.size:
        fkref.lib().fkref_fma_f32_n(a.ctypes.data, b.ctypes.data, c.ctypes.data, y.ctypes.data, a.size)
    return y


def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def min_number(x, y):
    """IEEE 754-2019 minimumNumber, -0 below +0, two NaNs the quiet NaN (Interp.hs:944-956)."""
    x, y = np.asarray(x, np.float32), np.asarray(y, np.float32)
    eq = (_bits(x) | _bits(y)).view(np.float32)
    r = np.where(x < y, x, np.where(y < x, y, eq))
    nx, ny = np.isnan(x), np.isnan(y)
    r = np.where(nx & ~ny, y, np.where(ny & ~nx, x, r))
    return np.where(nx & ny, QNAN32, r).astype(np.float32)


def max_number(x, y):
    x, y = np.asarray(x, np.float32), np.asarray(y, np.float32)
    eq = (_bits(x) & _bits(y)).view(np.float32)
    r = np.where(x > y, x, np.where(y > x, y, eq))
    nx, ny = np.isnan(x), np.isnan(y)
    r = np.where(nx & ~ny, y, np.where(ny & ~nx, x, r))
    return np.where(nx & ny, QNAN32, r).astype(np.float32)


def _float_op(op, x, y):
    with np.errstate(all="ignore"):
        if op == "add":
            return (x + y).astype(np.float32)
        if op == "sub":
            return (x - y).astype(np.float32)
        if op == "mul":
            return (x * y).astype(np.float32)
        if op == "div":
            return (x / y).astype(np.float32)
    if op == "min":
        return min_number(x, y)
    if op == "max":
        return max_number(x, y)
    raise RunError("Internal", f"float {op}")


def _compare(op, x, y):
    return {"eq": x == y, "ne": x != y, "lt": x < y, "le": x <= y, "gt": x > y, "ge": x >= y}[op]


def _int_op(op, t, x, y):
    if op in ("add", "sub", "mul"):
        a = x.view(np.uint32).astype(np.uint64)
        b = y.view(np.uint32).astype(np.uint64)
        with np.errstate(all="ignore"):
            r = {"add": a + b, "sub": a - b, "mul": a * b}[op]
        r = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        return r.view(np.int32) if t == I32 else r
    if op in ("div", "rem"):
        a, b = x.astype(np.int64), y.astype(np.int64)
        if np.any(b == 0):
            raise RunError("DivideByZero")
        if t == I32 and np.any((a == -2**31) & (b == -1)):
            raise RunError("IntegerOverflow")
        q = np.abs(a) // np.abs(b) * np.sign(a) * np.sign(b)
        r = q if op == "div" else a - q * b
        return r.astype(np.int32 if t == I32 else np.uint32)
    if op == "min":
        return np.minimum(x, y)
    if op == "max":
        return np.maximum(x, y)
    raise RunError("Internal", f"integer {op}")


def arith(op: str, t: str, x, y):
    """A binary operator of two values of type t (Interp.hs:893-942); the type of the result."""
    if op in I.COMPARISONS:
        if t == F16:
            return BOOL, _compare(op, widen_f16(x), widen_f16(y))
        return BOOL, _compare(op, x, y)
    if t == F32:
        return F32, _float_op(op, x, y)
    if t == F16:
        return F16, narrow_f16(_float_op(op, widen_f16(x), widen_f16(y)))
    if t in (I32, U32):
        return t, _int_op(op, t, x, y)
    if t == BOOL:
        if op == "and":
            return BOOL, x & y
        if op == "or":
            return BOOL, x | y
    raise RunError("Internal", f"binary {op} of {t}")


# The C library's codes of its binary64 functions (oracle/fkref.h).
_UN64 = {"rsqrt": 0, "exp": 1, "log": 2, "tanh": 3}


def unary(op: str, t: str, x):
    """Interp.hs:828-860."""
    if op == "not":
        return ~x
    if op == "neg":
        if t == F32:
            return (_bits(x) ^ np.uint32(0x80000000)).view(np.float32)
        if t == F16:
            return (x ^ np.uint16(0x8000)).astype(np.uint16)
        if t == I32:
            return ((-(x.astype(np.int64))) % (1 << 32)).astype(np.uint32).view(np.int32)
        return ((-(x.astype(np.int64))) % (1 << 32)).astype(np.uint32)
    if op == "abs":
        if t == F32:
            return (_bits(x) & np.uint32(0x7FFFFFFF)).view(np.float32)
        if t == F16:
            return (x & np.uint16(0x7FFF)).astype(np.uint16)
        if t == I32:
            return np.abs(x.astype(np.int64)).astype(np.uint32).view(np.int32)
        return x
    if op == "sqrt":
        with np.errstate(all="ignore"):
            if t == F32:
                return np.sqrt(x).astype(np.float32)
            return narrow_f16(np.sqrt(widen_f16(x)))
    code = _UN64[op]
    with np.errstate(all="ignore"):
        if t == F32:
            return unary_f64(code, x.astype(np.float64)).astype(np.float32)
        return narrow_f16_f64(unary_f64(code, widen_f16(x).astype(np.float64)))


def fma(t: str, a, b, c):
    """Interp.hs:862-891: binary32 by fmaf, binary16 exactly (through binary64,
    whose product of two binary16 is exact), a NaN the quiet NaN."""
    if t == F32:
        return fma_f32(a, b, c)
    with np.errstate(all="ignore"):
        s = widen_f16(a).astype(np.float64) * widen_f16(b).astype(np.float64) + widen_f16(c).astype(np.float64)
    r = narrow_f16_f64(s)
    return np.where(np.isnan(s), np.uint16(0x7E00), r).astype(np.uint16)


def convert(src: str, dst: str, x):
    """Interp.hs:958-969."""
    if src == dst:
        return x
    if (src, dst) == (BF16, F32):
        return widen_bf16(x)
    if (src, dst) == (F16, F32):
        return widen_f16(x)
    if (src, dst) in ((I8, I32), (U8, U32)):
        return x.astype(NP[dst])
    if (src, dst) == (F32, BF16):
        return narrow_bf16(x)
    if (src, dst) == (F32, F16):
        return narrow_f16(x)
    if src in (U32, I32) and dst == F32:
        return x.astype(np.float32)
    raise RunError("Internal", f"conversion of {src} to {dst}")


def narrow_int(o: str, t: str, x):
    if t == I8:
        return (np.clip(x, -128, 127) if o == "clamp" else x).astype(np.int8)
    return (np.minimum(x, np.uint32(255)) if o == "clamp" else x).astype(np.uint8)


def literal_value(l: I.Lit):
    if l.type == F32:
        return np.uint32(l.bits).view(np.float32)
    return NP[l.type](l.bits)


# ---------------------------------------------------------------------------
# Launch sizes (Interp.hs:441-467)

def host_u32(params: dict, e) -> int:
    if isinstance(e, I.ELit) and e.lit.type == U32:
        return e.lit.bits
    if isinstance(e, I.EParam):
        if e.name not in params:
            raise RunError("MissingParam", e.name)
        return int(params[e.name])
    if isinstance(e, I.EBin):
        x, y = host_u32(params, e.a), host_u32(params, e.b)
        if e.op in ("div", "rem") and y == 0:
            raise RunError("DivideByZero")
        v = {"add": lambda: x + y, "sub": lambda: x - y, "mul": lambda: x * y, "div": lambda: x // y,
             "rem": lambda: x % y}.get(e.op)
        if v is None:
            raise RunError("Internal", "launch size operator")
        v = v()
        if not 0 <= v <= 0xFFFFFFFF:
            raise RunError("LaunchSizeOutOfRange", I.render_expr(e), v)
        return v
    raise RunError("Internal", "launch size expression")


# ---------------------------------------------------------------------------
# Running a kernel

@dataclass
class _Group:
    index: int
    locals: dict
    tg: dict
    written: dict
    frags: dict


class _Run:
    def __init__(self, k: I.Kernel, width: int, params: dict, buffers: dict, tables: dict):
        self.k = k
        self.w = width
        self.params = params
        self.buffers = buffers
        self.tables = tables  # name -> (count, {entry: array})
        self.types = {}
        for p in k.params:
            self.types[("param", p.name)] = p.type
        self.buf_t = {b.name: b.type for b in k.buffers}
        self.tab_t = {t.name: t.type for t in k.tables}
        self.tg_t = {a.name: a.type for a in k.tg_arrays}
        self.all = np.arange(k.threads)
        self.simds = (k.threads + width - 1) // width

    # -- expressions: (type, values over the lanes)
    def ev(self, g: _Group, e, lanes):
        n = len(lanes)
        if isinstance(e, I.ELit):
            return e.lit.type, np.full(n, literal_value(e.lit), NP[e.lit.type])
        if isinstance(e, I.EVar):
            t, arr = g.locals[e.name]
            return t, arr[lanes]
        if isinstance(e, I.EParam):
            p = next(p for p in self.k.params if p.name == e.name)
            return p.type, np.full(n, self.params[e.name], NP[p.type])
        if isinstance(e, I.EBuiltin):
            v = {"thread": lanes, "group": np.full(n, g.index), "lane": lanes % self.w,
                 "simd_group": lanes // self.w}[e.which]
            return U32, v.astype(np.uint32)
        if isinstance(e, I.EUn):
            t, x = self.ev(g, e.a, lanes)
            return t, unary(e.op, t, x)
        if isinstance(e, I.EBin):
            t, x = self.ev(g, e.a, lanes)
            _, y = self.ev(g, e.b, lanes)
            return arith(e.op, t, x, y)
        if isinstance(e, I.ESelect):
            _, c = self.ev(g, e.c, lanes)
            t, a = self.ev(g, e.a, lanes)
            _, b = self.ev(g, e.b, lanes)
            return t, np.where(c, a, b).astype(NP[t])
        if isinstance(e, I.EFma):
            t, a = self.ev(g, e.a, lanes)
            _, b = self.ev(g, e.b, lanes)
            _, c = self.ev(g, e.c, lanes)
            return t, fma(t, a, b, c)
        if isinstance(e, I.EConvert):
            t, x = self.ev(g, e.a, lanes)
            return e.type, convert(t, e.type, x)
        if isinstance(e, I.ENarrowInt):
            _, x = self.ev(g, e.a, lanes)
            return e.type, narrow_int(e.overflow, e.type, x)
        if isinstance(e, I.ELoad):
            _, ix = self.ev(g, e.index, lanes)
            arr = self.buffers[e.buffer]
            self._bounds(e.buffer, ix, len(arr))
            return self.buf_t[e.buffer], arr[ix.astype(np.int64)]
        if isinstance(e, I.ELoadVia):
            _, ent = self.ev(g, e.entry, lanes)
            _, ix = self.ev(g, e.index, lanes)
            t = self.tab_t[e.table]
            out = np.empty(n, NP[t])
            for en in np.unique(ent):
                sel = ent == en
                arr = self._entry(e.table, int(en))
                self._bounds(e.table, ix[sel], len(arr))
                out[sel] = arr[ix[sel].astype(np.int64)]
            return t, out
        if isinstance(e, I.ETgLoad):
            _, ix = self.ev(g, e.index, lanes)
            arr = g.tg[e.array]
            self._bounds(e.array, ix, len(arr))
            ix = ix.astype(np.int64)
            bad = ~g.written[e.array][ix]
            if bad.any():
                raise RunError("UninitializedRead", e.array, int(ix[bad][0]))
            return self.tg_t[e.array], arr[ix]
        raise RunError("Internal", f"expression {e!r}")

    def _bounds(self, name, ix, extent):
        ix = np.asarray(ix)
        bad = ix.astype(np.int64) >= extent
        if bad.any():
            raise RunError("OutOfBounds", name, int(ix[bad][0]), extent)

    def _entry(self, table, entry):
        count, arrays = self.tables[table]
        if entry >= count:
            raise RunError("OutOfBounds", table, entry, count)
        if entry not in arrays:
            raise RunError("UnboundEntry", table, entry)
        return arrays[entry]

    # -- locals
    def bind(self, g: _Group, name: str, t: str, lanes, values):
        if name not in g.locals:
            g.locals[name] = (t, np.zeros(self.k.threads, NP[t]))
        g.locals[name][1][lanes] = values

    # -- statements (Interp.hs:471-662)
    def block(self, g: _Group, lanes, stmts):
        for s in stmts:
            if len(lanes) == 0:
                return
            self.stmt(g, lanes, s)

    def stmt(self, g: _Group, lanes, s):
        ev = self.ev
        if isinstance(s, (I.SLet, I.SVar)):
            _, v = ev(g, s.e, lanes)
            self.bind(g, s.name, s.type, lanes, v)
        elif isinstance(s, I.SAssign):
            _, v = ev(g, s.e, lanes)
            g.locals[s.name][1][lanes] = v
        elif isinstance(s, I.SStore):
            _, ix = ev(g, s.index, lanes)
            _, v = ev(g, s.value, lanes)
            arr = self.buffers[s.buffer]
            self._bounds(s.buffer, ix, len(arr))
            arr[ix.astype(np.int64)] = v
        elif isinstance(s, I.SStoreVia):
            _, ent = ev(g, s.entry, lanes)
            _, ix = ev(g, s.index, lanes)
            _, v = ev(g, s.value, lanes)
            for en in np.unique(ent):
                sel = ent == en
                arr = self._entry(s.table, int(en))
                self._bounds(s.table, ix[sel], len(arr))
                arr[ix[sel].astype(np.int64)] = v[sel]
        elif isinstance(s, I.STgStore):
            _, ix = ev(g, s.index, lanes)
            _, v = ev(g, s.value, lanes)
            arr = g.tg[s.array]
            self._bounds(s.array, ix, len(arr))
            arr[ix.astype(np.int64)] = v
            g.written[s.array][ix.astype(np.int64)] = True
        elif isinstance(s, (I.SLoadPack, I.SLoadPackVia)):
            width = len(s.names)
            _, j = ev(g, s.index, lanes)
            base = j.astype(np.int64) * width
            if isinstance(s, I.SLoadPack):
                arr = self.buffers[s.buffer]
                self._bounds(s.buffer, base + width - 1, len(arr))
                for i, name in enumerate(s.names):
                    self.bind(g, name, s.type, lanes, arr[base + i])
            else:
                _, ent = ev(g, s.entry, lanes)
                vals = [np.empty(len(lanes), NP[s.type]) for _ in s.names]
                for en in np.unique(ent):
                    sel = ent == en
                    arr = self._entry(s.table, int(en))
                    self._bounds(s.table, base[sel] + width - 1, len(arr))
                    for i in range(width):
                        vals[i][sel] = arr[base[sel] + i]
                for name, v in zip(s.names, vals):
                    self.bind(g, name, s.type, lanes, v)
        elif isinstance(s, (I.SStorePack, I.STgStorePack)):
            width = len(s.values)
            _, j = ev(g, s.index, lanes)
            vs = [ev(g, v, lanes)[1] for v in s.values]
            base = j.astype(np.int64) * width
            if isinstance(s, I.SStorePack):
                arr, name = self.buffers[s.buffer], s.buffer
            else:
                arr, name = g.tg[s.array], s.array
            self._bounds(name, base + width - 1, len(arr))
            for i, v in enumerate(vs):
                arr[base + i] = v
                if isinstance(s, I.STgStorePack):
                    g.written[s.array][base + i] = True
        elif isinstance(s, I.SIf):
            _, c = ev(g, s.cond, lanes)
            self.block(g, lanes[c], s.then)
            self.block(g, lanes[~c], s.orelse)
        elif isinstance(s, I.SFor):
            _, start = ev(g, s.start, lanes)
            self.bind(g, s.var, U32, lanes, start)
            live = lanes
            it = 0
            while True:
                if it > MAX_ITERATIONS:
                    raise RunError("NonTermination", s.var)
                cur = g.locals[s.var][1][live]
                _, end = ev(g, s.end, live)
                live = live[cur < end]
                if len(live) == 0:
                    break
                self.block(g, live, s.body)
                cur = g.locals[s.var][1][live].astype(np.int64)
                _, d = ev(g, s.step, live)
                nxt = cur + d.astype(np.int64)
                if np.any(d == 0) or np.any(nxt > 0xFFFFFFFF):
                    raise RunError("NonTermination", s.var)
                g.locals[s.var][1][live] = nxt.astype(np.uint32)
                it += 1
        elif isinstance(s, I.SBarrier):
            if len(lanes) != self.k.threads:
                raise RunError("DivergentBarrier")
        elif isinstance(s, I.SSimdBarrier):
            self._groups_of(lanes, "simdgroup barrier")
        elif isinstance(s, I.SSimd):
            groups = self._groups_of(lanes, s.name)
            t = s.type
            _, v = ev(g, s.e, lanes)
            out = np.empty(len(lanes), NP[t])
            op = {"simd_sum": "add", "simd_max": "max", "simd_min": "min"}[s.op]
            pos = {int(l): i for i, l in enumerate(lanes)}
            for gi in groups:
                idx = [pos[l] for l in range(gi * self.w, min(self.k.threads, (gi + 1) * self.w))]
                vals = v[idx]
                while len(vals) > 1:
                    pairs = len(vals) // 2
                    _, r = arith(op, t, vals[0:2 * pairs:2], vals[1:2 * pairs:2])
                    vals = np.concatenate([r, vals[2 * pairs:]]).astype(NP[t])
                out[idx] = vals[0]
            self.bind(g, s.name, t, lanes, out)
        else:
            self.fragment_stmt(g, lanes, s)

    def _groups_of(self, lanes, what):
        """The SIMD groups with an active lane, each wholly active (Interp.hs:596-607)."""
        active = set(int(l) for l in lanes)
        out = []
        for gi in range(self.simds):
            group = set(range(gi * self.w, min(self.k.threads, (gi + 1) * self.w)))
            present = group & active
            if present and present != group:
                raise RunError("DivergentSimd", what)
            if present:
                out.append(gi)
        return out

    # -- fragments: 64 elements a SIMD group, (r, c) at r * 8 + c (Interp.hs:608-662)
    def _frag(self, g: _Group, name, t=None):
        if name not in g.frags:
            g.frags[name] = (t or F32, np.zeros((self.simds, 64), NP[t or F32]))
        return g.frags[name]

    def _frag_mem(self, g, mem: I.FragMem, first):
        if mem.kind == "device":
            return self.buffers[mem.name], self.buf_t[mem.name], None
        if mem.kind == "threadgroup":
            return g.tg[mem.name], self.tg_t[mem.name], g.written[mem.name]
        _, ent = self.ev(g, mem.entry, np.array([first]))
        return self._entry(mem.name, int(ent[0])), self.tab_t[mem.name], None

    def _as_float(self, t, v):
        if t == BF16:
            return widen_bf16(v)
        if t == F16:
            return widen_f16(v)
        return v.astype(np.float32)

    def fragment_stmt(self, g: _Group, lanes, s):
        name = {I.SFragVar: "name", I.SFragLoad: "name", I.SFragStore: "name", I.SFragMma: "d",
                I.SFragConvert: "d", I.SFragScaleRows: "frag"}.get(type(s))
        if name is None:
            raise RunError("Internal", f"statement {s!r}")
        groups = self._groups_of(lanes, getattr(s, name))
        rr, cc = np.divmod(np.arange(64), 8)
        for gi in groups:
            first = gi * self.w
            if isinstance(s, I.SFragVar):
                g.frags[s.name] = g.frags.get(s.name) or (s.type, np.zeros((self.simds, 64), NP[s.type]))
                g.frags[s.name][1][gi] = 0
            elif isinstance(s, (I.SFragLoad, I.SFragStore)):
                _, base = self.ev(g, s.index, np.array([first]))
                _, stride = self.ev(g, s.stride, np.array([first]))
                base, stride = int(base[0]), int(stride[0])
                arr, t, written = self._frag_mem(g, s.mem, first)
                if isinstance(s, I.SFragLoad):
                    at = base + (cc * stride + rr if s.transposed else rr * stride + cc)
                    self._bounds(s.mem.name, at, len(arr))
                    if written is not None and not written[at].all():
                        raise RunError("UninitializedRead", s.mem.name, int(at[~written[at]][0]))
                    ft, fa = self._frag(g, s.name, t)
                    fa[gi] = arr[at]
                else:
                    at = base + rr * stride + cc
                    self._bounds(s.mem.name, at, len(arr))
                    _, fa = self._frag(g, s.name)
                    arr[at] = fa[gi]
                    if written is not None:
                        written[at] = True
            elif isinstance(s, I.SFragScaleRows):
                _, base = self.ev(g, s.index, np.array([first]))
                at = int(base[0]) + np.arange(8)
                arr = g.tg[s.array]
                self._bounds(s.array, at, len(arr))
                if not g.written[s.array][at].all():
                    raise RunError("UninitializedRead", s.array, int(at[~g.written[s.array][at]][0]))
                ft, fa = self._frag(g, s.frag)
                with np.errstate(all="ignore"):
                    fa[gi] = (self._as_float(ft, fa[gi]).reshape(8, 8) * arr[at].astype(np.float32)[:, None]).ravel()
            elif isinstance(s, I.SFragConvert):
                st, sa = self._frag(g, s.s)
                _, da = self._frag(g, s.d, F32)
                da[gi] = self._as_float(st, sa[gi])
            elif isinstance(s, I.SFragMma):
                at, aa = self._frag(g, s.a)
                bt, ba = self._frag(g, s.b)
                ct, ca = self._frag(g, s.c)
                A = self._as_float(at, aa[gi]).reshape(8, 8)
                B = self._as_float(bt, ba[gi]).reshape(8, 8)
                acc = self._as_float(ct, ca[gi]).reshape(8, 8).copy()
                with np.errstate(all="ignore"):
                    for kk in range(8):  # foldl (+) start products, each product rounded
                        acc = (acc + (A[:, kk][:, None] * B[kk, :][None, :]).astype(np.float32)).astype(np.float32)
                _, da = self._frag(g, s.d, F32)
                da[gi] = acc.ravel()


def run(k: I.Kernel, width: int, params: dict, buffers: dict, tables: dict | None = None):
    """Runs kernel k, built for SIMD width ``width``, on these parameters
    (name -> value), buffers (name -> numpy array of the buffer's element
    type: f16 and bf16 as their uint16 bits) and tables (name -> list of
    arrays, None or empty for an unbound entry).  Returns every buffer and
    every table's entries as they are afterwards (Interp.hs:224-371)."""
    tables = tables or {}
    for p in k.params:
        if p.name not in params:
            raise RunError("MissingParam", p.name)
        if p.dim is not None:
            v = int(params[p.name])
            r = p.dim
            if v < r.min or v > r.max or (r.multiple_of > 0 and v % r.multiple_of):
                raise RunError("DimOutOfRange", p.name, v, r)
    out = {}
    views = {}
    for b in k.buffers:
        if b.name not in buffers:
            raise RunError("MissingBuffer", b.name)
        arr = np.array(buffers[b.name], dtype=NP[b.type], copy=True)
        extent = host_u32(params, b.extent)
        if len(arr) < extent:
            raise RunError("ShortBuffer", b.name, extent, len(arr))
        out[b.name] = arr
        views[b.name] = arr[:extent]
    tabs, tab_out = {}, {}
    for t in k.tables:
        if t.name not in tables:
            raise RunError("MissingBuffer", t.name)
        count = host_u32(params, t.entries)
        extent = host_u32(params, t.extent)
        entries = [None if e is None else np.array(e, dtype=NP[t.type], copy=True) for e in tables[t.name]]
        arrays = {}
        for e, a in enumerate(entries[:count]):
            if a is None or len(a) == 0:
                continue
            if len(a) < extent:
                raise RunError("ShortBuffer", t.name, extent, len(a))
            arrays[e] = a[:extent]
        tabs[t.name] = (count, arrays)
        tab_out[t.name] = entries
    groups = host_u32(params, k.groups)
    r = _Run(k, width, params, views, tabs)
    for gi in range(groups):
        tg = {a.name: np.zeros(a.count, NP[a.type]) for a in k.tg_arrays}
        written = {a.name: np.zeros(a.count, bool) for a in k.tg_arrays}
        g = _Group(gi, {}, tg, written, {})
        r.block(g, r.all, k.body)
    return out, tab_out
