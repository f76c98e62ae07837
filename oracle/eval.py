"""The program evaluator in binary64: what a checked program's step computes,
each operation exact to double precision, rounded only where the program
rounds (its cache stores), following src/FuryKernel/Program/Eval.hs
operation for operation.  The values; the per-element bounds (`Approx`,
Eval.hs:686-966) are oracle/bounds.py's.

TEST INFRASTRUCTURE: imported only by tests/, as the f64 checker of the
target's f32 arithmetic (and of the oracle's CPU target).

Bindings (Eval.hs:126-140): ``inputs`` name -> rows of values; ``weights``
name -> flat values; ``row_ints`` name -> rows of integers; ``caches`` name ->
{slot: flat values of the slot}.  Rows are evaluated together, ``rows`` of
them.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from furykernel_amd.program.check import CheckedProgram
from furykernel_amd.program.graph import (
    CACHE_BF16, Add, ArgMax, Attend, CombineRanks, Concat, Gather, GatedGelu, GELU_TANH, GeluMul, Input, KvStore,
    Linear, LinearRouted, Ring, RmsNorm, Rope, Route, SCache, ScaleBy, SILU, Softcap, Standardize, STable)

from . import fkref


class EvalError(ValueError):
    """What the evaluator refuses, as Eval.hs's Left."""


@dataclass
class Bindings:
    rows: int = 1
    inputs: dict = field(default_factory=dict)
    weights: dict = field(default_factory=dict)
    row_ints: dict = field(default_factory=dict)
    caches: dict = field(default_factory=dict)
    tables: dict = field(default_factory=dict)  # name -> [entry's flat values, ...]


@dataclass
class Kept:
    """What a step's kernels stored (Eval.hs:174-184): ``caches`` name ->
    {slot: flat values as the step left them}; ``rows`` name -> [rows] of the
    values the kernels staged for the cache's store, if they staged them.

    ``values`` name -> [rows] of a value the kernels stored: this target's
    extension of evaluateStored from caches to stored values, so that each
    launch is checked from what the launches before it stored.  The value is
    evaluated (and recorded) from its inputs as usual, and what reads it
    downstream reads the stored rows instead."""
    caches: dict = field(default_factory=dict)
    rows: dict = field(default_factory=dict)
    values: dict = field(default_factory=dict)


@dataclass
class Evaluation:
    values: dict    # value name -> [rows] of f64 arrays
    outputs: dict   # output name -> [rows] of f64 arrays
    caches: dict    # cache name -> {slot: f64 array}


def hsum(xs) -> float:
    """Haskell's ``sum`` of a list of Doubles: a left fold from 0, each
    addition rounded (the evaluator's sums, e.g. ``dot`` at Eval.hs:973-974)."""
    s = 0.0
    for v in xs:
        s = s + float(v)
    return s


def round_bf16(x: float) -> float:
    """roundBF16 (Eval.hs:669-684): to eight significant bits, ties to even,
    binary32's exponent range with gradual underflow, overflow to infinity —
    directly from the double."""
    if math.isnan(x) or math.isinf(x) or x == 0:
        return x
    _, e = math.frexp(x)          # x = m 2^e, 1/2 <= |m| < 1: the leading bit is 2^(e-1)
    ulp = math.ldexp(1.0, max(-126, e - 1) - 7)
    r = round(x / ulp) * ulp      # x / ulp is exact; round() is to nearest, ties to even
    return math.copysign(math.inf, x) if abs(r) >= 2.0 ** 128 else r


def round_f16(x: float) -> float:
    """roundTo CacheF16 (Eval.hs:937-939): binary64 to binary16 in one rounding."""
    return float(fkref.widen_f16(fkref.narrow_f16_f64(x)))


def round_cache(elem: str, x: float) -> float:
    return round_bf16(x) if elem == CACHE_BF16 else round_f16(x)


def gelu(form: str, x: float) -> float:
    """GELU-tanh (Eval.hs:658-663), and the SiLU form this repository adds:
    x / (1 + e^-x)."""
    if form == GELU_TANH:
        return 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x * x * x)))
    if form == SILU:
        return x / (1 + math.exp(-x))
    raise EvalError(f"no GELU form {form}")


def rotate(theta: float, rotated: int, d: int, position: float, xs: np.ndarray) -> np.ndarray:
    """The exact rotation of one head of width d, NeoX halves (Eval.hs:634-645)."""
    half = d // 2
    out = np.empty(d)
    for j in range(d):
        i = j if j < half else j - half
        t = position * math.pow(theta, -(2 * i) / d) if i < rotated else 0.0
        if j < half:
            out[j] = xs[j] * math.cos(t) - xs[j + half] * math.sin(t)
        else:
            out[j] = xs[j] * math.cos(t) + xs[i] * math.sin(t)
    return out


def arg_max(xs) -> int:
    """Eval.hs:681-685: a later element wins only if strictly larger."""
    best = 0
    for j in range(1, len(xs)):
        if xs[j] > xs[best]:
            best = j
    return best


def evaluate(checked: CheckedProgram, b: Bindings, kept: Kept | None = None) -> Evaluation:
    """Eval.hs:186-228: every node in program order.  Given `kept`, each store
    into a cache keeps the element the kernels stored (staged, if they staged
    it, else as they left the cache), so that what attends over the caches
    reads what the kernels read; `oracle.bounds.evaluate_bounds` with the same
    `kept` checks that each element's bound allows it (evaluateStored,
    Eval.hs:189-198)."""
    p = checked.program
    m = b.rows
    sources = {s.id: s for s in p.sources}
    values = {v.id: v for v in p.values}
    env: dict = {}
    caches = {name: {u: np.array(xs, np.float64) for u, xs in units.items()} for name, units in b.caches.items()}
    stored: set = set()
    # Each cache a step stores into: its units before the step, and each
    # element's stores in row order, (row, position, value) (Eval.hs:415-473).
    before: dict = {}
    row_stores: dict = {}

    def weight(s: int) -> np.ndarray:
        src = sources[s]
        if src.name not in b.weights:
            raise EvalError(f"No weight {src.name}.")
        a = np.asarray(b.weights[src.name], np.float64).ravel()
        want = int(np.prod(src.kind.dims))
        if a.size != want:
            raise EvalError(f"{src.name} is bound to {a.size} elements, not the {want} it declares.")
        return a

    def ints(s: int) -> list:
        src = sources[s]
        if src.name not in b.row_ints:
            raise EvalError(f"No row integers {src.name}.")
        rows = b.row_ints[src.name]
        if len(rows) != m:
            raise EvalError(f"{src.name} has {len(rows)} rows, not {m}.")
        for r, row in enumerate(rows):
            for i in row:
                if i >= src.kind.bound:
                    raise EvalError(f"{src.name}: row {r} holds {i}, which isn't below its bound of {src.kind.bound}.")
        return [[int(i) for i in row] for row in rows]

    def cache_index(layout, seqs: list, position: int, h: int) -> tuple[int, int]:
        """Eval.hs:592-602: where head h of a position starts, its slot (a
        ring's) or its block (a paged pool's, through the block table)."""
        if isinstance(layout, Ring):
            s = seqs[0] if seqs else 0
            return s, (h * layout.length + position % layout.length) * layout.head_dim
        bs = layout.block_size
        if position // bs >= len(seqs):
            raise EvalError(f"Position {position} is past the block table.")
        return seqs[position // bs], (h * bs + position % bs) * layout.head_dim

    def unit_name(layout) -> str:
        return "slot" if isinstance(layout, Ring) else "block"

    recorded: dict = {}   # value id -> its evaluated rows, where downstream reads the stored ones

    def anchor(node) -> None:
        for v in node.outputs:
            name = values[v].name
            if kept is not None and name in kept.values and v in env:
                rows = [np.asarray(r, np.float64) for r in kept.values[name]]
                if len(rows) != len(env[v]) or any(r.shape != e.shape for r, e in zip(rows, env[v])):
                    raise EvalError(f"The kernels' {name} is not the shape of the value.")
                recorded[v] = env[v]
                env[v] = rows

    prev = None
    for n in p.nodes:
        if prev is not None:
            anchor(prev)
        prev = n
        op = n.op
        out = n.outputs[0] if n.outputs else None
        if isinstance(op, Input):
            src = sources[op.source]
            rows = b.inputs.get(src.name)
            if rows is None:
                raise EvalError(f"No input {src.name}.")
            env[out] = [np.asarray(r, np.float64) for r in rows]
        elif isinstance(op, Linear):
            w = weight(op.weight)
            k = values[op.x].shape.width
            n_out = values[out].shape.width
            wm = w.reshape(n_out, k)
            env[out] = [np.array([hsum(wm[j] * x) for j in range(n_out)]) for x in env[op.x]]
        elif isinstance(op, RmsNorm):
            gamma = None if op.gamma is None else weight(op.gamma)
            seg = values[op.x].shape.segment
            res = []
            for x in env[op.x]:
                parts = []
                for c in range(0, len(x), seg):
                    v = x[c:c + seg]
                    ms = hsum(v * v) / seg
                    s = (ms + op.eps) ** -0.5
                    g = gamma if gamma is not None else np.ones(seg)
                    parts.append(v * s * g[:seg] * op.factor)
                res.append(np.concatenate(parts))
            env[out] = res
        elif isinstance(op, Add):
            env[out] = [x + y for x, y in zip(env[op.a], env[op.b])]
        elif isinstance(op, Concat):
            env[out] = [np.concatenate([x, y]) for x, y in zip(env[op.a], env[op.b])]
        elif isinstance(op, ScaleBy):
            w = weight(op.weight)
            env[out] = [x * w[0] for x in env[op.x]]
        elif isinstance(op, GatedGelu):
            seg = values[op.x].shape.segment
            res = []
            for x in env[op.x]:
                parts = []
                for c in range(0, len(x), seg):
                    a, g = x[c:c + seg // 2], x[c + seg // 2:c + seg]
                    parts.append(np.array([gelu(op.form, u) * v for u, v in zip(a, g)]))
                res.append(np.concatenate(parts))
            env[out] = res
        elif isinstance(op, GeluMul):
            env[out] = [np.array([gelu(op.form, u) * v for u, v in zip(x, y)]) for x, y in zip(env[op.a], env[op.b])]
        elif isinstance(op, Rope):
            # Eval.hs:372-383: a head of d is `axes` parts of d / axes, part a
            # turned by the row's a-th position as a head of its own width.
            spec = op.spec
            d = values[op.x].shape.segment
            part = d // spec.axes
            ps = ints(op.positions)
            res = []
            for pos, x in zip(ps, env[op.x]):
                res.append(np.concatenate([rotate(spec.theta, spec.rotated, part, float(pos[a]), x[c + a * part:c + (a + 1) * part])
                                           for c in range(0, len(x), d) for a in range(spec.axes)]))
            env[out] = res
        elif isinstance(op, Standardize):
            # Eval.hs:536-543: (f x_j - bias_j) scale_j.
            bias, scale = weight(op.bias), weight(op.scale)
            env[out] = [np.array([(op.factor * v - bias[j]) * scale[j] for j, v in enumerate(x)]) for x in env[op.x]]
        elif isinstance(op, Softcap):
            env[out] = [np.array([op.cap * math.tanh(v / op.cap) for v in x]) for x in env[op.x]]
        elif isinstance(op, KvStore):
            src = sources[op.at.cache]
            if not isinstance(src.kind, SCache):
                raise EvalError(f"{src.name} is not a cache.")
            if src.name in stored:
                raise EvalError(f"{n.name} stores into {src.name} again: a program stores into a cache once.")
            stored.add(src.name)
            before[src.name] = {u: a.copy() for u, a in caches.get(src.name, {}).items()}
            row_stores[src.name] = elem_stores = {}
            lay, elem = src.kind.layout, src.kind.elem
            units = caches.get(src.name)
            if units is None:
                raise EvalError(f"No cache {src.name}.")
            ps, seqs = ints(op.at.positions), ints(op.at.sequences)
            d, heads = lay.head_dim, lay.kv_heads
            staged = kept.rows.get(src.name) if kept is not None else None
            left = kept.caches.get(src.name) if kept is not None else None
            for r, (pos, sq, x) in enumerate(zip(ps, seqs, env[op.x])):
                for h in range(heads):
                    u, at = cache_index(lay, sq, pos[0], h)
                    if u not in units:
                        raise EvalError(f"A store to {src.name} at {unit_name(lay)} {u}, element {at}, which "
                                        "isn't bound.")
                    for i in range(d):
                        if staged is not None:
                            v = float(staged[r][h * d + i])
                        elif left is not None:
                            v = float(left[u][at + i])
                        else:
                            v = round_cache(elem, float(x[h * d + i]))
                        units[u][at + i] = v
                        elem_stores.setdefault((u, at + i), []).append((r, pos[0], v))
        elif isinstance(op, Attend):
            spec = op.spec
            ksrc, vsrc = sources[op.to.keys], sources[op.to.values]
            lay = ksrc.kind.layout
            ps, seqs = ints(op.to.positions), ints(op.to.sequences)
            reaches = ps if spec.reach is None else ints(spec.reach.source)
            if spec.reach is not None:
                for i, (pos, rc) in enumerate(zip(ps, reaches)):
                    if rc[0] > pos[0] + spec.reach.ahead:
                        raise EvalError(f"{n.name}: row {i} reaches {rc[0]}, more than {spec.reach.ahead} past its "
                                        f"position, {pos[0]}.")
            d, heads = spec.head_dim, spec.heads
            group = heads // spec.kv_heads

            def read(name, u, at, r0, r, t):
                """Eval.hs:563-576: row r0 reads position t as the row r that
                stored its reach does: a store of t by a row after r0 up to
                r, else the last store of rows up to r0 into the element (of
                position t, or the read is refused), else the cache before
                the step."""
                units = before.get(name, caches.get(name, {}))
                if u not in units or at + d > len(units[u]):
                    raise EvalError(f"{name}: {unit_name(lay)} {u}, element {at}, isn't bound.")
                elems = row_stores.get(name)
                if elems is None:
                    return units[u][at:at + d]
                out = np.empty(d)
                for i in range(d):
                    st = elems.get((u, at + i), [])
                    ahead = [v for j, t2, v in reversed(st) if r0 < j <= r and t2 == t]
                    mine = [(t2, v) for j, t2, v in st if j <= r0]
                    if ahead:
                        out[i] = ahead[0]
                    elif mine:
                        if mine[-1][0] != t:
                            raise EvalError(f"{name}: row {r0} reads position {t} where a row stored {mine[-1][0]}.")
                        out[i] = mine[-1][1]
                    else:
                        out[i] = units[u][at + i]
                return out

            res = []
            for r0, (pos, rc, sq, q) in enumerate(zip(ps, reaches, seqs, env[op.q])):
                position = pos[0]
                # the row that stored this row's reach, if one of the step's did
                r = next((j for j in range(r0, len(ps)) if ps[j][0] == rc[0] and seqs[j] == sq), r0)
                first = max(0, position - spec.window + 1) if spec.window else 0
                ts = range(first, max(position, rc[0]) + 1)
                row = []
                for h in range(heads):
                    kvh = h // group
                    query = q[h * d:(h + 1) * d]
                    keys, vals = [], []
                    for t in ts:
                        u, at = cache_index(lay, sq, t, kvh)
                        keys.append(read(ksrc.name, u, at, r0, r, t))
                        vals.append(read(vsrc.name, u, at, r0, r, t))
                    scores = [spec.scale * hsum(query * kk) for kk in keys]
                    top = max(scores)
                    es = [math.exp(s - top) for s in scores]
                    total = hsum(es)
                    row.append(np.array([hsum(e / total * vv[i] for e, vv in zip(es, vals)) for i in range(d)]))
                res.append(np.concatenate(row))
            env[out] = res
        elif isinstance(op, Gather):
            table = weight(op.table)
            width = values[out].shape.width
            tm = table.reshape(-1, width)
            env[out] = [sum(tm[t] for t in toks) * op.factor for toks in ints(op.tokens)]
        elif isinstance(op, ArgMax):
            env[out] = [np.array([float(arg_max(list(x)))]) for x in env[op.x]]
        elif isinstance(op, Route):
            # Eval.hs:391-404, routeRow :648-655: the k largest logits, ties
            # to the lower index, in rank order; weights a softmax over them
            # (exp(x - best) / their sum, the sum a left fold from 0), each
            # times its expert's scale if there is one.
            scale = None if op.spec.expert_scale is None else weight(op.spec.expert_scale)
            ids_rows, w_rows = [], []
            for x in env[op.x]:
                order = sorted(range(len(x)), key=lambda i: (-x[i], i))
                top = order[:op.spec.k]
                best = x[order[0]]
                es = [math.exp(x[i] - best) for i in top]
                total = 0.0
                for e in es:
                    total = total + e
                ids_rows.append(np.array(top, np.float64))
                w_rows.append(np.array([e / total * (1.0 if scale is None else scale[i]) for i, e in zip(top, es)]))
            env[n.outputs[0]], env[n.outputs[1]] = ids_rows, w_rows
        elif isinstance(op, LinearRouted):
            # Eval.hs:291-321: rank r's segment is its expert's weights times
            # the row (shared by every rank when the row is one expert's
            # input wide, else the rank's slice of it).
            src = sources[op.table]
            if not isinstance(src.kind, STable):
                raise EvalError(f"{src.name} is not a table.")
            entries = b.tables.get(src.name)
            if entries is None:
                raise EvalError(f"No table {src.name}.")
            if len(entries) != src.kind.entries:
                raise EvalError(f"{src.name} has {len(entries)} entries bound, not {src.kind.entries}.")
            out_w, k = src.kind.dims
            mats = [np.asarray(e, np.float64).reshape(out_w, k) for e in entries]
            shared = values[op.x].shape.width == k
            res = []
            for idr, xr in zip(env[op.ids], env[op.x]):
                parts = []
                for rank, e in enumerate(idr):
                    entry = int(round(e))
                    if not 0 <= entry < len(mats):
                        raise EvalError(f"{n.name}: expert {entry} is not in the table.")
                    base = 0 if shared else rank * k
                    xs = xr[base:base + k]
                    parts.append(np.array([hsum(mats[entry][j] * xs) for j in range(out_w)]))
                res.append(np.concatenate(parts))
            env[out] = res
        elif isinstance(op, CombineRanks):
            # Eval.hs:405-414: sum over ranks of weight times the rank's
            # segment, a left fold from the first rank's product.
            seg = values[op.x].shape.segment
            res = []
            for wr, xr in zip(env[op.weights], env[op.x]):
                acc = wr[0] * xr[0:seg]
                for r in range(1, len(wr)):
                    acc = acc + wr[r] * xr[r * seg:(r + 1) * seg]
                res.append(acc)
            env[out] = res
        else:
            raise EvalError(f"{n.name}: {type(op).__name__} is not evaluated here")
    if prev is not None:
        anchor(prev)
    outs = {}
    for o in p.outputs:
        if o.value not in env:
            raise EvalError(f"The output {o.name} was never made.")
        outs[o.name] = recorded.get(o.value, env[o.value])
    return Evaluation({values[v].name: recorded.get(v, rows) for v, rows in env.items()}, outs, caches)


def evaluate_fast(checked: CheckedProgram, b: Bindings) -> Evaluation:
    """The same evaluation with numpy's binary64 sums over all rows at once:
    equal to ``evaluate`` but for the order of each sum's additions (the last
    bits of binary64), so within 1e-12 of it — the evaluator for programs too
    big for the left folds (tests pin the two together).  Supports the
    operations the decoder programs use."""
    p = checked.program
    m = b.rows
    sources = {s.id: s for s in p.sources}
    values = {v.id: v for v in p.values}
    env: dict = {}
    caches = {name: {u: np.array(xs, np.float64) for u, xs in units.items()} for name, units in b.caches.items()}

    def weight(s: int) -> np.ndarray:
        src = sources[s]
        if src.name not in b.weights:
            raise EvalError(f"No weight {src.name}.")
        a = np.asarray(b.weights[src.name], np.float64).ravel()
        if a.size != int(np.prod(src.kind.dims)):
            raise EvalError(f"{src.name} is bound to {a.size} elements.")
        return a

    def ints(s: int) -> np.ndarray:
        src = sources[s]
        rows = np.asarray(b.row_ints[src.name], np.int64).reshape(m, -1)
        if np.any(rows >= src.kind.bound):
            raise EvalError(f"{src.name}: a row holds an integer not below its bound of {src.kind.bound}.")
        return rows

    for n in p.nodes:
        op = n.op
        out = n.outputs[0] if n.outputs else None
        if isinstance(op, Input):
            env[out] = np.asarray(b.inputs[sources[op.source].name], np.float64).reshape(m, -1)
        elif isinstance(op, Linear):
            k = values[op.x].shape.width
            w = weight(op.weight).reshape(-1, k)
            env[out] = env[op.x] @ w.T
        elif isinstance(op, RmsNorm):
            seg = values[op.x].shape.segment
            x = env[op.x].reshape(m, -1, seg)
            s = (np.sum(x * x, axis=-1, keepdims=True) / seg + op.eps) ** -0.5
            g = weight(op.gamma)[:seg] if op.gamma is not None else np.ones(seg)
            env[out] = (x * s * g * op.factor).reshape(m, -1)
        elif isinstance(op, Add):
            env[out] = env[op.a] + env[op.b]
        elif isinstance(op, GeluMul):
            a = env[op.a]
            if op.form == SILU:
                ga = a / (1 + np.exp(-a))
            else:
                ga = 0.5 * a * (1 + np.tanh(math.sqrt(2 / math.pi) * (a + 0.044715 * a * a * a)))
            env[out] = ga * env[op.b]
        elif isinstance(op, GatedGelu):
            seg = values[op.x].shape.segment
            x = env[op.x].reshape(m, -1, seg)
            a, c = x[..., :seg // 2], x[..., seg // 2:]
            if op.form == SILU:
                ga = a / (1 + np.exp(-a))
            else:
                ga = 0.5 * a * (1 + np.tanh(math.sqrt(2 / math.pi) * (a + 0.044715 * a * a * a)))
            env[out] = (ga * c).reshape(m, -1)
        elif isinstance(op, Softcap):
            env[out] = op.cap * np.tanh(env[op.x] / op.cap)
        elif isinstance(op, Rope):
            spec = op.spec
            d = values[op.x].shape.segment // spec.axes        # the width each axis turns
            half = d // 2
            pos = ints(op.positions).astype(np.float64)          # [m, axes]
            i = np.arange(half)
            freq = np.array([math.pow(spec.theta, -(2 * j) / d) if j < spec.rotated else 0.0 for j in i])
            t = pos[:, None, :, None] * freq[None, None, None, :]   # [m, 1, axes, half]
            c, s_ = np.cos(t), np.sin(t)
            x = env[op.x].reshape(m, -1, spec.axes, d)
            lo, hi = x[..., :half], x[..., half:]
            env[out] = np.concatenate([lo * c - hi * s_, hi * c + lo * s_], axis=-1).reshape(m, -1)
        elif isinstance(op, Standardize):
            env[out] = (op.factor * env[op.x] - weight(op.bias)[None, :]) * weight(op.scale)[None, :]
        elif isinstance(op, Concat):
            env[out] = np.concatenate([env[op.a], env[op.b]], axis=1)
        elif isinstance(op, ScaleBy):
            env[out] = env[op.x] * weight(op.weight)[0]
        elif isinstance(op, KvStore):
            src = sources[op.at.cache]
            lay, elem = src.kind.layout, src.kind.elem
            if not isinstance(lay, Ring):
                raise EvalError("the fast evaluation takes ring caches; evaluate paged ones with evaluate")
            pos, seq = ints(op.at.positions)[:, 0], ints(op.at.sequences)[:, 0]
            d, heads = lay.head_dim, lay.kv_heads
            x = env[op.x].reshape(m, heads, d)
            rounded = x.astype(np.float16).astype(np.float64) if elem != CACHE_BF16 else \
                np.vectorize(round_bf16)(x)
            for r in range(m):
                unit = caches[src.name][int(seq[r])].reshape(heads, lay.length, d)
                unit[:, int(pos[r]) % lay.length, :] = rounded[r]
        elif isinstance(op, Attend):
            spec = op.spec
            lay = sources[op.to.keys].kind.layout
            if not isinstance(lay, Ring) or spec.reach is not None:
                raise EvalError("the fast evaluation takes ring caches and no reach; evaluate others with evaluate")
            pos, seq = ints(op.to.positions)[:, 0], ints(op.to.sequences)[:, 0]
            d, heads, kvh = spec.head_dim, spec.heads, spec.kv_heads
            group = heads // kvh
            q = env[op.q].reshape(m, heads, d)
            res = np.empty((m, heads, d))
            # The rows of one sequence together: row r's scores over positions
            # t in [first_r, pos_r] (the others masked to weight zero), the
            # key of position t at ring index t mod length.
            for u in np.unique(seq):
                rows = np.nonzero(seq == u)[0]
                ps = pos[rows]
                ts = np.arange(int(ps.max()) + 1)
                keys = caches[sources[op.to.keys].name][int(u)].reshape(kvh, lay.length, d)[:, ts % lay.length, :]
                vals = caches[sources[op.to.values].name][int(u)].reshape(kvh, lay.length, d)[:, ts % lay.length, :]
                first = np.maximum(0, ps - spec.window + 1) if spec.window else np.zeros_like(ps)
                seen = (ts[None, :] <= ps[:, None]) & (ts[None, :] >= first[:, None])
                for h in range(heads):
                    scores = np.where(seen, spec.scale * (q[rows, h, :] @ keys[h // group].T), -np.inf)
                    e = np.exp(scores - scores.max(axis=1, keepdims=True))
                    res[rows, h] = (e / e.sum(axis=1, keepdims=True)) @ vals[h // group]
            env[out] = res.reshape(m, -1)
        elif isinstance(op, Gather):
            width = values[out].shape.width
            tm = weight(op.table).reshape(-1, width)
            toks = ints(op.tokens)
            env[out] = tm[toks].sum(axis=1) * op.factor
        elif isinstance(op, ArgMax):
            env[out] = np.argmax(env[op.x], axis=1).astype(np.float64)[:, None]
        else:
            raise EvalError(f"{n.name}: {type(op).__name__} is not evaluated here")
    outs = {o.name: env[o.value] for o in p.outputs}
    return Evaluation({values[v].name: rows for v, rows in env.items()}, outs, caches)
