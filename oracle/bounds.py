"""The binary64 evaluator's per-element bounds (src/FuryKernel/Program/Eval.hs:
686-966, `Approx`): for each element of each value a step computes, its exact
value and how far from it a kernel's binary32 value can be, for kernels whose
arithmetic keeps to the contract (sums and dot products in any order, fused or
not; exp, tanh within a few ulp; division correctly rounded); and for each
cache element a step stores, what a kernel may have stored there.

TEST INFRASTRUCTURE: imported only by tests/, as the checker of the target's
binary32 results against the evaluator's exact ones.

`evaluate_bounds` follows Eval.hs's node cases for the operations the decode
programs use (Input, Linear, RmsNorm, Add, Concat, ScaleBy, Standardize, GatedGelu,
GeluMul, Rope, Softcap, KvStore, Attend, Gather, ArgMax) on one row a step,
given the exact values `oracle.eval.evaluate` made.  The SiLU form of GeluMul
is this target's addition: silu(a) = a / (1 + e^-a), bounded as that
quotient with e^-a within 4 ulp, times b.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from furykernel_amd.program.graph import (
    Add, ArgMax, Attend, Concat, GatedGelu, GELU_TANH, GeluMul, Gather, Input, KvStore, Linear, Ring, RmsNorm, Rope,
    SCache, ScaleBy, SILU, Softcap, Standardize)

from .eval import EvalError, Evaluation, round_cache

UNIT = 2.0 ** -24       # binary32's unit roundoff (Eval.hs:693-695)
FLUSH = 2.0 ** -126     # the most a value flushed to zero loses
OVERFLOW = 2.0 ** 128 - 2.0 ** 103   # the least magnitude binary32 rounds to infinity
INF = math.inf


@dataclass(frozen=True)
class Approx:
    exact: float
    bound: float


def f32(x: float) -> float:
    return float(np.float32(x)) if math.isfinite(x) else x


def gamma_n(n: int) -> float:
    """n u / (1 - n u), infinite where n roundings could lose everything (Eval.hs:697-707)."""
    if n <= 0:
        return 0.0
    nu = n * UNIT
    return INF if nu >= 0.5 else nu / (1 - nu)


def exact_a(x: float) -> Approx:
    return Approx(float(x), 0.0)


def const_a(c: float) -> Approx:
    """A constant rounded once to binary32 (Eval.hs:712-714)."""
    with np.errstate(over="ignore"):
        return settle(Approx(c, abs(c - float(np.float32(c)))))


def neg_a(a: Approx) -> Approx:
    return Approx(-a.exact, a.bound)


def mag(a: Approx) -> float:
    return abs(a.exact) + a.bound


def settle(a: Approx) -> Approx:
    """Unbounded if not a number or if a kernel's value can overflow; at least
    the magnitude if a kernel can flush it to zero (Eval.hs:724-738)."""
    x, e = a.exact, a.bound
    if math.isnan(x):
        return a
    if math.isnan(e) or mag(a) >= OVERFLOW:
        return Approx(x, INF)
    if abs(x) - e < FLUSH:
        return Approx(x, max(e, abs(x)))
    return a


def sum_a(ts: list) -> Approx:
    """Terms added in any order (Eval.hs:740-746)."""
    n = len(ts)
    return settle(Approx(sum(t.exact for t in ts),
                         sum(t.bound for t in ts) + gamma_n(n - 1) * sum(mag(t) for t in ts) + 2 * n * FLUSH))


def dot_a(ps: list) -> Approx:
    """Products added in any order, fused or not (Eval.hs:748-756)."""
    n = len(ps)

    def spread(a, c):
        return abs(a.exact) * c.bound + a.bound * abs(c.exact) + a.bound * c.bound
    return settle(Approx(sum(a.exact * c.exact for a, c in ps),
                         sum(spread(a, c) for a, c in ps) + gamma_n(n) * sum(mag(a) * mag(c) for a, c in ps)
                         + 4 * n * FLUSH))


def product_a(fs: list) -> Approx:
    """Factors multiplied in any order (Eval.hs:758-768)."""
    whole, spread = 1.0, 0.0
    for f in fs:
        whole, spread = whole * abs(f.exact), spread * mag(f) + whole * f.bound
    count = len(fs)
    exact = 1.0
    for f in fs:
        exact *= f.exact
    scale = 1.0
    for f in fs:
        scale *= max(1.0, mag(f))
    return settle(Approx(exact, spread + gamma_n(count - 1) * (whole + spread) + 2 * count * FLUSH * scale))


def quotient_a(a: Approx, c: Approx) -> Approx:
    """Correctly rounded; unbounded if the divisor's bound reaches zero (Eval.hs:770-777)."""
    q = a.exact / c.exact if c.exact != 0 else math.copysign(INF, a.exact) if a.exact else math.nan
    if math.isnan(c.exact) or math.isnan(c.bound) or abs(c.exact) <= c.bound:
        return Approx(q, INF)
    low = abs(c.exact) - c.bound
    return settle(Approx(q, (abs(a.exact) * c.bound + a.bound * abs(c.exact)) / (abs(c.exact) * low)
                         + UNIT * mag(a) / low + FLUSH))


def worst(xs: list) -> float:
    if any(math.isnan(x) for x in xs):
        return math.nan
    return max([0.0] + list(xs))


def monotone_a(k: float, f, a: Approx) -> Approx:
    """A function within k ulp, monotone over the bound (Eval.hs:779-790)."""
    y = f(a.exact)
    if math.isinf(a.bound):
        return Approx(y, INF)
    lo, hi = f(a.exact - a.bound), f(a.exact + a.bound)
    return settle(Approx(y, worst([abs(lo - y), abs(hi - y)]) + 2 * k * UNIT * worst([abs(lo), abs(hi)]) + FLUSH))


def _safe_exp(x: float) -> float:
    try:
        return math.exp(x)
    except OverflowError:
        return INF


def gelu_a(form: str, a: Approx) -> Approx:
    """GELU in the contract's form (Eval.hs:797-807); SiLU as a / (1 + e^-a)."""
    if form == GELU_TANH:
        inner = product_a([const_a(math.sqrt(2 / math.pi)), sum_a([a, product_a([const_a(0.044715), a, a, a])])])
        return product_a([const_a(0.5), a, sum_a([exact_a(1.0), monotone_a(5, math.tanh, inner)])])
    if form == SILU:
        return quotient_a(a, sum_a([exact_a(1.0), monotone_a(4, _safe_exp, neg_a(a))]))
    raise EvalError(f"no bounds of the GELU form {form}")


def norm_bounds(eps: float, gamma, f: float, seg: int, xs: list) -> list:
    """A segment's RMSNorm (Eval.hs:809-815)."""
    mean_square = product_a([dot_a([(x, x) for x in xs]), const_a(1.0 / seg)])
    r = monotone_a(2, lambda v: 1 / math.sqrt(v) if v > 0 else INF, sum_a([mean_square, const_a(eps)]))
    out = []
    for j, x in enumerate(xs):
        fs = [x, r, const_a(f)] + ([exact_a(float(gamma[j]))] if gamma is not None else [])
        out.append(product_a(fs).bound)
    return out


def rope_trig(theta: float, d: int, i: int, position: float):
    """Cosine and sine of pair i's angle (Eval.hs:817-832)."""
    freq = theta ** (-(2 * i) / d)
    angle = product_a([const_a(position), settle(Approx(freq, 8 * UNIT * freq + FLUSH))])

    def trig(fn):
        if math.isinf(angle.bound):
            return Approx(fn(angle.exact), INF)
        y, e = fn(angle.exact), angle.bound
        return settle(Approx(y, min(2.0, e) + 8 * UNIT * min(1.0, abs(y) + e) + FLUSH))
    return trig(math.cos), trig(math.sin)


def rotation_bounds(theta: float, rotated: int, d: int, position: float, xs: list) -> list:
    """One head's rotation, NeoX halves (Eval.hs:834-846)."""
    half = d // 2
    out = []
    for j in range(d):
        if j < half and j < rotated:
            c, s = rope_trig(theta, d, j, position)
            out.append(dot_a([(xs[j], c), (neg_a(xs[j + half]), s)]).bound)
        elif j >= half and j - half < rotated:
            c, s = rope_trig(theta, d, j - half, position)
            out.append(dot_a([(xs[j], c), (xs[j - half], s)]).bound)
        else:
            out.append(xs[j].bound)
    return out


def certainly_before(ia, jc) -> bool:
    (i, a), (j, c) = ia, jc
    lo, hi = a.exact - a.bound, c.exact + c.bound
    return lo > hi or (lo == hi and i < j)


def arg_max_decided(xs: list) -> bool:
    """Whether every binary32 value within the bounds has the same arg-max (Eval.hs:879-882)."""
    ranked = sorted(enumerate(xs), key=lambda ix: (-ix[1].exact, ix[0]))
    return all(certainly_before(ranked[0], r) for r in ranked[1:]) if ranked else True


def gather_a(ws: list, f: float) -> Approx:
    """Rows' elements summed then scaled, or scaled then summed (Eval.hs:884-889)."""
    by_dot = dot_a([(exact_a(w), const_a(f)) for w in ws])
    by_sum = product_a([sum_a([exact_a(w) for w in ws]), const_a(f)])
    return Approx(by_dot.exact, max(by_dot.bound, by_sum.bound))


def attend_bounds(scores: list, values: list) -> list:
    """Attention's output elements from each key's score and, element by
    element, the keys' values (Eval.hs:891-918)."""
    t = float(len(scores))
    top = max([-INF] + [s.exact for s in scores])
    ws = [math.exp(s.exact - top) for s in scores]
    total = sum(ws)
    ps = [w / total for w in ws]
    highest = max([0.0] + [mag(s) for s in scores])
    rhos = [s.bound + 2 * UNIT * (mag(s) + highest) + 12 * (t + 1) * UNIT + FLUSH for s in scores]
    gs = [math.expm1(r) if r < 700 else INF for r in rhos]
    gbar = sum(p * g for p, g in zip(ps, gs))
    out = []
    for vs in values:
        if math.isnan(gbar) or gbar >= 1:
            out.append(INF)
            continue
        o = sum(p * v.exact for p, v in zip(ps, vs))
        spread = (sum(p * (g + gbar) * abs(v.exact) for p, g, v in zip(ps, gs, vs))
                  + sum(p * math.exp(r) * v.bound for p, r, v in zip(ps, rhos, vs))) / (1 - gbar) \
            + 4 * t * FLUSH * max([0.0] + [mag(v) for v in vs])
        out.append(settle(Approx(o, spread + UNIT * (abs(o) + spread) + FLUSH)).bound)
    return out


def widened(e: float) -> float:
    """The bound widened for the f64 evaluation's own rounding (Eval.hs:920-922)."""
    return e * (1 + 2.0 ** -20)


def storable(elem: str, a: Approx):
    e = widened(a.bound)
    return round_cache(elem, a.exact - e), round_cache(elem, a.exact + e)


def may_store(elem: str, a: Approx, k: float) -> bool:
    """Whether a kernel can have stored k for the element (Eval.hs:935-943)."""
    if math.isinf(a.bound):
        return True
    if math.isnan(a.exact):
        return math.isnan(k)
    lo, hi = storable(elem, a)
    return lo <= k <= hi


def own_rounding(elem: str, a: Approx) -> Approx:
    """The evaluator's rounding of the element, with how far a kernel's store
    can be from it (Eval.hs:953-966)."""
    own = round_cache(elem, a.exact)
    if math.isnan(a.exact):
        return Approx(own, 0.0)
    lo, hi = storable(elem, a)
    if lo == hi:
        return Approx(own, 0.0)
    if math.isinf(a.bound) or math.isinf(lo) or math.isinf(hi):
        return Approx(own, INF)
    return Approx(own, max(hi - own, own - lo))


@dataclass
class Bounds:
    values: dict   # value name -> [rows] of f64 bound arrays
    stores: dict   # cache name -> {(slot, element): (element Approx, stored Approx)}


def evaluate_bounds(checked, b, ev: Evaluation, kept=None) -> Bounds:
    """Every value's element bounds, in program order (Eval.hs:268-560), from
    the bindings `b` and the exact values of `ev = evaluate(checked, b, kept)`.
    Given what the kernels stored (`kept`, an `oracle.eval.Kept`), each stored
    element must be one its bound allows (else EvalError, as
    evaluateStored's Left), and it is then read exactly."""
    p = checked.program
    sources = {s.id: s for s in p.sources}
    values = {v.id: v for v in p.values}
    if b.rows != 1:
        raise EvalError("bounds are evaluated here for one row a step")
    env: dict = {}       # value id -> list of Approx (one row)
    stores: dict = {}    # cache name -> {(slot, index): (element, stored)}

    def exact_of(vid):
        return [float(x) for x in ev.values[values[vid].name][0]]

    def approx(vid):
        return env[vid]

    def weight(s):
        return np.asarray(b.weights[sources[s].name], np.float64).ravel()

    def row_int(s):
        return [int(i) for i in b.row_ints[sources[s].name][0]]

    def put(vid, bounds):
        env[vid] = [Approx(x, e) for x, e in zip(exact_of(vid), bounds)]

    recorded: dict = {}   # value id -> its bounds, where downstream reads the stored value exactly

    def anchor(node) -> None:
        """A value the kernels stored (`kept.values`) must be within its
        bound of its exact value; what reads it then reads it exactly."""
        for v in node.outputs:
            name = values[v].name
            if kept is None or name not in kept.values or v not in env:
                continue
            got = [float(x) for x in np.asarray(kept.values[name][0], np.float64)]
            for i, (g, a) in enumerate(zip(got, env[v])):
                if not within(g, a.exact, a.bound):
                    raise EvalError(f"The kernels stored {g} as {name}[{i}], not within {a.bound} of {a.exact}.")
            recorded[v] = env[v]
            env[v] = [exact_a(g) for g in got]

    prev = None
    for n in p.nodes:
        if prev is not None:
            anchor(prev)
        prev = n
        op = n.op
        out = n.outputs[0] if n.outputs else None
        if isinstance(op, Input):
            src = sources[op.source]
            row = [float(x) for x in b.inputs[src.name][0]]
            put(out, [settle(Approx(x, abs(x - f32(x)))).bound for x in row])
        elif isinstance(op, Linear):
            w = weight(op.weight)
            xs = approx(op.x)
            k = len(xs)
            xe = np.array([x.exact for x in xs])
            xb = np.array([x.bound for x in xs])
            wm = np.abs(w.reshape(-1, k))
            ex = exact_of(out)
            # dotA of exact weights: spread |w| e_x, then gamma_k sum |w| (|x| + e_x)
            raw = wm @ xb + gamma_n(k) * (wm @ (np.abs(xe) + xb)) + 4 * k * FLUSH
            put(out, [settle(Approx(e, float(r))).bound for e, r in zip(ex, raw)])
        elif isinstance(op, RmsNorm):
            gamma = None if op.gamma is None else weight(op.gamma)
            xs = approx(op.x)
            seg = values[op.x].shape.segment
            bs = []
            for c in range(0, len(xs), seg):
                bs += norm_bounds(op.eps, None if gamma is None else gamma[:seg], op.factor, seg, xs[c:c + seg])
            put(out, bs)
        elif isinstance(op, Add):
            put(out, [sum_a([u, v]).bound for u, v in zip(approx(op.a), approx(op.b))])
        elif isinstance(op, Concat):
            put(out, [x.bound for x in approx(op.a)] + [x.bound for x in approx(op.b)])
        elif isinstance(op, ScaleBy):
            w0 = float(weight(op.weight)[0])
            put(out, [product_a([u, exact_a(w0)]).bound for u in approx(op.x)])
        elif isinstance(op, GatedGelu):
            xs = approx(op.x)
            seg = values[op.x].shape.segment
            bs = []
            for c in range(0, len(xs), seg):
                a, g = xs[c:c + seg // 2], xs[c + seg // 2:c + seg]
                bs += [product_a([gelu_a(op.form, u), v]).bound for u, v in zip(a, g)]
            put(out, bs)
        elif isinstance(op, GeluMul):
            put(out, [product_a([gelu_a(op.form, u), v]).bound for u, v in zip(approx(op.a), approx(op.b))])
        elif isinstance(op, Rope):
            spec = op.spec
            d = values[op.x].shape.segment
            part = d // spec.axes
            pos = row_int(op.positions)
            xs = approx(op.x)
            bs = []
            for c in range(0, len(xs), d):
                for a in range(spec.axes):
                    bs += rotation_bounds(float(spec.theta), spec.rotated, part, float(pos[a]),
                                          xs[c + a * part:c + (a + 1) * part])
            put(out, bs)
        elif isinstance(op, Standardize):
            bias, scale = weight(op.bias), weight(op.scale)
            put(out, [product_a([sum_a([product_a([const_a(op.factor), u]), neg_a(exact_a(float(bias[j])))]),
                                 exact_a(float(scale[j]))]).bound for j, u in enumerate(approx(op.x))])
        elif isinstance(op, Softcap):
            put(out, [product_a([const_a(op.cap), monotone_a(5, math.tanh, product_a([u, const_a(1 / op.cap)]))]).bound
                      for u in approx(op.x)])
        elif isinstance(op, KvStore):
            src = sources[op.at.cache]
            lay, elem = src.kind.layout, src.kind.elem
            if not isinstance(src.kind, SCache) or not isinstance(lay, Ring):
                raise EvalError(f"{src.name}: bounds of ring caches only")
            pos, seqs = row_int(op.at.positions)[0], row_int(op.at.sequences)
            s = seqs[0] if seqs else 0
            d = lay.head_dim
            xs = approx(op.x)
            held = stores.setdefault(src.name, {})
            staged = kept.rows.get(src.name) if kept is not None else None
            left = kept.caches.get(src.name) if kept is not None else None
            for h in range(lay.kv_heads):
                at = (h * lay.length + pos % lay.length) * d
                for i in range(d):
                    el = xs[h * d + i]
                    if staged is None and left is None:
                        held[(s, at + i)] = (el, own_rounding(elem, el))
                        continue
                    k = float(staged[0][h * d + i]) if staged is not None else float(left[s][at + i])
                    if not may_store(elem, el, k):
                        lo, hi = storable(elem, el)
                        raise EvalError(f"The kernels stored {k} in {src.name} at slot {s}, element {at + i}, where "
                                        f"the exact {el.exact}, within {el.bound}, rounds to between {lo} and {hi}.")
                    if staged is not None and left is not None and float(left[s][at + i]) != k and \
                            not (math.isnan(k) and math.isnan(float(left[s][at + i]))):
                        raise EvalError(f"The kernels left {left[s][at + i]} in {src.name} at slot {s}, element "
                                        f"{at + i}, not the {k} they staged for it.")
                    held[(s, at + i)] = (el, exact_a(k))
        elif isinstance(op, Attend):
            spec = op.spec
            ksrc, vsrc = sources[op.to.keys], sources[op.to.values]
            lay = ksrc.kind.layout
            pos, seqs = row_int(op.to.positions)[0], row_int(op.to.sequences)
            s = seqs[0] if seqs else 0
            d, heads = spec.head_dim, spec.heads
            group = heads // spec.kv_heads
            first = max(0, pos - spec.window + 1) if spec.window else 0
            qa = approx(op.q)
            found_k = b.caches[ksrc.name][s]
            found_v = b.caches[vsrc.name][s]

            def read(name, found, at):
                held = stores.get(name, {})
                return held[(s, at)][1] if (s, at) in held else exact_a(float(found[at]))
            bs = []
            scale = float(spec.scale)
            for h in range(heads):
                kvh = h // group
                query = qa[h * d:(h + 1) * d]
                keys, vals = [], []
                for t in range(first, pos + 1):
                    at = (kvh * lay.length + t % lay.length) * d
                    keys.append([read(ksrc.name, found_k, at + i) for i in range(d)])
                    vals.append([read(vsrc.name, found_v, at + i) for i in range(d)])
                scores = []
                for ks in keys:
                    sc = scale * sum(query[i].exact * ks[i].exact for i in range(d))
                    e1 = product_a([dot_a(list(zip(query, ks))), const_a(scale)]).bound
                    e2 = dot_a(list(zip([product_a([e, const_a(scale)]) for e in query], ks))).bound
                    scores.append(Approx(sc, max(e1, e2)))
                bs += attend_bounds(scores, [list(col) for col in zip(*vals)])
            put(out, bs)
        elif isinstance(op, Gather):
            table = weight(op.table)
            width = values[out].shape.width
            toks = row_int(op.tokens)
            put(out, [gather_a([float(table[t * width + j]) for t in toks], op.factor).bound for j in range(width)])
        elif isinstance(op, ArgMax):
            put(out, [0.0 if arg_max_decided(approx(op.x)) else INF])
        else:
            raise EvalError(f"{n.name}: no bounds of {type(op).__name__} here")
    if prev is not None:
        anchor(prev)
    return Bounds({values[v].name: [np.array([a.bound for a in recorded.get(v, row)])] for v, row in env.items()},
                  stores)


def evaluate_stored(checked, b, kept):
    """evaluateStored (Eval.hs:189-198): the evaluation given what the
    kernels stored, and its bounds; EvalError where a stored element is not
    one its bound allows."""
    from .eval import evaluate

    ev = evaluate(checked, b, kept)
    return ev, evaluate_bounds(checked, b, ev, kept)


def within(value: float, exact: float, bound: float) -> bool:
    """A kernel's value within the element's bound of the exact, or both NaN."""
    if math.isinf(bound):
        return True
    if math.isnan(exact):
        return math.isnan(value)
    return abs(value - exact) <= widened(bound)
