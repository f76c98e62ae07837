"""The evaluator's per-element bounds (oracle/bounds.py, Eval.hs:686-966),
pinned three ways.

- Soundness, by brute force: binary32 sums, dot products (fused or not),
  products and quotients of random and cancellation-heavy operands, computed
  in many orders, each within its bound of the exact value.  A dropped term
  (the gamma factor, the operands' own bounds) fails these.
- The cases the definitions fix: exact constants, NaN, overflow, flushing,
  divisors whose bound reaches zero, decided and undecided arg-maxes.
- The tiny decode: every value the CPU target stores (SIMD widths 64 and 32)
  within its element bounds of the exact values, every new cache element one
  a kernel may store, the token equal where its arg-max is decided.  With the
  gamma factor planted away in the oracle, some element falls outside.
"""

import math

import numpy as np
import pytest

from oracle import bounds as B
from oracle.bounds import Approx
from test_evaluator import run_cpu_target, run_evaluator, tiny_state
from furykernel_amd.program.plan import PlanOptions


def f32(x):
    return np.float32(x)


def orders(n, rng, count=12):
    out = [list(range(n)), list(range(n))[::-1]]
    out += [list(rng.permutation(n)) for _ in range(count)]
    return out


def f32_sum(vals, order):
    s = np.float32(0.0)
    for i in order:
        s = np.float32(s + vals[i])
    return float(s)


def f32_pairwise(vals):
    v = [np.float32(x) for x in vals]
    while len(v) > 1:
        v = [np.float32(v[i] + v[i + 1]) if i + 1 < len(v) else v[i] for i in range(0, len(v), 2)]
    return float(v[0])


def operands(rng, n, kind):
    if kind == "random":
        return (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 3, n)).astype(np.float32)
    # cancellation-heavy: large pairs that cancel, small terms between
    big = (rng.standard_normal(n // 2) * 1e4).astype(np.float32)
    small = (rng.standard_normal(n - 2 * (n // 4)) * 1e-3).astype(np.float32)
    return np.concatenate([big[: n // 4], -big[: n // 4], small]).astype(np.float32)


@pytest.mark.parametrize("kind", ["random", "cancelling"])
@pytest.mark.parametrize("n", [2, 7, 64, 257])
def test_sum_bound_holds_in_every_order(n, kind):
    rng = np.random.default_rng(n * 7 + len(kind))
    for _ in range(20):
        x = operands(rng, n, kind)
        a = B.sum_a([B.exact_a(float(v)) for v in x])
        exact = math.fsum(float(v) for v in x)
        got = [f32_sum(x, o) for o in orders(n, rng)] + [f32_pairwise(x)]
        for g in got:
            assert abs(g - exact) <= a.bound, (g, exact, a.bound)


@pytest.mark.parametrize("kind", ["random", "cancelling"])
@pytest.mark.parametrize("n", [3, 16, 64, 200])
def test_dot_bound_holds_in_every_order_fused_or_not(n, kind):
    rng = np.random.default_rng(n * 11 + len(kind))
    for _ in range(20):
        x = operands(rng, n, kind)
        w = (rng.standard_normal(n)).astype(np.float32)
        a = B.dot_a([(B.exact_a(float(u)), B.exact_a(float(v))) for u, v in zip(w, x)])
        exact = math.fsum(float(u) * float(v) for u, v in zip(w, x))
        for o in orders(n, rng, 8):
            s = np.float32(0.0)
            f = np.float32(0.0)
            for i in o:
                s = np.float32(s + np.float32(w[i] * x[i]))
                f = np.float32(float(w[i]) * float(x[i]) + float(f))   # a fused multiply-add
            assert abs(float(s) - exact) <= a.bound
            assert abs(float(f) - exact) <= a.bound


def test_dot_bound_covers_operand_bounds():
    """Operands known only within bounds: every binary32 value within them,
    multiplied and summed in binary32, stays within the dot product's bound."""
    rng = np.random.default_rng(5)
    n = 32
    for _ in range(50):
        xe = rng.standard_normal(n)
        xb = np.abs(rng.standard_normal(n)) * 1e-3
        w = rng.standard_normal(n).astype(np.float32)
        a = B.dot_a([(B.exact_a(float(u)), Approx(float(v), float(e))) for u, v, e in zip(w, xe, xb)])
        exact = sum(float(u) * float(v) for u, v in zip(w, xe))
        for _ in range(10):
            xk = (xe + xb * rng.uniform(-1, 1, n)).astype(np.float32)
            got = f32_sum([np.float32(u * v) for u, v in zip(w, xk)], rng.permutation(n))
            assert abs(got - exact) <= a.bound


def test_product_and_quotient_bounds_hold():
    rng = np.random.default_rng(9)
    for _ in range(200):
        fs = rng.standard_normal(4) * 10.0 ** rng.uniform(-2, 2, 4)
        a = B.product_a([B.exact_a(float(f32(v))) for v in fs])
        exact = math.prod(float(f32(v)) for v in fs)
        for o in orders(4, rng, 6):
            p = np.float32(1.0)
            for i in o:
                p = np.float32(p * f32(fs[i]))
            assert abs(float(p) - exact) <= a.bound
        n, d = float(f32(fs[0])), float(f32(fs[1]))
        q = B.quotient_a(B.exact_a(n), B.exact_a(d))
        assert abs(float(np.float32(f32(n) / f32(d))) - n / d) <= q.bound


def test_the_cases_the_definitions_fix():
    assert B.const_a(0.5).bound == 0 and B.const_a(3.0).bound == 0
    assert B.const_a(0.1).bound == abs(0.1 - float(np.float32(0.1)))
    assert math.isinf(B.settle(Approx(3e38, 1e38)).bound)        # a value that can overflow
    assert math.isnan(B.settle(Approx(math.nan, 0.0)).exact)
    assert B.settle(Approx(1e-39, 0.0)).bound == 1e-39             # can flush to zero
    assert math.isinf(B.quotient_a(B.exact_a(1.0), Approx(1.0, 1.0)).bound)
    assert B.gamma_n(0) == 0 and math.isinf(B.gamma_n(2 ** 23))
    assert B.arg_max_decided([Approx(1.0, 0.1), Approx(0.5, 0.1)])
    assert not B.arg_max_decided([Approx(1.0, 0.3), Approx(0.5, 0.3)])
    # a tie decided towards the lower index
    assert B.arg_max_decided([Approx(1.0, 0.0), Approx(1.0, 0.0)])
    assert B.may_store("f16", Approx(1.0, 0.0), 1.0) and not B.may_store("f16", Approx(1.0, 0.0), 1.0009765625)


def written(lowered) -> set:
    """The buffers some launch of the lowered step writes (the manifest's
    write and read_write bindings)."""
    from furykernel_amd import runtime
    out = set()
    for L in lowered.launches:
        a = runtime.abi_of(L.entry)
        for i in range(a.n_buffers):
            name = a.buffers[i].name.decode()
            if a.buffers[i].access.decode() != "read" and L.bind.get(name):
                out.add(L.bind[name])
    return out


def check_tiny(cpu, ev, bd, checked, caches):
    bad = []
    stored = written(cpu.lowered)
    for name, rows in bd.values.items():
        buf = f"value:{name}"
        if buf not in cpu.lowered.buffers or buf not in stored:
            continue
        got = cpu.read(buf).astype(np.float64)
        exact = ev.values[name][0]
        for i, (g, x, e) in enumerate(zip(got, exact, rows[0])):
            if not B.within(float(g), float(x), float(e)):
                bad.append((name, i, float(g), float(x), float(e)))
    for cname, held in bd.stores.items():
        got = cpu.read(f"cache:{cname}").astype(np.float64)
        elem = [s for s in checked.program.sources if s.name == cname][0].kind.elem
        for (slot, at), (element, _) in held.items():
            if not B.may_store(elem, element, float(got[at])):
                bad.append((cname, at, float(got[at]), element.exact, element.bound))
    return bad


@pytest.mark.parametrize("width", [64, 32])
@pytest.mark.parametrize("store_gelus", [False, True])
@pytest.mark.parametrize("position", [16, 31])
def test_tiny_decode_within_the_element_bounds(width, store_gelus, position):
    checked, w, c, x, _ = tiny_state(position=position)
    ev = run_evaluator(checked, w, c, x, position)
    bd = B.evaluate_bounds(checked, bindings(w, c, x, position), ev)
    cpu = run_cpu_target(checked, w, c, x, position, width, PlanOptions(store_gelus=store_gelus))
    assert check_tiny(cpu, ev, bd, checked, c) == []
    # A decided arg-max (bound 0) fixes the token; an undecided one (the top
    # logits within each other's bounds) allows any of them.
    if bd.values["token"][0][0] == 0:
        assert int(cpu.read("value:token")[0]) == int(ev.values["token"][0][0])
    # Worst-case bounds compound through each RMSNorm (they scale by the
    # inverse of the row's RMS): the first layer's are all finite; later ones
    # may lose everything (infinite, which any value meets).
    first = np.concatenate([r[0] for n, r in bd.values.items() if n == "x" or n.startswith("l0_")])
    assert np.all(np.isfinite(first))


def bindings(w, c, x, position):
    from oracle.eval import Bindings

    return Bindings(1, inputs={"x": [x.astype(np.float64)]}, weights={k: v.astype(np.float64) for k, v in w.items()},
                    row_ints={"position": [[position]], "slot": [[0]]},
                    caches={k: {0: v.astype(np.float64)} for k, v in c.items()})


def test_a_dropped_gamma_factor_is_caught(monkeypatch):
    """The brute-force checks have teeth: bounds without the roundings'
    gamma factor fail them (sums and dot products, random and cancelling)."""
    monkeypatch.setattr(B, "gamma_n", lambda n: 0.0)
    for check, n in ((test_sum_bound_holds_in_every_order, 64), (test_dot_bound_holds_in_every_order_fused_or_not, 64)):
        for kind in ("random", "cancelling"):
            with pytest.raises(AssertionError):
                check(n, kind)


def test_a_wrong_exact_value_falls_outside_the_bounds(monkeypatch):
    """The decode check has teeth: an evaluator whose RoPE forgets the
    partner term (planted in the oracle) leaves the CPU target's values
    outside their bounds."""
    import oracle.eval as E

    checked, w, c, x, position = tiny_state()
    cpu = run_cpu_target(checked, w, c, x, position, 64)
    good = E.rotate

    def dropped(theta, rotated, d, pos, xs):
        ys = good(theta, rotated, d, pos, xs)
        half = d // 2
        for i in range(rotated):
            ang = pos * theta ** (-(2.0 * i) / d)
            ys[i] = xs[i] * math.cos(ang)
            ys[i + half] = xs[i + half] * math.cos(ang)
        return ys
    monkeypatch.setattr(E, "rotate", dropped)
    ev = run_evaluator(checked, w, c, x, position)
    bd = B.evaluate_bounds(checked, bindings(w, c, x, position), ev)
    assert check_tiny(cpu, ev, bd, checked, c) != []


def kept_of(cpu, checked):
    from oracle.eval import Kept

    names = [src.name for src in checked.program.sources if type(src.kind).__name__ == "SCache"]
    return Kept(caches={n: {0: cpu.read(f"cache:{n}").astype(np.float64)} for n in names})


def kept_values_of(cpu, checked):
    """What the launches stored of every value some launch writes, with the
    caches they left (oracle.eval.Kept)."""
    kept = kept_of(cpu, checked)
    stored = written(cpu.lowered)
    kept.values = {v.name: [cpu.read(f"value:{v.name}").astype(np.float64)]
                   for v in checked.program.values if f"value:{v.name}" in stored}
    return kept


def check_anchored(cpu, checked, w, c, x, position):
    """Every stored value within its bound of the exact value of its own
    launch's stored inputs (EvalError otherwise), every bound finite: each
    layer is pinned, not only the first.  The bounds, relative to the
    largest exact element of each value."""
    from oracle.eval import evaluate
    kept = kept_values_of(cpu, checked)
    b = bindings(w, c, x, position)
    ev = evaluate(checked, b, kept)
    bd = B.evaluate_bounds(checked, b, ev, kept)
    rel = {}
    for name in kept.values:
        bound = bd.values[name][0]
        assert np.all(np.isfinite(bound)), name
        rel[name] = float(np.max(bound) / max(np.max(np.abs(ev.values[name][0])), 1e-300))
    return ev, bd, rel


@pytest.mark.parametrize("width", [64, 32])
@pytest.mark.parametrize("store_gelus", [False, True])
def test_tiny_decode_within_bounds_anchored_at_every_stored_value(width, store_gelus):
    """This target's extension of evaluateStored from caches to stored values
    (oracle.eval.Kept.values): each launch's outputs checked from what the
    launches before it stored, so the worst-case bounds no longer compound
    through the layers' norms; both layers' values are held to about 1e-5
    of their largest elements."""
    checked, w, c, x, position = tiny_state(position=31)
    cpu = run_cpu_target(checked, w, c, x, position, width, PlanOptions(store_gelus=store_gelus))
    ev, bd, rel = check_anchored(cpu, checked, w, c, x, position)
    assert any(n.startswith("l1_") for n in rel) and "logits" in rel
    assert max(v for n, v in rel.items() if n != "token") < 1e-4
    assert int(cpu.read("value:token")[0]) == int(ev.values["token"][0][0]) or bd.values["token"][0][0] != 0


def test_an_anchored_value_moved_past_its_bound_is_refused():
    """The anchored check has teeth at the last layer: one element of the
    second layer's residual (planted in what the oracle is given as stored)
    moved by ten times its bound."""
    from oracle.eval import EvalError, evaluate
    checked, w, c, x, position = tiny_state(position=31)
    cpu = run_cpu_target(checked, w, c, x, position, 64)
    _, bd, _ = check_anchored(cpu, checked, w, c, x, position)
    kept = kept_values_of(cpu, checked)
    row = kept.values["l1_x1"][0].copy()
    row[7] += 10 * max(float(bd.values["l1_x1"][0][7]), 1e-30)
    kept.values["l1_x1"] = [row]
    b = bindings(w, c, x, position)
    with pytest.raises(EvalError, match="l1_x1"):
        B.evaluate_bounds(checked, b, evaluate(checked, b, kept), kept)


def test_evaluate_stored_reads_what_the_kernels_stored():
    """evaluateStored (Eval.hs:189-198): given the caches the CPU target left,
    the evaluation keeps its stores, checks each against its bound, and the
    step's values stay within their bounds of the new exact values."""
    checked, w, c, x, position = tiny_state()
    cpu = run_cpu_target(checked, w, c, x, position, 64)
    kept = kept_of(cpu, checked)
    ev, bd = B.evaluate_stored(checked, bindings(w, c, x, position), kept)
    assert check_tiny(cpu, ev, bd, checked, c) == []
    for name, units in kept.caches.items():
        assert np.array_equal(ev.caches[name][0], units[0])


def test_evaluate_stored_refuses_a_store_its_bound_does_not_allow():
    from oracle.eval import EvalError

    checked, w, c, x, position = tiny_state()
    cpu = run_cpu_target(checked, w, c, x, position, 64)
    kept = kept_of(cpu, checked)
    name = "l0_k_cache"
    lay = [s for s in checked.program.sources if s.name == name][0].kind.layout
    at = (position % lay.length) * lay.head_dim          # kv head 0, element 0 of the new row
    kept.caches[name][0][at] += 0.25
    with pytest.raises(EvalError, match="The kernels stored"):
        B.evaluate_stored(checked, bindings(w, c, x, position), kept)
