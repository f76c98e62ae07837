"""The evaluator's store bounds and gathers, pinned by the reference's own
known answers (test/Test/FuryKernel/ProgramTest.hs):

- ``evalStored`` (:1108-1142): a kernel's store of the bf16 midpoint 1 + 2^-8
  is kept either way it rounds, and what attends to it reads it exactly; a
  store two steps off, or below the midpoint's rounding, is refused;
- ``boundsF16`` (:1191-1200): an f16 cache keeps f16's 0.1, not bf16's, and
  a bf16 cache the other way round;
- ``boundsRefuse`` (:1202-1216): for a well-conditioned 1 and 1 + 3·2^-9,
  bf16's uneven steps beside 1 and the truncation are refused;
- ``boundsAccept`` (:1218-1243): binary32's cancellation to 0 and the exact
  2^-30, both sides of a subnormal tie, the overflow tie's largest finite
  value and infinity, and NaN;
- ``boundsLongRope`` (:1256-1294): a head turned at position 2^18 - 1 with
  angles made as binary32 products, or from tables by the angle-addition
  formulas, is kept, though those roundings differ from the exact ones;
- ``boundsLongDots`` (:1296-1312) and ``boundsTight`` (:1318-1332): long
  binary32 dot products summed in order or pairwise are kept; the bf16
  steps beside a well-conditioned product's rounding are refused (drawn
  here from fixed seeds, where the reference draws them with hedgehog);
- ``evalPooledGather`` (:1623-1635): a gather of two rows sums them, then
  scales; and ``embedProgram`` (:785-789), a gather scaled by 5.65625.
"""

import math

import numpy as np
import pytest

from furykernel_amd.program.build import program
from furykernel_amd.program.check import check_program
from furykernel_amd.program.graph import AttnSpec, CACHE_BF16, CACHE_F16, F32, Ring, RopeSpec, Shape, whole_row
from oracle import bounds as B
from oracle.eval import Bindings, EvalError, Kept, evaluate, evaluate_fast, round_bf16


def slots(n, xs):
    """ProgramTest.hs:1060-1061: a flat list cut into slots of n."""
    return {i: list(xs[j:j + n]) for i, j in enumerate(range(0, len(xs), n))}


def kept_ok(checked, b, kept) -> bool:
    try:
        B.evaluate_stored(checked, b, kept)
    except EvalError:
        return False
    return True


# evalStored ------------------------------------------------------------------

def stored_attention():
    def body(b):
        q = b.input("q", Shape(4, 2), F32)
        pos = b.row_ints("position", 1, 4)
        slot = b.row_ints("slot", 1, 1)
        k = b.cache("k", Ring(1, 1, 4, 2))
        v = b.cache("v", Ring(1, 1, 4, 2))
        one = b.weight("one", [1])
        kv = b.scale_by("scaled", one, b.input("kv", Shape(2, 2), F32))
        b.kv_store("store_k", k, pos, slot, kv)
        b.kv_store("store_v", v, pos, slot, kv)
        o = b.attend("o", AttnSpec(2, 1, 2, None, 1), q, k, v, pos, slot)
        b.output("o", o)

    return check_program(program("attention", body))


def test_eval_stored_keeps_either_rounding_of_a_midpoint():
    """ProgramTest.hs:1108-1142."""
    checked = stored_attention()
    midpoint, ulp = 1 + 2.0 ** -8, 2.0 ** -7
    second = round_bf16(0.2)
    b = Bindings(1, inputs={"q": [[1, 2, 3, 4]], "kv": [[midpoint, 0.2]]}, weights={"one": [1.0]},
                 row_ints={"position": [[0]], "slot": [[0]]},
                 caches={"k": slots(8, [0.0] * 8), "v": slots(8, [0.0] * 8)})

    def kept(x):
        row = [x, second] + [0.0] * 6
        return Kept(caches={"k": slots(8, row), "v": slots(8, row)})

    # the evaluator's own rounding takes the midpoint to the even 1
    assert evaluate(checked, b).caches["k"][0][0] == 1.0
    ev, _ = B.evaluate_stored(checked, b, kept(1 + ulp))
    assert ev.outputs["o"][0].tolist() == [1 + ulp, second, 1 + ulp, second]
    assert not kept_ok(checked, b, kept(1 + 2 * ulp)), "a store two steps from the midpoint's rounding was kept"
    assert not kept_ok(checked, b, kept(1 - ulp / 2)), "a store a step below the midpoint's rounding was kept"
    assert kept_ok(checked, b, kept(1.0))


# The evaluator's bounds on one stored dot product ---------------------------------

def stored_dot_in(elem, k):
    """ProgramTest.hs:1168-1178: a linear layer of one output over k
    inputs, stored into a cache of one element."""
    def body(b):
        x = b.input("x", whole_row(k), F32)
        w = b.weight("w", [1, k])
        pos = b.row_ints("position", 1, 1)
        slot = b.row_ints("slot", 1, 1)
        c = b.cache("c", Ring(1, 1, 1, 1), elem)
        y = b.linear("y", w, 0, x)
        b.kv_store("store", c, pos, slot, y)
        b.output("y", y)

    return check_program(program("stored_dot", body))


def dot_bindings(w, x):
    return Bindings(1, inputs={"x": [list(map(float, x))]}, weights={"w": list(map(float, w))},
                    row_ints={"position": [[0]], "slot": [[0]]}, caches={"c": slots(1, [0.0])})


def keeps_in(elem, w, x, k) -> bool:
    """ProgramTest.hs:1183-1189: whether the evaluator keeps a kernel's store
    of k for the dot product of w and x."""
    return kept_ok(stored_dot_in(elem, len(x)), dot_bindings(w, x), Kept(caches={"c": slots(1, [k])}))


def keeps(w, x, k) -> bool:
    return keeps_in(CACHE_BF16, w, x, k)


def test_bounds_f16():
    """ProgramTest.hs:1191-1200: 0.1 is 0.0999755859375 in f16 and
    0.10009765625 in bf16."""
    assert keeps_in(CACHE_F16, [1], [0.1], 0.0999755859375), "f16's 0.1 was refused in an f16 cache"
    assert not keeps_in(CACHE_F16, [1], [0.1], 0.10009765625), "bf16's 0.1 was kept in an f16 cache"
    assert keeps_in(CACHE_BF16, [1], [0.1], 0.10009765625), "bf16's 0.1 was refused in a bf16 cache"
    assert not keeps_in(CACHE_BF16, [1], [0.1], 0.0999755859375), "f16's 0.1 was kept in a bf16 cache"
    ev = evaluate(stored_dot_in(CACHE_F16, 1), dot_bindings([1], [0.1]))
    assert ev.caches["c"] == {0: [0.0999755859375]} or list(ev.caches["c"][0]) == [0.0999755859375]


def test_bounds_refuse():
    """ProgramTest.hs:1202-1216: 1 exactly, bf16's steps 2^-8 below it and
    2^-7 above; 1 + 3·2^-9 rounds up to 1 + 2^-7, and truncated is 1."""
    assert keeps([1], [1], 1), "1 was refused for 1"
    assert not keeps([1], [1], 1 - 2.0 ** -7), "two steps below 1 were kept for 1"
    assert not keeps([1], [1], 1 - 2.0 ** -8), "a step below 1 was kept for 1"
    assert not keeps([1], [1], 1 + 2.0 ** -7), "a step above 1 was kept for 1"
    x = 1 + 3 * 2.0 ** -9
    assert keeps([1], [x], 1 + 2.0 ** -7), "the rounding was refused"
    assert not keeps([1], [x], 1), "the truncation was kept"
    assert keeps([1], [-x], -(1 + 2.0 ** -7)), "the negative rounding was refused"
    assert not keeps([1], [-x], -1), "the negative truncation was kept"


def test_bounds_accept():
    """ProgramTest.hs:1218-1243."""
    # binary32 adds 1 + 2^-30 to 1, then -1 to 0; the exact sum is 2^-30
    xs = [1, 2.0 ** -30, -1]
    s = np.float32(0)
    for v in xs:
        s = np.float32(s + np.float32(v))
    assert s == 0
    assert keeps([1, 1, 1], xs, 0), "binary32's 0 was refused"
    assert keeps([1, 1, 1], xs, 2.0 ** -30), "the exact 2^-30 was refused"
    # 2^-134 is halfway between 0 and bf16's least subnormal, 2^-133
    assert keeps([2.0 ** -67], [2.0 ** -67], 0), "0 was refused at the tie"
    assert keeps([2.0 ** -67], [2.0 ** -67], 2.0 ** -133), "2^-133 was refused at the tie"
    # 3 · 2^-134 is halfway between the subnormals 2^-133 and 2^-132
    assert keeps([3 * 2.0 ** -67], [2.0 ** -67], 2.0 ** -133), "2^-133 was refused"
    assert keeps([3 * 2.0 ** -67], [2.0 ** -67], 2.0 ** -132), "2^-132 was refused"
    # (2 - 2^-8) · 2^127 is halfway between bf16's largest finite value and
    # 2^128, which overflows to infinity
    w, x = [2.0 ** 63], [(2 - 2.0 ** -8) * 2.0 ** 64]
    assert keeps(w, x, (2 - 2.0 ** -7) * 2.0 ** 127), "the largest finite value was refused"
    assert keeps(w, x, math.inf), "infinity was refused"
    assert not keeps(w, x, (2 - 2.0 ** -6) * 2.0 ** 127), "a step below the largest finite value was kept"
    # NaN stores as NaN
    assert keeps([1], [math.nan], math.nan), "NaN was refused for NaN"
    assert not keeps([1], [math.nan], 0), "0 was kept for NaN"


def test_a_planted_bound_mistake_fails_the_known_answers():
    """The known answers have teeth: a may_store that forgets the
    evaluator's widening and takes the exact value's neighbours in the cache
    type (one step either side) keeps what boundsRefuse refuses."""
    good = B.storable

    def loose(elem, a):
        lo, hi = good(elem, a)
        step = 2.0 ** (math.frexp(a.exact)[1] - 8) if a.exact else 0.0
        return lo - step, hi + step

    B.storable = loose
    try:
        assert keeps([1], [1], 1 + 2.0 ** -7)
    finally:
        B.storable = good
    assert not keeps([1], [1], 1 + 2.0 ** -7)


# A rotary embedding far into the context -----------------------------------------

def stored_rope():
    """ProgramTest.hs:1246-1254: a head of 16 turned at positions below 2^18
    by θ = 10000, and stored."""
    def body(b):
        x = b.input("x", Shape(16, 16), F32)
        pos = b.row_ints("position", 1, 262144)
        slot = b.row_ints("slot", 1, 1)
        c = b.cache("c", Ring(1, 1, 1, 16))
        turned = b.rope("turned", RopeSpec(10000, 8, 1), pos, x)
        b.kv_store("store", c, pos, slot, turned)
        b.output("turned", turned)

    return check_program(program("stored_rope", body))


def test_bounds_long_rope():
    """ProgramTest.hs:1256-1294: at position 2^18 - 1, a kernel's angles as
    binary32 products of the position and the frequency, or from tables of
    256 q θ_i and r θ_i by the angle-addition formulas, turn some elements
    to other bf16 than the exact angles do; both are kept."""
    p = 262143
    xs = [np.float32(v) for v in (0.3, -0.7, 1.1, 0.25, -1.3, 0.9, 0.6, -0.2, 0.45, -0.35, 0.8, -1.05, 0.15,
                                  0.55, -0.65, 1.2)]
    f32 = np.float32

    def freq(i):
        return 10000 ** -(2 * i / 16)

    def trig32(angle):
        """A binary32 angle's cosine and sine, rounded once to binary32."""
        return f32(math.cos(float(angle))), f32(math.sin(float(angle)))

    def by_product(i):
        return trig32(f32(p) * f32(freq(i)))

    def by_tables(i):
        q, r = divmod(p, 256)

        def at(fn, n):
            return f32(fn(n * freq(i)))
        ch, sh, cl, sl = at(math.cos, 256 * q), at(math.sin, 256 * q), at(math.cos, r), at(math.sin, r)
        return f32(f32(ch * cl) - f32(sh * sl)), f32(f32(sh * cl) + f32(ch * sl))

    def turned_by(cs):
        out = []
        for j in range(16):
            i = j % 8
            c, s = cs(i)
            v = f32(f32(xs[j] * c) - f32(xs[j + 8] * s)) if j < 8 else f32(f32(xs[j] * c) + f32(xs[i] * s))
            out.append(round_bf16(float(v)))
        return out

    checked = stored_rope()
    b = Bindings(1, inputs={"x": [[float(v) for v in xs]]}, row_ints={"position": [[p]], "slot": [[0]]},
                 caches={"c": slots(16, [0.0] * 16)})
    own = list(evaluate(checked, b).caches["c"][0])
    assert own != turned_by(by_product), "binary32's angles rounded as the exact ones"
    for how, cs in (("products", by_product), ("tables", by_tables)):
        B.evaluate_stored(checked, b, Kept(caches={"c": slots(16, turned_by(cs))}))  # raises if refused, naming `how`


# Long dot products, and tight ones ------------------------------------------------

@pytest.mark.parametrize("k,seed", [(2048, 1), (2048, 2), (4096, 3), (4096, 4)])
def test_bounds_long_dots(k, seed):
    """ProgramTest.hs:1296-1312: binary32 dot products of k uniform terms,
    summed left to right or pairwise, stored rounded to bf16, are kept."""
    rng = np.random.default_rng(seed)
    w = rng.uniform(-1, 1, k).astype(np.float32)
    x = rng.uniform(-1, 1, k).astype(np.float32)
    products = (w * x).astype(np.float32)

    def pairwise(ps):
        if len(ps) == 0:
            return np.float32(0)
        if len(ps) == 1:
            return ps[0]
        h = len(ps) // 2
        return np.float32(pairwise(ps[:h]) + pairwise(ps[h:]))

    in_order = np.float32(0)
    for t in products:
        in_order = np.float32(in_order + t)
    checked = stored_dot_in(CACHE_BF16, k)
    b = dot_bindings(w.astype(np.float64), x.astype(np.float64))
    for v in (in_order, pairwise(products)):
        B.evaluate_stored(checked, b, Kept(caches={"c": slots(1, [round_bf16(float(v))])}))


@pytest.mark.parametrize("seed", range(12))
def test_bounds_tight(seed):
    """ProgramTest.hs:1318-1332: 64 positive terms; the rounding of the
    exact dot product is kept, and unless the exact value is within 2^-14
    (relative) of a midpoint, the bf16 values beside it are refused."""
    rng = np.random.default_rng(100 + seed)
    ws = rng.uniform(0.5, 1, 64).astype(np.float32).astype(np.float64)
    xs = rng.uniform(0.5, 1, 64).astype(np.float32).astype(np.float64)
    exact = 0.0
    for a, c in zip(ws, xs):
        exact += a * c
    own = round_bf16(exact)
    e = math.frexp(own)[1]
    step = 2.0 ** (e - 8)
    above = own + step
    below = own - step / 2 if own == 2.0 ** (e - 1) else own - step
    from_midpoints = min(exact - (below + own) / 2, (own + above) / 2 - exact) / exact
    assert keeps(ws, xs, own)
    if from_midpoints > 2.0 ** -14:
        assert not keeps(ws, xs, above)
        assert not keeps(ws, xs, below)


# Gathers ------------------------------------------------------------------------

def summed_program():
    def body(b):
        t = b.weight("table", [4, 2])
        tok = b.row_ints("rows", 2, 4)
        b.output("summed", b.gather("summed", t, tok, 0.5))

    return check_program(program("summed", body))


def test_eval_pooled_gather():
    """ProgramTest.hs:1623-1635: rows (0, 1) and (2, 3) of a table of 4 × 2,
    summed and halved: [[2, 3], [6, 7]]."""
    b = Bindings(2, weights={"table": [1, 2, 3, 4, 5, 6, 7, 8]}, row_ints={"rows": [[0, 1], [2, 3]]})
    checked = summed_program()
    assert [r.tolist() for r in evaluate(checked, b).outputs["summed"]] == [[2, 3], [6, 7]]
    assert [r.tolist() for r in evaluate_fast(checked, b).outputs["summed"]] == [[2, 3], [6, 7]]


def test_gather_bound_of_a_scaled_sum():
    """gatherA (Eval.hs:884-889): a sum of rows times a factor, bounded as
    the sum then the product or the products then the sum.  Every binary32
    order of the two lies within it, on rows whose sums round; a single
    row's bound is one binary32 rounding of its product, γ₁ |w f|."""
    rng = np.random.default_rng(7)
    f = 5.65625
    for _ in range(200):
        ws = (rng.standard_normal(3) * 10.0 ** rng.uniform(-3, 3, 3)).astype(np.float32).astype(np.float64)
        a = B.gather_a(list(ws), f)
        assert a.exact == (ws[0] + ws[1] + ws[2]) * f
        s = np.float32(np.float32(np.float32(ws[0]) + np.float32(ws[1])) + np.float32(ws[2]))
        by_sum = float(np.float32(s * np.float32(f)))
        by_dot = float(np.float32(np.float32(np.float32(ws[0] * f) + np.float32(ws[1] * f)) + np.float32(ws[2] * f)))
        for got in (by_sum, by_dot):
            assert abs(got - a.exact) <= a.bound
    one = B.gather_a([3.0], 0.5)
    assert one.exact == 1.5 and math.isclose(one.bound, 1.5 * B.gamma_n(1), rel_tol=1e-12)


def embed_program():
    """ProgramTest.hs:785-789: tokens to the residual stream, scaled."""
    def body(b):
        tokens = b.row_ints("tokens", 1, 64)
        embed = b.weight("embed", [64, 32])
        b.output("x", b.gather("x", embed, tokens, 5.65625))

    return check_program(program("embed", body))


def test_embed_program_scales_the_row():
    """The embedding row times 5.65625 (= 181/32); each element's bound is
    one binary32 rounding of its product."""
    rng = np.random.default_rng(9)
    table = np.array([round_bf16(v) for v in rng.standard_normal(64 * 32)])
    b = Bindings(1, weights={"embed": table.tolist()}, row_ints={"tokens": [[37]]})
    ev = evaluate(embed_program(), b)
    assert ev.outputs["x"][0].tolist() == (table.reshape(64, 32)[37] * 5.65625).tolist()
    bd = B.evaluate_bounds(embed_program(), b, ev)
    want = np.abs(table.reshape(64, 32)[37] * 5.65625) * B.gamma_n(1)
    assert np.allclose(bd.values["x"][0], want, rtol=1e-9, atol=1e-36)
