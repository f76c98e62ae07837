"""The oracle's decode attention — the KV store, the split attention and the
combine of the splits (oracle/fkref.c, the order the GPU kernels keep) —
against binary64 attention (src/FuryKernel/Program/Eval.hs:474-527): every
element within attendBounds' bound (:891-918) and within 1e-4 of the row's
largest magnitude, and within 1e-5 of binary64 attention whose query is
rotated by the binary32 RoPE table the kernels read.  Cases: the 1B shape (32 heads over 8, width 64, 32
splits of 128, position 4095), GQA groups 1 to 8, windows inside a split and
across a split boundary, splits of 64, bf16 caches, the new key RoPE'd.

Planted mistakes (in the oracle's outputs, on the CPU) show the checks see
what a wrong combine or grouping would do: a split dropped from the combine,
the query heads paired with the wrong kv heads."""

import numpy as np
import pytest

from attention_cases import WIDE, CASES, case_id, f64_attention, inputs, oracle, oracle_wide, within_bounds
from oracle import fkref


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_split_attention_and_combine_within_the_f64_bounds(case):
    x = inputs(case)
    o = oracle(x)
    heads = x["heads"]
    # the bound (pure Python) on the first and last query head of the first
    # and last kv head; the relative bars on every head
    group = heads // x["kv"]
    within_bounds(x, o, o["out"], sorted({0, group - 1, heads - group, heads - 1}))


@pytest.mark.parametrize("case,split", WIDE, ids=lambda c: case_id(c) if isinstance(c, tuple) else f"S{c}")
def test_wide_split_attention_and_combine_within_the_f64_bounds(case, split):
    """The wide-split order (runs of 64, merged in the threadgroup) against the
    same binary64 attention and bounds; its caches are the narrow order's."""
    x = inputs(case)
    o = oracle_wide(x, split)
    heads, group = x["heads"], x["heads"] // x["kv"]
    within_bounds(x, o, o["out"], sorted({0, heads - 1}))
    n = oracle(x)
    assert np.array_equal(o["kc"], n["kc"]) and np.array_equal(o["vc"], n["vc"])


def test_the_new_rows_are_ones_a_kernel_may_store():
    """Each stored key element is one a kernel may store for the binary64
    rotation of the new row (mayStore, Eval.hs:935-943, with the rotation's
    bound, :834-846); each value element is the new value rounded once."""
    from attention_cases import _rotate, widen_cache
    from oracle import bounds as B
    from oracle.eval import round_cache
    for case in CASES:
        x = inputs(case)
        if not x["store"]:
            continue
        o = oracle(x)
        kv, d, length, pos = x["kv"], x["d"], x["length"], x["pos"]
        elem = "bf16" if x["bf16"] else "f16"
        K = widen_cache(o["kc"], x["bf16"]).reshape(kv, length, d)
        V = widen_cache(o["vc"], x["bf16"]).reshape(kv, length, d)
        for g in range(kv):
            k = x["knew"][g * d:(g + 1) * d].astype(np.float64)
            if x["rope"]:
                ex = _rotate(x, k)
                bd = B.rotation_bounds(x["theta"], x["rotated"], d, float(pos), [B.exact_a(v) for v in k])
            else:
                ex, bd = k, [0.0] * d
            for j in range(d):
                assert B.may_store(elem, B.Approx(float(ex[j]), bd[j]), float(K[g, pos % length, j])), (case, g, j)
            v = x["vnew"][g * d:(g + 1) * d].astype(np.float64)
            assert np.array_equal(V[g, pos % length], [round_cache(elem, float(e)) for e in v])


def _combine(part, heads, d, splits):
    out = np.zeros(heads * d, np.float32)
    assert fkref.lib().fkref_step_combine(part.ctypes.data, out.ctypes.data, heads, d, splits) == 0
    return out


def test_a_dropped_split_fails_the_check():
    """The 1B shape with one of the 32 splits left out of the combine (its sum
    zeroed, its maximum at -inf): far outside the bound."""
    x = inputs(CASES[6])
    o = oracle(x)
    heads, d, splits = x["heads"], x["d"], x["splits"]
    part = o["partials"].copy()
    stats = part[heads * splits * d:].reshape(heads, splits, 2)
    acc = part[:heads * splits * d].reshape(heads, splits, d)
    stats[:, 17, 0] = -np.inf
    stats[:, 17, 1] = 0.0
    acc[:, 17, :] = 0.0
    bad = _combine(part, heads, d, splits)
    with pytest.raises(AssertionError):
        within_bounds(x, o, bad, [0])


def test_a_wrong_grouping_fails_the_check():
    """Query head h paired with kv head h mod kv_heads instead of h div group."""
    x = inputs(CASES[6])
    o = oracle(x)
    heads, kv, d = x["heads"], x["kv"], x["d"]
    group = heads // kv
    perm = np.array([(h % kv) * group + h // kv for h in range(heads)])
    # running the oracle with the query heads permuted so that its head
    # perm[h] works on kv head h mod kv: the outputs put back in order
    y = dict(x, q=x["q"].reshape(heads, d)[np.argsort(perm)].reshape(-1).copy())
    wrong = oracle(y)["out"].reshape(heads, d)[perm].reshape(-1)
    assert not np.allclose(wrong, o["out"])
    with pytest.raises(AssertionError):
        within_bounds(x, o, wrong, [1])


def test_f64_attention_closed_form():
    """The binary64 reference itself: with every key equal the weights are
    uniform and the output is the mean of the values; with one key far above
    the rest the output is that position's value."""
    x = inputs(CASES[4])
    kv, d, length = x["kv"], x["d"], x["length"]
    kc = np.full(kv * length * d, np.float16(0.25)).view(np.uint16)
    vc = x["vc"]
    got = f64_attention(dict(x, rope=0), kc, vc)
    V = vc.view(np.float16).astype(np.float64).reshape(kv, length, d)
    ts = np.arange(0, x["pos"] + 1)
    group = x["heads"] // kv
    for h in range(x["heads"]):
        assert np.allclose(got[h], V[h // group, ts].mean(axis=0), rtol=1e-12, atol=1e-12)
    kc2 = np.zeros(kv * length * d, np.float16)
    kc2.reshape(kv, length, d)[:, 5, :] = 60.0
    q = np.abs(x["q"]) + 1.0
    got2 = f64_attention(dict(x, rope=0, q=q.astype(np.float32)), kc2.view(np.uint16), vc)
    for h in range(x["heads"]):
        assert np.allclose(got2[h], V[h // group, 5], rtol=1e-9, atol=1e-9)
