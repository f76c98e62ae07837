"""The decode attention cases the direct tests share (on the GPU, and the
oracle against binary64 on the CPU): seeded inputs, the oracle's run of the
KV store, the split attention and the combine, and the binary64 attention
with each output element's bound (src/FuryKernel/Program/Eval.hs:474-527,
attendBounds :891-918) over the caches the store left."""

from __future__ import annotations

import math

import numpy as np

from furykernel_amd.lower import rope_table
from oracle import bounds as B
from oracle import fkref

THETA = 10000.0

# heads, kv_heads, head_dim, split, length, position, window, bf16, rope, store
CASES = [
    (32, 4, 64, 128, 1024, 1000, 0, 0, 1, 1),
    (16, 4, 64, 64, 512, 200, 0, 0, 0, 0),
    (8, 4, 32, 128, 512, 300, 0, 1, 1, 1),
    (8, 1, 64, 128, 256, 250, 48, 0, 1, 0),
    (4, 4, 8, 64, 128, 70, 0, 0, 0, 1),
    (6, 2, 16, 128, 256, 128, 0, 1, 1, 1),
    (32, 8, 64, 128, 4096, 4095, 0, 0, 1, 1),
    # a window of 48 across the split boundary at 128, GQA 4
    (16, 4, 32, 128, 512, 150, 48, 0, 1, 1),
    # groups of 8 (two heads a lane); position 2048: split 16 holds one
    # position, splits 17-31 none
    (16, 2, 64, 128, 4096, 2048, 0, 1, 1, 1),
    # the 1B decode's shape (groups of 4, heads of 64, splits of 128, f16)
    # short of full splits: the new rows mid-split, the last wavefronts'
    # runs partly or wholly past the split's positions
    (16, 4, 64, 128, 1024, 1000, 0, 0, 1, 1),
    # ... a window starting mid-split, no RoPE, nothing stored
    (8, 2, 64, 128, 512, 300, 100, 0, 0, 0),
    # ... position 130: split 1 holds three positions, splits 2-31 none
    (32, 8, 64, 128, 4096, 130, 0, 0, 1, 1),
]


def case_id(c) -> str:
    return "h{}_kv{}_d{}_s{}_p{}_w{}_bf{}_r{}_st{}".format(c[0], c[1], c[2], c[3], c[5], c[6], c[7], c[8], c[9])


def _cache(rng, n, bf16):
    x = rng.standard_normal(n).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16) if bf16 else x.astype(np.float16).view(np.uint16)


def inputs(case) -> dict:
    heads, kv, d, split, length, pos, window, bf16, rope, store = case
    rng = np.random.default_rng(heads * 1000 + d * 10 + split + pos)
    splits = -(-length // split)
    return dict(
        heads=heads, kv=kv, d=d, split=split, length=length, pos=pos, window=window, bf16=bf16, rope=rope,
        store=store, splits=splits, rotated=d // 2, scale=float(np.float32(1.0 / np.sqrt(d))),
        theta=float(np.float32(THETA)),
        q=(rng.standard_normal(heads * d) * 0.5).astype(np.float32),
        knew=(rng.standard_normal(kv * d) * 0.5).astype(np.float32),
        vnew=rng.standard_normal(kv * d).astype(np.float32),
        kc=_cache(rng, kv * length * d, bf16), vc=_cache(rng, kv * length * d, bf16),
        table=rope_table(float(np.float32(THETA)), d, d // 2, length).astype(np.float32))


def oracle(x: dict) -> dict:
    """The oracle's store (if asked), split attention and combine."""
    L = fkref.lib()
    kc, vc = x["kc"].copy(), x["vc"].copy()
    heads, kv, d, splits = x["heads"], x["kv"], x["d"], x["splits"]
    part = np.zeros(heads * splits * (d + 2), np.float32)
    out = np.zeros(heads * d, np.float32)
    if x["store"]:
        assert L.fkref_step_store(x["knew"].ctypes.data, x["vnew"].ctypes.data, kc.ctypes.data, vc.ctypes.data, 2,
                                  x["rope"], 0, kv, d, x["length"], 1, x["rotated"], x["theta"], x["pos"], 0,
                                  x["bf16"]) == 0
    assert L.fkref_step_attend(x["q"].ctypes.data, kc.ctypes.data, vc.ctypes.data, part.ctypes.data, heads, kv, d,
                               x["length"], 1, splits, x["split"], x["rope"], x["rotated"], x["theta"], x["scale"],
                               x["window"], x["pos"], 0, x["bf16"]) == 0
    assert L.fkref_step_combine(part.ctypes.data, out.ctypes.data, heads, d, splits) == 0
    return dict(kc=kc, vc=vc, partials=part, out=out)


def oracle_wide(x: dict, split: int) -> dict:
    """The oracle's store (if asked), wide-split attention (splits of `split`
    positions, 64 a run) and combine: the kernels' other attention order."""
    L = fkref.lib()
    kc, vc = x["kc"].copy(), x["vc"].copy()
    heads, kv, d = x["heads"], x["kv"], x["d"]
    splits = -(-x["length"] // split)
    part = np.zeros(heads * splits * (d + 2), np.float32)
    out = np.zeros(heads * d, np.float32)
    if x["store"]:
        assert L.fkref_step_store(x["knew"].ctypes.data, x["vnew"].ctypes.data, kc.ctypes.data, vc.ctypes.data, 2,
                                  x["rope"], 0, kv, d, x["length"], 1, x["rotated"], x["theta"], x["pos"], 0,
                                  x["bf16"]) == 0
    assert L.fkref_step_attend_wide(x["q"].ctypes.data, kc.ctypes.data, vc.ctypes.data, part.ctypes.data, heads, kv,
                                    d, x["length"], 1, splits, split, x["rope"], x["rotated"], x["theta"], x["scale"],
                                    x["window"], x["pos"], 0, x["bf16"]) == 0
    assert L.fkref_step_combine(part.ctypes.data, out.ctypes.data, heads, d, splits) == 0
    return dict(kc=kc, vc=vc, partials=part, out=out, splits=splits)


# Cases the wide kernel takes (heads of 16, 32 or 64), with its splits.
WIDE = [(c, S) for c in CASES if c[2] in (16, 32, 64) for S in ((64, 512) if c[4] >= 1024 else (64, 192))]


def widen_cache(c: np.ndarray, bf16: int) -> np.ndarray:
    """Cache elements as binary64 (exact)."""
    if bf16:
        return (c.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return c.view(np.float16).astype(np.float64)


def positions(x: dict) -> np.ndarray:
    pos, window = x["pos"], x["window"]
    first = max(0, pos - window + 1) if window else 0
    return np.arange(first, pos + 1)


def table_rotate(x: dict, v: np.ndarray) -> np.ndarray:
    """One head rotated in binary64 by the cosines and sines of the binary32
    RoPE table the kernels read (row pos): the kernels' rotation without their
    roundings."""
    d, half, rot = x["d"], x["d"] // 2, x["rotated"]
    cs = x["table"].reshape(-1, rot, 2)[x["pos"]].astype(np.float64)
    out = v.copy()
    for j in range(half):
        if j < rot:
            c, s = cs[j]
            out[j] = v[j] * c - v[j + half] * s
            out[j + half] = v[j + half] * c + v[j] * s
    return out


def f64_attention(x: dict, kc: np.ndarray, vc: np.ndarray, rotate=None) -> np.ndarray:
    """[heads, d]: each query head (RoPE'd exactly, or by `rotate`) over its
    kv head h div group, positions [first, pos], reading the caches as they
    stand."""
    heads, kv, d, length = x["heads"], x["kv"], x["d"], x["length"]
    group = heads // kv
    K = widen_cache(kc, x["bf16"]).reshape(kv, length, d)
    V = widen_cache(vc, x["bf16"]).reshape(kv, length, d)
    ts = positions(x) % length
    out = np.empty((heads, d))
    for h in range(heads):
        q = x["q"][h * d:(h + 1) * d].astype(np.float64)
        if x["rope"]:
            q = (rotate or _rotate)(x, q)
        s = x["scale"] * (K[h // group, ts] @ q)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ V[h // group, ts]
    return out


def _rotate(x: dict, v: np.ndarray) -> np.ndarray:
    from oracle.eval import rotate
    return rotate(x["theta"], x["rotated"], x["d"], float(x["pos"]), v)


def element_bounds(x: dict, kc: np.ndarray, vc: np.ndarray, h: int) -> np.ndarray:
    """Query head h's output elements' bounds (attendBounds, Eval.hs:891-918):
    the scores' from the query's rotation bound and dotA, the values exact."""
    heads, kv, d, length = x["heads"], x["kv"], x["d"], x["length"]
    group = heads // kv
    K = widen_cache(kc, x["bf16"]).reshape(kv, length, d)
    V = widen_cache(vc, x["bf16"]).reshape(kv, length, d)
    ts = positions(x) % length
    q = x["q"][h * d:(h + 1) * d].astype(np.float64)
    qa = [B.exact_a(v) for v in q]
    if x["rope"]:
        ex = _rotate(x, q)
        bd = B.rotation_bounds(x["theta"], x["rotated"], d, float(x["pos"]), qa)
        qa = [B.Approx(float(e), float(b)) for e, b in zip(ex, bd)]
    sc = B.const_a(x["scale"])
    scores = []
    for t in ts:
        ks = [B.exact_a(v) for v in K[h // group, t]]
        on_dot = B.product_a([B.dot_a(list(zip(qa, ks))), sc])
        on_query = B.dot_a([(B.product_a([e, sc]), k) for e, k in zip(qa, ks)])
        scores.append(B.Approx(on_dot.exact, max(on_dot.bound, on_query.bound)))
    values = [[B.exact_a(v) for v in V[h // group, ts, i]] for i in range(d)]
    return np.array([B.widened(b) for b in B.attend_bounds(scores, values)])


def within_bounds(x: dict, o: dict, got: np.ndarray, heads_checked) -> None:
    """Asserts, over the caches `o` left:
    * each checked head's output elements within their bounds of the binary64
      attention (the evaluator's exact rotation), and every head within 1e-4
      of the row's largest magnitude (the f32-against-f64 bar);
    * every head within 1e-5 of binary64 attention whose query is rotated by
      the same binary32 table the kernels read: what is left is the kernels'
      binary32 scores, exponentials, split sums and combine."""
    want = f64_attention(x, o["kc"], o["vc"])
    got = np.asarray(got, np.float64).reshape(want.shape)
    err = np.abs(got - want)
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    for h in heads_checked:
        b = element_bounds(x, o["kc"], o["vc"], h)
        assert np.all(err[h] <= b), (h, float(np.max(err[h] - b)))
    assert np.all(err <= 1e-4 * scale), float(np.max(err / scale))
    tab = f64_attention(x, o["kc"], o["vc"], rotate=table_rotate)
    err_t = np.abs(got - tab)
    assert np.all(err_t <= 1e-5 * np.max(np.abs(tab), axis=1, keepdims=True)), \
        float(np.max(err_t / np.max(np.abs(tab), axis=1, keepdims=True)))
