"""The oracle's kernels against what the mathematics fixes, as the reference's
own properties do (test/Test/FuryKernel/GemvTest.hs, ReduceTest.hs).
"""

import numpy as np
import pytest

from oracle import fkref

RNG = np.random.default_rng(2026)


def eighths(shape):
    """Multiples of 1/8 in [-1, 1]: products and sums exact in f32 (GemvTest.hs:77-79)."""
    return (RNG.integers(-8, 9, shape) / 8).astype(np.float32)


@pytest.mark.parametrize("width,pack,split", [(32, 4, 1), (32, 8, 2), (8, 4, 4), (64, 4, 1), (64, 8, 1)])
def test_gemv_exact_sums_give_the_spec_bit_for_bit(width, pack, split):
    """GemvTest.hs:105-109: on eighths every variant is its f64 spec, rounded once."""
    n, k = 24, pack * 40
    w, x = eighths((n, k)), eighths((3, k))
    y = fkref.gemv(w, x, width, pack, split)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.array_equal(y, exact.astype(np.float32))


def test_gemv_within_f32_accumulation_bound():
    """GemvTest.hs:111-135: within 2 (k + 64) 2^-24 sum|x w| + 2^-126 of f64."""
    n, k = 32, 1024
    w = RNG.uniform(-2, 2, (n, k)).astype(np.float32)
    x = RNG.uniform(-2, 2, (2, k)).astype(np.float32)
    y = fkref.gemv(w, x, 32, 4, 1)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    bound = 2 * (k + 64) * 2.0**-24 * mag + 2.0**-126
    assert np.all(np.abs(y - exact) <= bound)


def test_wave64_split1_is_the_cpu_targets_width32_split2():
    """The identity the gfx950 GEMV rests on: lane v of width 64 visits the packs
    lane v of split v // 32 does at width 32, and the width-64 pairwise tree's
    last addition is split-K's combine of the two width-32 partials."""
    for wdt, pack, k in [(np.float32, 4, 4096), (np.float16, 8, 2048), (np.float16, 8, 8192 + 8)]:
        w = RNG.uniform(-1, 1, (16, k)).astype(wdt)
        x = RNG.uniform(-1, 1, k).astype(np.float32)
        a = fkref.gemv(w, x, 64, pack, 1)
        b = fkref.gemv(w, x, 32, pack, 2)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # ...and differs, in general, from the width-32 split-1 order.
    w = RNG.uniform(-1, 1, (64, 4096)).astype(np.float32)
    x = RNG.uniform(-1, 1, 4096).astype(np.float32)
    assert not np.array_equal(fkref.gemv(w, x, 64, 4, 1), fkref.gemv(w, x, 32, 4, 1))


def test_gemv_rows_do_not_depend_on_the_batch():
    """GemvTest.hs:137-152."""
    k = 512
    w = RNG.uniform(-1, 1, (8, k)).astype(np.float32)
    row = RNG.uniform(-1, 1, k).astype(np.float32)
    batch = RNG.uniform(-1, 1, (5, k)).astype(np.float32)
    batch[3] = row
    assert np.array_equal(fkref.gemv(w, batch, 64, 4)[3], fkref.gemv(w, row, 64, 4))


def test_int8_gemv_closed_form():
    """Small-integer x: every product and partial sum is an integer below 2^24,
    exact in f32, so y = round(scale * exact sum)."""
    n, k = 16, 8192
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    x = RNG.integers(-8, 9, k).astype(np.float16)
    s = RNG.uniform(0.001, 0.01, n).astype(np.float32)
    y = fkref.gemv(w, x, 64, 16, 1, row_scale=s)
    exact = w.astype(np.int64) @ x.astype(np.int64)
    assert np.array_equal(y, (exact.astype(np.float32) * s).astype(np.float32))


@pytest.mark.parametrize("width", [8, 32, 64])
def test_rmsnorm_within_an_ulp_of_its_spec(width):
    """ReduceTest.hs:97-108: within one bf16 ulp of the f64 spec on every SIMD
    width; here the f32 output, within a few f32 ulps."""
    x = RNG.uniform(-8, 8, (3, 1000)).astype(np.float32)
    g = RNG.uniform(-2, 2, 1000).astype(np.float32)
    y = fkref.rmsnorm(x, g, 1e-6, threads=256, width=width, pack=1)
    xd = x.astype(np.float64)
    spec = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + np.float64(np.float32(1e-6))) * g
    assert np.max(np.abs(y - spec) / (np.abs(spec) + 1e-30)) < 2e-6


def test_rmsnorm_rows_do_not_depend_on_the_batch():
    x = RNG.uniform(-8, 8, (3, 256)).astype(np.float32)
    g = RNG.uniform(-2, 2, 256).astype(np.float32)
    alone = fkref.rmsnorm(x[1], g, 1e-6, threads=256, width=64)
    assert np.array_equal(fkref.rmsnorm(x, g, 1e-6, threads=256, width=64)[1], alone)


def test_softmax_against_f64():
    x = RNG.uniform(-1, 1, (4, 4096)).astype(np.float32)
    y = fkref.softmax(x, threads=256, width=64)
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(axis=1, keepdims=True))
    spec = e / e.sum(axis=1, keepdims=True)
    assert np.max(np.abs(y - spec) / spec) < 1e-5
    assert np.allclose(y.sum(axis=1), 1.0, atol=1e-5)


def _fold(x):
    """src/FuryKernel/Program/Eval.hs:681-685: foldl1, a later element wins
    only if strictly larger."""
    best = 0
    for i in range(1, len(x)):
        if x[i] > x[best]:
            best = i
    return best


@pytest.mark.parametrize("seed", range(40))
def test_argmax_keys_give_the_folds_index(seed):
    """The 64-bit key maximum the logits' GEMV step folds the greedy token into
    picks the index the evaluator's fold picks: ties to the lowest index, +0
    and -0 equal, a NaN at index 0 kept, NaNs elsewhere never taken."""
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 300))
    pool = np.array([0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan, 1e-40, -1e-40], np.float32)
    x = np.where(rng.random(n) < 0.5, rng.choice(pool, n), rng.integers(-3, 4, n)).astype(np.float32)
    if seed % 5 == 0:
        x[0] = np.nan
    L = fkref.lib()
    key = int(L.fkref_argmax_keyed(x.ctypes.data, n))
    assert 0xFFFFFFFF - (key & 0xFFFFFFFF) == _fold(x.tolist()) == int(L.fkref_argmax(x.ctypes.data, n))


def test_argmax_key_special_cases():
    L = fkref.lib()
    for x, want in [([-0.0, 0.0], 0), ([0.0, -0.0], 0), ([np.nan, 5.0], 0), ([5.0, np.nan, 6.0], 2),
                    ([-np.inf, np.nan], 0), ([1.0, 1.0, 2.0, 2.0], 2), ([-np.inf] * 3, 0), ([np.nan] * 3, 0)]:
        a = np.array(x, np.float32)
        key = int(L.fkref_argmax_keyed(a.ctypes.data, len(a)))
        assert 0xFFFFFFFF - (key & 0xFFFFFFFF) == want == _fold(a.tolist()), x


def test_gemv_rows_spread_over_threads_are_the_same_bits():
    """The all-cores CPU figure spreads the GEMV's rows over threads: each
    row's arithmetic, and so its bits, is the one thread's."""
    rng = np.random.default_rng(11)
    w = rng.standard_normal((300, 512)).astype(np.float16)
    x = rng.standard_normal(512).astype(np.float32)
    one = fkref.gemv(w, x, width=32, pack=8)
    L = fkref.lib()
    assert L.fkref_set_threads(8) == 0
    try:
        many = fkref.gemv(w, x, width=32, pack=8)
    finally:
        L.fkref_set_threads(1)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))
    assert L.fkref_set_threads(0) != 0
