"""The prefill GEMM (fk_gemm.h) on the GPU against f64 sums of its f16 operands.

The matrix cores sum over k in their own order, so the bar is the reference's
bound for binary32 accumulation (test/Test/FuryKernel/GemvTest.hs:127-130;
the tile contract of src/FuryKernel/Tile.hs:5-24): |C - exact| <=
2 (k + 64) 2^-24 sum |a b| + 2^-126.  Small shapes check every element (and so
the lane layout of v_mfma_f32_16x16x32_f16 and the tile layout); the 1B
prefill's shapes check sampled rows.  The SiLU·mul epilogue rounds to f16:
within 2e-3 relative (the f16 bar) of the f64 value.
"""

import numpy as np
import pytest

from furykernel_amd.layout import pack, pair, unpack

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(2028)


def f16(shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float16)


def bound(a, b):
    """Per element of a b^T: 2 (k + 64) 2^-24 sum |a b| + 2^-126."""
    k = a.shape[1]
    mag = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)).T
    return 2 * (k + 64) * 2.0**-24 * mag + 2.0**-126


def run(device, kernels, a, bs, mode="store", r=None, act=0):
    """bs: the weights; for "silu_mul", [gate, up] (act: the activation,
    SiLU 0 or GELU-tanh 1)."""
    m, k = a.shape
    ba = device.upload(pack(a))
    if mode == "silu_mul":
        rows = [bs[0].shape[0]]
        bb = [device.upload(pack(pair(*bs)))]
        cs = [device.alloc(m * rows[0] * 2)]
    else:
        rows = [b.shape[0] for b in bs]
        bb = [device.upload(pack(b)) for b in bs]
        cs = [device.alloc(m * n * 4) for n in rows]
    br = device.upload(r) if r is not None else None
    print(f"gemm {mode} m {m} k {k} rows {rows}", flush=True)
    kernels.gemm(ba, bb, cs, m, k, rows, mode, br, act=act)
    device.sync()
    if mode == "silu_mul":
        out = [unpack(cs[0].read(np.float16, m * rows[0]), m, rows[0])]
    else:
        out = [c.read(np.float32, m * n).reshape(m, n) for c, n in zip(cs, rows)]
    for buf in [ba, *bb, *cs] + ([br] if br is not None else []):
        buf.free()
    return out


def silu_mul(a, g, u):
    ge = a.astype(np.float64) @ g.astype(np.float64).T
    ue = a.astype(np.float64) @ u.astype(np.float64).T
    return ge / (1 + np.exp(-ge)) * ue


@pytest.mark.parametrize("m,k,n", [(256, 64, 256), (256, 128, 256), (512, 192, 512), (256, 2048, 768)])
def test_gemm_every_element_within_the_accumulation_bound(device, kernels, m, k, n):
    a, b = f16((m, k)), f16((n, k))
    (c,) = run(device, kernels, a, [b])
    exact = a.astype(np.float64) @ b.astype(np.float64).T
    assert np.all(np.abs(c - exact) <= bound(a, b))


def test_gemm_exact_on_small_integers(device, kernels):
    """Integers of f16 whose products and sums stay below 2^24: every order
    gives the exact sum, so the kernel's result is bit for bit the sum."""
    a = RNG.integers(-8, 9, (256, 256)).astype(np.float16)
    b = RNG.integers(-8, 9, (512, 256)).astype(np.float16)
    (c,) = run(device, kernels, a, [b])
    assert np.array_equal(c, (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32))


def test_gemm_three_anchors_into_three_outputs(device, kernels):
    """q, k, v projections of one input: anchors of 512, 256, 256 rows."""
    a = f16((256, 128))
    bs = [f16((512, 128)), f16((256, 128)), f16((256, 128))]
    outs = run(device, kernels, a, bs)
    for b, c in zip(bs, outs):
        exact = a.astype(np.float64) @ b.astype(np.float64).T
        assert np.all(np.abs(c - exact) <= bound(a, b))


def test_gemm_residual_epilogue(device, kernels):
    a, b = f16((512, 256)), f16((256, 256))
    r = RNG.standard_normal((512, 256)).astype(np.float32)
    (c,) = run(device, kernels, a, [b], "add", r)
    exact = r.astype(np.float64) + a.astype(np.float64) @ b.astype(np.float64).T
    # the residual's addition rounds once more
    assert np.all(np.abs(c - exact) <= bound(a, b) + np.abs(exact) * 2.0**-24)


def test_gemm_residual_in_place(device, kernels):
    """The residual epilogue reads and writes the same rows: R may be C."""
    a, b = f16((256, 128)), f16((256, 128))
    r = RNG.standard_normal((256, 256)).astype(np.float32)
    ba, bb, br = device.upload(pack(a)), device.upload(pack(b)), device.upload(r)
    kernels.gemm(ba, [bb], [br], 256, 128, [256], "add", br)
    device.sync()
    c = br.read(np.float32, 256 * 256).reshape(256, 256)
    exact = r.astype(np.float64) + a.astype(np.float64) @ b.astype(np.float64).T
    assert np.all(np.abs(c - exact) <= bound(a, b) + np.abs(exact) * 2.0**-24)
    for x in (ba, bb, br):
        x.free()


def gelu_mul(a, g, u):
    """0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) u in binary64."""
    ge = a.astype(np.float64) @ g.astype(np.float64).T
    ue = a.astype(np.float64) @ u.astype(np.float64).T
    return 0.5 * ge * (1 + np.tanh(np.sqrt(2 / np.pi) * (ge + 0.044715 * ge ** 3))) * ue


@pytest.mark.parametrize("act", [0, 1], ids=["silu", "gelu-tanh"])
def test_gemm_act_mul_epilogue_writes_the_tile_layout(device, kernels, act):
    """The gate/up GEMM's epilogue with each activation, within the f16 bar
    of binary64 (gate values of either sign, out to |g| of about 8, where
    both activations bend)."""
    a = f16((256, 256), 0.5)
    g, u = f16((384, 256), 0.5), f16((384, 256), 0.5)
    (c,) = run(device, kernels, a, [g, u], "silu_mul", act=act)
    exact = (gelu_mul if act else silu_mul)(a, g, u)
    ge = a.astype(np.float64) @ g.astype(np.float64).T
    assert np.min(ge) < -4 and np.max(ge) > 4
    err = np.abs(c.astype(np.float64) - exact)
    assert np.max(err) <= 2e-3 * np.max(np.abs(exact))
    # the two activations differ far beyond the bar: the branch is taken
    other = (silu_mul if act else gelu_mul)(a, g, u)
    assert np.max(np.abs(other - exact)) > 4 * 2e-3 * np.max(np.abs(exact))


@pytest.mark.parametrize("k,rows,mode", [(2048, [2048, 512, 512], "store"), (2048, [2048], "add"),
                                         (2048, [8192], "silu_mul"), (8192, [2048], "add")])
def test_gemm_at_the_1b_prefill_shapes(device, kernels, k, rows, mode):
    """8192 rows (4 sequences of 2048); QKV, O, gate/up with SiLU·mul, down.
    Sampled rows against f64."""
    m = 8192
    a = f16((m, k), 0.5)
    bs = [f16((n, k), 0.02) for n in rows] if mode != "silu_mul" else [f16((rows[0], k), 0.02) for _ in range(2)]
    r = RNG.standard_normal((m, rows[0])).astype(np.float32) if mode == "add" else None
    outs = run(device, kernels, a, bs, mode, r)
    pick = np.sort(RNG.choice(m, 48, replace=False))
    if mode == "silu_mul":
        exact = silu_mul(a[pick], bs[0], bs[1])
        err = np.abs(outs[0][pick].astype(np.float64) - exact)
        assert np.max(err) <= 2e-3 * np.max(np.abs(exact))
        return
    ad = a[pick].astype(np.float64)
    for b, c in zip(bs, outs):
        exact = ad @ b.astype(np.float64).T
        bnd = bound(a[pick], b)
        if r is not None:
            exact = exact + r[pick]
            bnd = bnd + np.abs(exact) * 2.0**-24
        assert np.all(np.abs(c[pick] - exact) <= bnd)


def test_gemm_refuses_shapes_it_does_not_take(device, kernels):
    from furykernel_amd.kernels import LaunchError

    a, b = device.alloc(256 * 64 * 2), device.alloc(256 * 64 * 2)
    c = device.alloc(256 * 256 * 4)
    with pytest.raises(LaunchError):
        kernels.gemm(a, [b], [c], 200, 64, [256])      # m not a multiple of 256
    with pytest.raises(LaunchError):
        kernels.gemm(a, [b], [c], 256, 32, [256])      # k not a multiple of 64
    with pytest.raises(LaunchError):
        kernels.gemm(a, [b], [c], 256, 64, [300])      # rows not a multiple of 256
    with pytest.raises(LaunchError):
        kernels.gemm(a, [b], [c], 256, 64, [1024])     # B smaller than the launch reads
    with pytest.raises(LaunchError):
        kernels.gemm(a, [b], [c], 256, 64, [256], "silu_mul")  # the pair is 2 x 256 rows
    for x in (a, b, c):
        x.free()


def _tokens_three_ways(device, kernels, a, b):
    """C = a bᵀ by the store GEMM and by the keys GEMM; the tokens of the
    keys, of fk_prefill_argmax over the stored rows, and of the oracle's
    fold over them."""
    from oracle import fkref
    L = fkref.lib()
    m, k = a.shape
    n = b.shape[0]
    ba, bb = device.upload(pack(a)), device.upload(pack(b))
    c0, c1 = device.alloc(m * n * 4), device.alloc(m * n * 4)
    keys, t0, t1 = device.alloc(m * (n // 128) * 8), device.alloc(m * 4), device.alloc(m * 4)
    print(f"gemm store_keys m {m} k {k} n {n}", flush=True)
    kernels.gemm(ba, [bb], [c0], m, k, [n], "store")
    kernels.gemm(ba, [bb], [c1], m, k, [n], "store_keys", keys=keys)
    kernels.prefill_argmax(c0, t0, m, n)
    kernels.prefill_argmax_keys(keys, t1, m, n // 128)
    device.sync()
    s0, s1 = c0.read(np.float32, m * n), c1.read(np.float32, m * n)
    by_keys, by_rows = t1.read(np.uint32, m), t0.read(np.uint32, m)
    for x in (ba, bb, c0, c1, keys, t0, t1):
        x.free()
    rows = s0.reshape(m, n)
    folded = np.array([L.fkref_argmax(np.ascontiguousarray(r).ctypes.data, n) for r in rows], np.uint32)
    return s0, s1, by_keys, by_rows, folded


def test_the_keys_gemm_stores_the_same_rows_and_leaves_the_greedy_tokens(device, kernels):
    """Random operands (ties are rare; the fold decides them)."""
    a, b = f16((512, 128)), f16((1024, 128))
    s0, s1, by_keys, by_rows, folded = _tokens_three_ways(device, kernels, a, b)
    assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32))
    assert np.array_equal(by_keys, folded) and np.array_equal(by_rows, folded)


# Rows of logits the fold has rules for, made exactly by one-hot rows of A
# against weights whose column 0 holds the pattern (every other column 0).
def _patterns(n=512):
    rng = np.random.default_rng(11)
    base = lambda: rng.standard_normal(n).astype(np.float16)  # noqa: E731
    pats = {}
    p = np.full(n, 1.5, np.float16)
    pats["all equal"] = p
    p = base(); p[5] = p[300] = 9.0
    pats["tie inside the row"] = p
    p = base(); p[127] = p[128] = 9.0
    pats["tie across 128 columns"] = p
    p = base(); p[16] = p[4] = 9.0
    pats["tie between lanes"] = p
    p = base(); p[n - 1] = 9.0
    pats["largest last"] = p
    p = base(); p[0] = np.nan; p[9] = 9.0
    pats["NaN first"] = p
    p = base(); p[7] = np.nan; p[100] = 9.0
    pats["NaN elsewhere"] = p
    p = base(); p[200] = p[300] = np.inf
    pats["two infinities"] = p
    pats["all -inf"] = np.full(n, -np.inf, np.float16)
    pats["all NaN"] = np.full(n, np.nan, np.float16)
    p = np.zeros(n, np.float16); p[::2] = -0.0
    pats["signed zeros"] = p
    p = -np.abs(base()); p[77] = -0.0; p[78] = 0.0
    pats["zero the largest"] = p
    return pats


@pytest.mark.parametrize("name", list(_patterns()))
def test_the_keys_gemm_follows_the_folds_rules(device, kernels, name):
    pat = _patterns()[name]
    m, k, n = 256, 64, len(pat)
    a = np.zeros((m, k), np.float16)
    a[:, 0] = 1.0
    b = np.zeros((n, k), np.float16)
    b[:, 0] = pat
    s0, s1, by_keys, by_rows, folded = _tokens_three_ways(device, kernels, a, b)
    assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32))
    assert np.array_equal(by_keys, folded) and np.array_equal(by_rows, folded)
    want = {"all equal": 0, "tie inside the row": 5, "tie across 128 columns": 127, "tie between lanes": 4,
            "largest last": n - 1, "NaN first": 0, "NaN elsewhere": 100, "two infinities": 200, "all -inf": 0,
            "all NaN": 0, "signed zeros": 0, "zero the largest": 77}[name]
    assert set(folded.tolist()) == {want}
