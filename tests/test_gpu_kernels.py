"""The standalone kernels on the GPU, through the C ABI, against the oracle.

Bars (the reference's CPU target is SIMD width 32, gfx950's wavefront 64):
* bit for bit against the oracle in the kernel's own order (width 64), which
  for the GEMVs is also the CPU target's width-32 split-2 order;
* within 1e-5 relative (to the row's magnitude) of the CPU target's default
  width-32 split-1 order, and of f64;
* exps are binary64's rounded once: the oracle's libm and the GPU's may round
  a value within their error of a binary32 midpoint differently, so those
  outputs are held to 1 ulp (src/FuryKernel/IR.hs:119-127 states the same
  leeway between platforms), and to being rare.
"""

import numpy as np
import pytest

from oracle import fkref

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(2027)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def ulps(a, b):
    ia = bits(a).astype(np.int64)
    ib = bits(b).astype(np.int64)
    ia = np.where(ia & 0x80000000, 0x80000000 - ia, ia)
    ib = np.where(ib & 0x80000000, 0x80000000 - ib, ib)
    return np.abs(ia - ib)


def run_gemv(device, kernels, w, x, wtype, r=1, scale=None):
    n, k = w.shape
    bw, bx, by = device.upload(w), device.upload(x), device.alloc(n * 4)
    bs = device.upload(scale) if scale is not None else None
    print(f"gemv {wtype} {n}x{k} r{r}", flush=True)
    kernels.gemv(bw, bx, by, n, k, wtype=wtype, rows_per_wave=r, scale=bs)
    device.sync()
    out = by.read(np.float32, n)
    for b in (bw, bx, by, bs):
        if b is not None:
            b.free()
    return out


@pytest.mark.parametrize("r", [1, 2, 4])
def test_gemv_f32_4096(device, kernels, r):
    n = k = 4096
    w = RNG.uniform(-1, 1, (n, k)).astype(np.float32)
    x = RNG.uniform(-1, 1, k).astype(np.float32)
    got = run_gemv(device, kernels, w, x, "f32", r)
    assert np.array_equal(bits(got), bits(fkref.gemv(w, x, 64, 4, 1)))
    assert np.array_equal(bits(got), bits(fkref.gemv(w, x, 32, 4, 2)))
    mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
    cpu32 = fkref.gemv(w, x, 32, 4, 1)
    assert np.max(np.abs(got - cpu32) / mag) < 1e-5
    exact = w.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - exact) / mag) < 1e-5


@pytest.mark.parametrize("n,k,r", [(3072, 2048, 1), (2048, 2048, 2), (8192, 2048, 4), (2048, 8192, 1),
                                   (37, 8, 1), (65, 136, 2), (1, 2048, 4)])
def test_gemv_f16_decode_shapes_and_ragged(device, kernels, n, k, r):
    w = RNG.normal(0, 0.02, (n, k)).astype(np.float16)
    x = RNG.normal(0, 1, k).astype(np.float32)
    got = run_gemv(device, kernels, w, x, "f16", r)
    assert np.array_equal(bits(got), bits(fkref.gemv(w, x, 64, 8, 1)))


def test_gemv_i8_8192(device, kernels):
    n = k = 8192
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    x = RNG.normal(0, 1, k).astype(np.float16)
    s = RNG.uniform(0.001, 0.01, n).astype(np.float32)
    got = run_gemv(device, kernels, w, x, "i8", 2, scale=s)
    assert np.array_equal(bits(got), bits(fkref.gemv(w, x, 64, 16, 1, row_scale=s)))
    assert np.array_equal(bits(got), bits(fkref.gemv(w, x, 32, 16, 2, row_scale=s)))


@pytest.mark.parametrize("r,k", [(1, 8192), (2, 8192), (4, 8192), (1, 1040), (2, 4096), (4, 2064)])
def test_gemv_i8_edge_values_bit_exact(device, kernels, r, k):
    """The reference chain's order bit for bit on the whole int8 range (-128
    and 0 included) against x with f16 subnormals, signed zeros, its
    largest values and cancelling pairs, full and ragged rows, every load in
    flight and the loop form of the widest rows."""
    n = 512
    rng = np.random.default_rng(17 + r)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    w[:, ::7] = 0
    pick = rng.integers(0, 6, k)
    x = np.select([pick == 0, pick == 1, pick == 2, pick == 3, pick == 4],
                  [rng.integers(1, 1024, k) * 2.0 ** -24, np.where(rng.integers(0, 2, k) == 1, -0.0, 0.0),
                   rng.choice([-65504.0, 65504.0], k), rng.normal(0, 1, k) * 2.0 ** 10, rng.normal(0, 1, k)],
                  rng.normal(0, 1e-3, k)).astype(np.float16)
    x[1::2][:100] = -x[0::2][:100]  # pairs that cancel
    s = np.ones(n, np.float32)
    got = run_gemv(device, kernels, w, x, "i8", r, scale=s)
    assert np.array_equal(bits(got), bits(fkref.gemv(w, x, 64, 16, 1, row_scale=s)))


@pytest.mark.parametrize("n,r,threads", [(37, 1, 256), (9, 2, 256), (5, 1, 128), (70, 2, 64)])
def test_gemv_i8_ragged_rows_full_width(device, kernels, n, r, threads):
    """Full rows of 8192 with fewer rows than the last threadgroup holds: in
    256-thread groups x goes through LDS and every wavefront reaches its
    barrier (rows past n read row n - 1 and store nothing); smaller groups
    take the loop form.  Bit for bit against the oracle, and y past n left
    as it was."""
    k = 8192
    rng = np.random.default_rng(n * 10 + r)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    x = rng.normal(0, 1, k).astype(np.float16)
    s = rng.uniform(0.001, 0.01, n).astype(np.float32)
    rows_per_group = threads // 64 * r
    pad = -(-n // rows_per_group) * rows_per_group
    bw, bx, bs = device.upload(w), device.upload(x), device.upload(s)
    by = device.upload(np.full(pad, 7.0, np.float32))
    print(f"gemv i8 {n}x{k} r{r} {threads} threads", flush=True)
    kernels.gemv(bw, bx, by, n, k, wtype="i8", rows_per_wave=r, threads=threads, scale=bs)
    device.sync()
    out = by.read(np.float32, pad)
    for b in (bw, bx, by, bs):
        b.free()
    assert np.array_equal(bits(out[:n]), bits(fkref.gemv(w, x, 64, 16, 1, row_scale=s)))
    assert np.all(out[n:] == 7.0)


def test_gemv_i8_integer_closed_form(device, kernels):
    n, k = 256, 8192
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    x = RNG.integers(-8, 9, k).astype(np.float16)
    s = RNG.uniform(0.001, 0.01, n).astype(np.float32)
    got = run_gemv(device, kernels, w, x, "i8", 1, scale=s)
    exact = w.astype(np.int64) @ x.astype(np.int64)
    assert np.array_equal(got, (exact.astype(np.float32) * s).astype(np.float32))


@pytest.mark.parametrize("threads", [256, 1024])
def test_rmsnorm_64x4096(device, kernels, threads):
    rows, h = 64, 4096
    x = RNG.uniform(-1, 1, (rows, h)).astype(np.float32)
    g = RNG.uniform(-1, 1, h).astype(np.float32)
    bx, bg, by = device.upload(x), device.upload(g), device.alloc(x.nbytes)
    print(f"rmsnorm {rows}x{h} t{threads}", flush=True)
    kernels.rmsnorm(bx, bg, by, rows, h, eps=1e-6, threads=threads)
    device.sync()
    got = by.read(np.float32).reshape(rows, h)
    want = fkref.rmsnorm(x, g, 1e-6, threads=threads, width=64, pack=4)
    # rsqrt is binary64's rounded once: one value a row, held to 1 ulp.
    u = ulps(got, want)
    assert u.max() <= 1
    assert np.mean(u > 0) < 1e-3
    cpu32 = fkref.rmsnorm(x, g, 1e-6, threads=256, width=32, pack=1)
    assert np.max(np.abs(got - cpu32) / (np.abs(cpu32) + 1e-30)) < 1e-5
    for b in (bx, bg, by):
        b.free()


def test_rmsnorm_segments_factor_no_gamma(device, kernels):
    rows, h, seg = 3, 512, 64
    x = RNG.uniform(-4, 4, (rows, h)).astype(np.float32)
    bx, by = device.upload(x), device.alloc(x.nbytes)
    print("rmsnorm segments", flush=True)
    kernels.rmsnorm(bx, None, by, rows, h, seg=seg, eps=1e-5, factor=0.5, threads=64)
    device.sync()
    got = by.read(np.float32).reshape(rows, h)
    want = fkref.rmsnorm(x, None, 1e-5, threads=64, width=64, pack=4, seg=seg, factor=0.5)
    assert ulps(got, want).max() <= 1


@pytest.mark.parametrize("threads", [256, 1024])
def test_softmax_64x4096(device, kernels, threads):
    rows, n = 64, 4096
    x = RNG.uniform(-1, 1, (rows, n)).astype(np.float32)
    bx, by = device.upload(x), device.alloc(x.nbytes)
    print(f"softmax {rows}x{n} t{threads}", flush=True)
    kernels.softmax(bx, by, rows, n, threads=threads)
    device.sync()
    got = by.read(np.float32).reshape(rows, n)
    want = fkref.softmax(x, threads=threads, width=64, pack=4)
    u = ulps(got, want)
    assert u.max() <= 2
    assert np.mean(u > 0) < 1e-3
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(axis=1, keepdims=True))
    spec = e / e.sum(axis=1, keepdims=True)
    assert np.max(np.abs(got - spec) / spec) < 1e-5


def test_memset_is_refused_while_the_stream_is_captured(device, kernels):
    """fk_memset_async returns FK_ERR_STATE under capture (a graph clears
    memory with a kernel); outside capture it sets the bytes."""
    from furykernel_amd import runtime

    buf = device.alloc(4096)
    print("memset under capture", flush=True)
    with pytest.raises(runtime.FkError) as err:
        with device.capture() as out:
            buf.fill_bytes(7)
    assert err.value.status == -5
    buf.fill_bytes(7)
    device.sync()
    assert np.all(buf.read(np.uint8, 4096) == 7)
    kernels.fill_u32(buf, 0)
    device.sync()
    assert np.all(buf.read(np.uint32, 1024) == 0)
    buf.free()
