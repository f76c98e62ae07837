"""The reference's kernels for the IR target's tests, restated with the
builder: test/Test/FuryKernel/Kernels.hs (scale, scalePacked, rmsnorm,
throughBlocks), Gemv.hs (the bf16 GEMV family), InterpTest.hs's and
BuildTest.hs's kernels, and test/cpu/Cases.hs's (the CPU target's cases).

Each is a function of the target's caps.  The reference writes some for a
32-lane target with 32 threads; on a target of wider SIMD groups their thread
count is the SIMD width (``at_least``), the rest as written.
"""

from __future__ import annotations

from dataclasses import dataclass

from furykernel_amd.ir import ir as I
from furykernel_amd.ir.build import (KernelBuilder, TargetCaps, exp_e, f32, fma_e, group_index, lit, log_e, max_e,
                                     min_e, narrow, narrow_clamped, narrow_wrapped, quot, rem, rsqrt_e, select,
                                     simd_group_index, simd_lane, sqrt_e, tanh_e, thread_index, to_f32, u32, widen)
from furykernel_amd.ir.reduce import combine_splits, tg_reduce_max, tg_reduce_sum
from furykernel_amd.ir.tile import GemmTile, gemm_tile
from furykernel_amd.program.graph import BF16, BOOL, F16, F32, I8, I32, U8, U32

# The reference's test targets (test/Test/FuryKernel/Targets.hs:26-58).
T8 = TargetCaps("T8", 8, 256, 16384, 31, 16, ())
T16 = TargetCaps("T16", 16, 512, 32768, 31, 16, ())
T32 = TargetCaps("T32", 32, 1024, 32768, 31, 16, (BF16, F16, F32))
T64 = TargetCaps("T64", 64, 1024, 65536, 31, 16, (F16,))
R, W, RW = I.READ, I.WRITE, I.READ_WRITE


def D(lo, hi, m=1):
    return I.DimRange(lo, hi, m)


def at_least(caps: TargetCaps, n: int) -> int:
    return max(n, caps.simd_width)


def built(k: KernelBuilder) -> I.Kernel:
    kernel, problems = k.done()
    assert problems == [], problems
    return kernel


# ---------------------------------------------------------------------------
# test/Test/FuryKernel/Kernels.hs

def scale(caps):
    k = KernelBuilder("scale", caps)
    n = k.dim("n", D(1, 65536))
    s = k.param("s", F32)
    x = k.buffer("x", R, BF16, n)
    y = k.buffer("y", W, BF16, n)
    k.threads(64)
    k.groups(1)
    with k.strided("i", n) as i:
        v = k.let("v", widen(F32, k.load(x, i)))
        k.store(y, i, narrow(BF16, v * s))
    return built(k)


def scale_packed(caps):
    k = KernelBuilder("scale_packed", caps)
    packs = k.dim("packs", D(1, 8192))
    s = k.param("s", F32)
    x = k.buffer("x", R, BF16, packs * 8)
    y = k.buffer("y", W, BF16, packs * 8)
    k.threads(64)
    k.groups(1)
    with k.strided("j", packs) as j:
        v = k.load_pack("v", 8, x, j)
        k.store_pack(y, j, [narrow(BF16, widen(F32, e) * s) for e in v])
    return built(k)


def rmsnorm(caps, hidden: int):
    """Kernels.hs:53-74: y = x / sqrt(mean x² + eps) * w, bf16 rows."""
    k = KernelBuilder("rmsnorm", caps)
    rows = k.dim("rows", D(1, 4096))
    eps = k.param("eps", F32)
    h = u32(hidden)
    x = k.buffer("x", R, BF16, rows * h)
    w = k.buffer("w", R, BF16, h)
    y = k.buffer("y", W, BF16, rows * h)
    k.threads(256)
    k.groups(rows)
    scratch = k.tg_array("scratch", F32, 32)
    base = k.let("base", group_index * h)
    acc = k.var("acc", f32(0.0))
    with k.strided("i", h) as i:
        v = k.let("v", widen(F32, k.load(x, base + i)))
        k.assign(acc, acc.get + v * v)
    total = tg_reduce_sum(k, "sum_sq", scratch, acc.get)
    sc = k.let("scale", rsqrt_e(total / to_f32(h) + eps))
    with k.strided("j", h) as j:
        k.store(y, base + j, narrow(BF16, widen(F32, k.load(x, base + j)) * sc * widen(F32, k.load(w, j))))
    return built(k)


def through_blocks(caps, distinct: bool = True, apart: bool = True):
    """Kernels.hs:82-101."""
    k = KernelBuilder("through_blocks", caps)
    entries = k.dim("entries", D(1, 2 ** 30))
    ids = k.buffer("ids", R, U32, 4)
    x = k.buffer("x", R, F32, 256)
    y = k.buffer("y", W, F32, 256)
    blocks = k.table("blocks", F32, entries, 16384, access=RW)
    if distinct:
        k.distinct(blocks)
    if apart:
        k.apart_via(blocks)
    k.threads(64)
    k.groups(4)
    e = k.let("e", k.load(ids, group_index))
    at = k.let("at", 16320 + thread_index)
    k.store_via(blocks, e, at, k.load(x, group_index * 64 + thread_index) * 2)
    k.store(y, group_index * 64 + thread_index, k.load_via(blocks, e, at))
    return built(k)


# ---------------------------------------------------------------------------
# test/Test/FuryKernel/Gemv.hs: the bf16 GEMV family, furykernel_amd/ir/gemv.py

from furykernel_amd.ir.gemv import GemvShape, GemvVariant  # noqa: E402
from furykernel_amd.ir.gemv import gemv as _gemv  # noqa: E402


def gemv(caps, name: str, sh: GemvShape, v: GemvVariant):
    kernel, problems = _gemv(caps, name, sh, v)
    assert problems == [], problems
    return kernel


# ---------------------------------------------------------------------------
# test/Test/FuryKernel/BuildTest.hs

def controlled(caps):
    k = KernelBuilder("controlled", caps)
    y = k.buffer("y", W, F32, 2)
    k.threads(64)
    k.groups(1)
    partial = k.tg_array("partial", F32, 2)
    s = k.simd_sum("s", f32(1.0))
    with k.when_lane(simd_lane.eq(0)):
        k.tg_store(partial, simd_group_index, s)
    k.barrier()
    with k.when_lane(thread_index < 2):
        k.store(y, thread_index, k.tg_load(partial, thread_index))
    return built(k)


def via_table(caps):
    k = KernelBuilder("via_table", caps)
    e = k.param("e", U32)
    arrays = k.table("arrays", F32, 4, 8)
    y = k.buffer("y", W, F32, 8)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index < 8):
        k.store(y, thread_index, k.load_via(arrays, e, thread_index))
    return built(k)


def product8(caps):
    k = KernelBuilder("product8", caps)
    a = k.buffer("a", R, F32, 64)
    b = k.buffer("b", R, F32, 64)
    c = k.buffer("c", W, F32, 64)
    k.threads(at_least(caps, 32))
    k.groups(1)
    acc = k.fragment("acc", F32)
    fa = k.fragment("fa", F32)
    fb = k.fragment("fb", F32)
    k.frag_load(fa, a, 0, 8)
    k.frag_load(fb, b, 0, 8)
    k.frag_mma(acc, fa, fb, acc)
    k.frag_store(c, 0, 8, acc)
    return built(k)


# ---------------------------------------------------------------------------
# test/Test/FuryKernel/InterpTest.hs

def lanes(caps):
    k = KernelBuilder("lanes", caps)
    y = k.buffer("y", W, U32, 64)
    k.threads(64)
    k.groups(1)
    with k.when_lane(simd_lane < 3):
        k.store(y, thread_index, 1)
    with k.when_lane(simd_lane >= 3):
        k.store(y, thread_index, 2)
    return built(k)


def count(caps):
    k = KernelBuilder("count", caps)
    n = k.dim("n", D(1, 1024))
    y = k.buffer("y", RW, U32, n)
    k.threads(64)
    k.groups(1)
    with k.strided("i", n) as i:
        k.store(y, i, k.load(y, i) + 1)
    return built(k)


def total(caps):
    k = KernelBuilder("total", caps)
    y = k.buffer("y", W, U32, 1)
    k.threads(64)
    k.groups(1)
    partial = k.tg_array("partial", U32, 8)
    s = k.simd_sum("s", thread_index)
    with k.when_lane(simd_lane.eq(0)):
        k.tg_store(partial, simd_group_index, s)
    k.barrier()
    groups = k.simd_group_count()
    with k.when_lane(thread_index.eq(0)):
        acc = k.var("acc", u32(0))
        with k.for_u("g", 0, groups) as g:
            k.assign(acc, acc.get + k.tg_load(partial, g))
        k.store(y, 0, acc.get)
    return built(k)


def pick(caps):
    k = KernelBuilder("pick", caps)
    entry = k.param("entry", U32)
    arrays = k.table("arrays", F32, 3, 4)
    y = k.buffer("y", W, F32, 6)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index < 4):
        k.store(y, thread_index, k.load_via(arrays, entry, thread_index))
    pair = k.load_pack_via("pair", 2, arrays, entry, 1)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 4, pair[0])
        k.store(y, 5, pair[1])
    return built(k)


def _ordered_sums(caps, name, f32_big, f16_big, ones):
    k = KernelBuilder(name, caps)
    n = at_least(caps, 32)
    y = k.buffer("y", W, F32, n)
    h = k.buffer("h", W, F16, n)
    k.threads(n)
    k.groups(1)
    s = k.simd_sum("s", select(simd_lane.eq(0), f32(f32_big), ones(F32)))
    k.store(y, thread_index, s)
    t = k.simd_sum("t", select(simd_lane.eq(0), lit(F16, f16_big), ones(F16)))
    k.store(h, thread_index, t)
    return built(k)


def pairwise(caps):
    """2^24 (2048 in f16) at lane 0, ones elsewhere (InterpTest.hs:467-477)."""
    return _ordered_sums(caps, "pairwise", 16777216.0, 2048, lambda t: lit(t, 1))


def neighbours(caps):
    """2^24 at lane 0, ones at lanes 16 and 17 (InterpTest.hs:479-490)."""
    def ones(t):
        return select(simd_lane.eq(16) | simd_lane.eq(17), lit(t, 1), lit(t, 0))
    return _ordered_sums(caps, "neighbours", 16777216.0, 2048, ones)


def fmas(caps):
    k = KernelBuilder("fmas", caps)
    n = k.dim("n", D(1, 64))
    m = k.dim("m", D(1, 64))
    a, b, c = (k.buffer(x, R, F32, n) for x in "abc")
    ah, bh, ch = (k.buffer(x, R, F16, m) for x in ("ah", "bh", "ch"))
    y = k.buffer("y", W, F32, n)
    g = k.buffer("g", W, F16, m)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.strided("i", n) as i:
        k.store(y, i, fma_e(k.load(a, i), k.load(b, i), k.load(c, i)))
    with k.strided("j", m) as j:
        k.store(g, j, fma_e(k.load(ah, j), k.load(bh, j), k.load(ch, j)))
    return built(k)


def transcendentals(caps):
    k = KernelBuilder("transcendentals", caps)
    n = k.dim("n", D(1, 65536))
    m = k.dim("m", D(1, 65536))
    x = k.buffer("x", R, F32, n)
    h = k.buffer("h", R, F16, m)
    y = k.buffer("y", W, F32, n * 4)
    g = k.buffer("g", W, F16, m * 4)
    k.threads(256)
    k.groups(1)
    for name, src, dst, count in (("i", x, y, n), ("j", h, g, m)):
        with k.strided(name, count) as i:
            a = k.let("a" if name == "i" else "b", k.load(src, i))
            k.store(dst, i * 4, rsqrt_e(a))
            k.store(dst, i * 4 + 1, exp_e(a))
            k.store(dst, i * 4 + 2, log_e(a))
            k.store(dst, i * 4 + 3, tanh_e(a))
    return built(k)


def narrowings(caps, n: int = 4):
    """InterpTest.hs:580-593 (4 elements) and Cases.hs's (16)."""
    k = KernelBuilder("narrowings", caps)
    a = k.buffer("a", R, I32, n)
    b = k.buffer("b", R, U32, n)
    ca = k.buffer("clamped_a", W, I8, n)
    wa = k.buffer("wrapped_a", W, I8, n)
    cb = k.buffer("clamped_b", W, U8, n)
    wb = k.buffer("wrapped_b", W, U8, n)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index < n):
        k.store(ca, thread_index, narrow_clamped(I8, k.load(a, thread_index)))
        k.store(wa, thread_index, narrow_wrapped(I8, k.load(a, thread_index)))
        k.store(cb, thread_index, narrow_clamped(U8, k.load(b, thread_index)))
        k.store(wb, thread_index, narrow_wrapped(U8, k.load(b, thread_index)))
    return built(k)


def int32s(caps):
    k = KernelBuilder("int32s", caps)
    a = k.param("a", I32)
    b = k.param("b", I32)
    y = k.buffer("y", W, I32, 5)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 0, a + b)
        k.store(y, 1, a - b)
        k.store(y, 2, a * b)
        k.store(y, 3, -a)
        k.store(y, 4, abs(a))
    return built(k)


def int32_quotient(caps):
    k = KernelBuilder("int32_quotient", caps)
    a = k.param("a", I32)
    b = k.param("b", I32)
    y = k.buffer("y", W, I32, 2)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 0, quot(a, b))
        k.store(y, 1, rem(a, b))
    return built(k)


def floats(caps):
    k = KernelBuilder("floats", caps)
    n = k.dim("n", D(1, 64))
    x = k.buffer("x", R, F32, n)
    y = k.buffer("y", R, F32, n)
    h = k.buffer("h", R, F16, n)
    g = k.buffer("g", R, F16, n)
    out = k.buffer("out", W, F32, n * 4)
    out_h = k.buffer("out_h", W, F16, n * 4)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.strided("i", n) as i:
        a = k.let("a", k.load(x, i))
        b = k.let("b", k.load(y, i))
        k.store(out, i * 4, min_e(a, b))
        k.store(out, i * 4 + 1, max_e(a, b))
        k.store(out, i * 4 + 2, -a)
        k.store(out, i * 4 + 3, abs(a))
        c = k.let("c", k.load(h, i))
        d = k.let("d", k.load(g, i))
        k.store(out_h, i * 4, min_e(c, d))
        k.store(out_h, i * 4 + 1, max_e(c, d))
        k.store(out_h, i * 4 + 2, -c)
        k.store(out_h, i * 4 + 3, abs(c))
    return built(k)


def from_by(caps):
    k = KernelBuilder("from_by", caps)
    start = k.param("start", U32)
    step = k.param("step", U32)
    y = k.buffer("y", W, U32, 1)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index.eq(0)):
        n = k.var("n", u32(0))
        with k.for_step("i", start, 4294967295, step):
            k.assign(n, n.get + 1)
        k.store(y, 0, n.get)
    return built(k)


def eights(caps):
    k = KernelBuilder("eights", caps)
    n = k.dim("n", D(8, 64, 8))
    y = k.buffer("y", W, U32, 64)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.strided("i", n) as i:
        k.store(y, i, i)
    return built(k)


def through_table(caps):
    k = KernelBuilder("through_table", caps)
    e = k.param("e", U32)
    i = k.param("i", U32)
    arrays = k.table("arrays", F32, 3, 4)
    y = k.buffer("y", W, F32, 1)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 0, k.load_via(arrays, e, i))
    return built(k)


def uninitialised(caps):
    k = KernelBuilder("uninitialised", caps)
    y = k.buffer("y", W, U32, 1)
    k.threads(at_least(caps, 32))
    k.groups(1)
    t = k.tg_array("t", U32, 2)
    with k.when_lane(thread_index.eq(0)):
        k.tg_store(t, 0, 7)
    k.barrier()
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 0, k.tg_load(t, 1))
    return built(k)


def divide(caps):
    k = KernelBuilder("divide", caps)
    d = k.param("d", U32)
    y = k.buffer("y", W, U32, 1)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 0, quot(u32(1), d))
    return built(k)


def past_end(caps):
    k = KernelBuilder("past_end", caps)
    x = k.buffer("x", R, F32, 4)
    y = k.buffer("y", W, F32, 1)
    k.threads(at_least(caps, 32))
    k.groups(1)
    v = k.load_pack("v", 4, x, 1)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 0, ((f32(0.0) + v[0] + v[1]) + v[2]) + v[3])
    return built(k)


def grid_less(caps):
    k = KernelBuilder("grid_less", caps)
    n = k.dim("n", D(0, 16))
    y = k.buffer("y", W, U32, 1)
    k.threads(at_least(caps, 32))
    k.groups(n - 1)
    with k.when_lane(thread_index.eq(0) & group_index.eq(0)):
        k.store(y, 0, 1)
    return built(k)


# ---------------------------------------------------------------------------
# test/cpu/Cases.hs

def sum_rows(caps):
    k = KernelBuilder("sum_rows", caps)
    n = k.dim("n", D(1, 16))
    x = k.buffer("x", R, F32, n * 64)
    y = k.buffer("y", W, F32, n)
    rows = k.table("rows", F32, n, 64)
    k.threads(at_least(caps, 32))
    k.groups(n)
    acc = k.var("acc", f32(0.0))
    with k.strided("i", 64) as i:
        k.assign(acc, acc.get + k.load(x, group_index * 64 + i) * k.load_via(rows, group_index, i))
    tot = k.simd_sum("total", acc.get)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, group_index, tot)
    return built(k)


def gemm(caps, t: str, name: str = "gemm"):
    """C = A · Bᵀ in 8×8 fragments, B's tiles loaded transposed."""
    k = KernelBuilder(name, caps)
    kd = k.dim("k", D(8, 256, 8))
    a = k.buffer("a", R, t, kd * 16)
    b = k.buffer("b", R, t, kd * 16)
    c = k.buffer("c", W, F32, 256)
    k.threads(4 * caps.simd_width)
    k.groups(1)
    row0 = k.let("row0", quot(simd_group_index, 2) * 8)
    col0 = k.let("col0", rem(simd_group_index, 2) * 8)
    acc = k.fragment("acc", F32)
    fa = k.fragment("fa", t)
    fb = k.fragment("fb", t)
    with k.for_u("p", 0, quot(kd, 8)) as p:
        k.frag_load(fa, a, row0 * kd + p * 8, kd)
        k.frag_load_t(fb, b, col0 * kd + p * 8, kd)
        k.frag_mma(acc, fa, fb, acc)
    k.frag_store(c, row0 * 16 + col0, 16, acc)
    return built(k)


def gemm_via(caps):
    k = KernelBuilder("gemm_via", caps)
    kd = k.dim("k", D(8, 256, 8))
    ab = k.table("ab", BF16, 3, kd * 16)
    cs = k.table("cs", F32, 2, 256, access=W)
    k.distinct(cs)
    k.threads(4 * caps.simd_width)
    k.groups(1)
    row0 = k.let("row0", quot(simd_group_index, 2) * 8)
    col0 = k.let("col0", rem(simd_group_index, 2) * 8)
    acc = k.fragment("acc", F32)
    fa = k.fragment("fa", BF16)
    fb = k.fragment("fb", BF16)
    with k.for_u("p", 0, quot(kd, 8)) as p:
        k.frag_load_via(fa, ab, 1, row0 * kd + p * 8, kd)
        k.frag_load_via_t(fb, ab, 2, col0 * kd + p * 8, kd)
        k.frag_mma(acc, fa, fb, acc)
    k.frag_store_via(cs, 1, row0 * 16 + col0, 16, acc)
    return built(k)


def staged(caps):
    k = KernelBuilder("staged", caps)
    kd = k.dim("k", D(8, 256, 8))
    a = k.buffer("a", R, BF16, kd * 16)
    b = k.buffer("b", R, BF16, kd * 16)
    c = k.buffer("c", W, F32, 256)
    threads = 4 * caps.simd_width
    k.threads(threads)
    k.groups(1)
    tile = k.tg_array("tile", BF16, 128)
    row0 = k.let("row0", quot(simd_group_index, 2) * 8)
    col0 = k.let("col0", rem(simd_group_index, 2) * 8)
    acc = k.fragment("acc", F32)
    fa = k.fragment("fa", BF16)
    fb = k.fragment("fb", BF16)
    with k.for_u("p", 0, quot(kd, 8)) as p:
        with k.when_lane(thread_index < 128):
            k.tg_store(tile, thread_index, k.load(b, quot(thread_index, 8) * kd + p * 8 + rem(thread_index, 8)))
        k.barrier()
        k.frag_load(fa, a, row0 * kd + p * 8, kd)
        k.frag_load_tg_t(fb, tile, col0 * 8, 8)
        k.frag_mma(acc, fa, fb, acc)
        k.barrier()
    k.frag_store(c, row0 * 16 + col0, 16, acc)
    return built(k)


def scaled_rows(caps):
    k = KernelBuilder("scaled_rows", caps)
    kd = k.dim("k", D(8, 256, 8))
    a = k.buffer("a", R, F32, kd * 16)
    b = k.buffer("b", R, BF16, kd * 16)
    c = k.buffer("c", W, F32, 256)
    k.threads(4 * caps.simd_width)
    k.groups(1)
    scales = k.tg_array("scales", F32, 8)
    for r in range(8):
        with k.when_lane(thread_index.eq(0)):
            k.tg_store(scales, r, lit(F32, 2 ** r) * 0.3)
    k.barrier()
    row0 = k.let("row0", quot(simd_group_index, 2) * 8)
    col0 = k.let("col0", rem(simd_group_index, 2) * 8)
    acc = k.fragment("acc", F32)
    fa = k.fragment("fa", F32)
    fbh = k.fragment("fbh", BF16)
    fb = k.fragment("fb", F32)
    with k.for_u("p", 0, quot(kd, 8)) as p:
        k.frag_load(fa, a, row0 * kd + p * 8, kd)
        k.frag_load_t(fbh, b, col0 * kd + p * 8, kd)
        k.frag_convert(fb, fbh)
        k.frag_mma(acc, fa, fb, acc)
    k.frag_scale_rows(acc, scales, 0)
    k.frag_store(c, row0 * 16 + col0, 16, acc)
    return built(k)


def tiled(caps, t: GemmTile, na: int, nb: int, nc: int, name: str = "tiled"):
    k = KernelBuilder(name, caps)
    m = k.dim("m", D(1, 256))
    n = k.dim("n", D(8, 256, 8))
    kd = k.dim("k", D(t.step, 256, t.step))
    a = k.buffer("a", R, BF16, m * kd)
    b = k.buffer("b", R, BF16, n * kd)
    c = k.buffer("c", W, F32, m * n)
    k.threads(256)
    k.groups(quot(m + t.rows - 1, t.rows) * quot(n + t.cols - 1, t.cols))
    a_slice = k.tg_array("a_slice", F32, na)
    b_slice = k.tg_array("b_slice", F32, nb)
    c_tile = k.tg_array("c_tile", F32, nc)
    tiles_n = k.let("tiles_n", quot(n + t.cols - 1, t.cols))
    row0 = k.let("row0", quot(group_index, tiles_n) * t.rows)
    col0 = k.let("col0", rem(group_index, tiles_n) * t.cols)

    def a_run(r, p):
        return [widen(F32, k.load(a, min_e(row0 + r, m - 1) * kd + p + x)) for x in range(4)]

    def b_run(col, p):
        return [widen(F32, k.load(b, min_e(col0 + col, n - 1) * kd + p + x)) for x in range(8)]

    def element(r, col, v):
        with k.when_lane((row0 + r < m) & (col0 + col < n)):
            k.store(c, (row0 + r) * n + col0 + col, v)

    gemm_tile(k, "t", t, a_slice, b_slice, c_tile, kd, a_run, b_run, element)
    return built(k)


def _binary_case(caps, name, t, outs):
    k = KernelBuilder(name, caps)
    n = k.dim("n", D(1, 100000))
    x = k.buffer("x", R, t, n)
    y = k.buffer("y", R, t, n)
    bufs = {o: k.buffer(o, W, ot, n) for o, ot in outs}
    k.threads(64)
    k.groups(1)
    return k, n, x, y, bufs


def _cmp_bits(a, b):
    one = lambda v: u32(v)  # noqa: E731
    return (select(a < b, one(1), one(0)) + select(a <= b, one(2), one(0)) + select(a > b, one(4), one(0))
            + select(a >= b, one(8), one(0)) + select(a.eq(b), one(16), one(0)) + select(a.ne(b), one(32), one(0)))


def arith_f32(caps):
    names = ["o_add", "o_sub", "o_mul", "o_div", "o_min", "o_max", "o_sqrt", "o_rsqrt", "o_exp", "o_log", "o_tanh",
             "o_abs", "o_neg"]
    outs = [(o, F32) for o in names] + [("o_cmp", U32), ("o_bf", BF16), ("o_h", F16), ("o_sel", F32)]
    k, n, x, y, o = _binary_case(caps, "arith_f32", F32, outs)
    with k.strided("i", n) as i:
        a = k.let("a", k.load(x, i))
        b = k.let("b", k.load(y, i))
        for name, v in (("o_add", a + b), ("o_sub", a - b), ("o_mul", a * b), ("o_div", a / b),
                        ("o_min", min_e(a, b)), ("o_max", max_e(a, b)), ("o_sqrt", sqrt_e(a)),
                        ("o_rsqrt", rsqrt_e(a)), ("o_exp", exp_e(a)), ("o_log", log_e(a)), ("o_tanh", tanh_e(a)),
                        ("o_abs", abs(a)), ("o_neg", -a), ("o_cmp", _cmp_bits(a, b)), ("o_bf", narrow(BF16, a)),
                        ("o_h", narrow(F16, a)), ("o_sel", select(a < b, a, b))):
            k.store(o[name], i, v)
    return built(k)


def arith_f16(caps):
    names = ["o_add", "o_sub", "o_mul", "o_div", "o_min", "o_max", "o_sqrt", "o_rsqrt", "o_exp", "o_log", "o_tanh",
             "o_abs", "o_neg"]
    outs = [(o, F16) for o in names] + [("o_cmp", U32), ("o_wide", F32), ("o_lit", F16)]
    k, n, x, y, o = _binary_case(caps, "arith_f16", F16, outs)
    with k.strided("i", n) as i:
        a = k.let("a", k.load(x, i))
        b = k.let("b", k.load(y, i))
        for name, v in (("o_add", a + b), ("o_sub", a - b), ("o_mul", a * b), ("o_div", a / b),
                        ("o_min", min_e(a, b)), ("o_max", max_e(a, b)), ("o_sqrt", sqrt_e(a)),
                        ("o_rsqrt", rsqrt_e(a)), ("o_exp", exp_e(a)), ("o_log", log_e(a)), ("o_tanh", tanh_e(a)),
                        ("o_abs", abs(a)), ("o_neg", -a), ("o_cmp", _cmp_bits(a, b)), ("o_wide", widen(F32, a)),
                        ("o_lit", a * 0.1 + (-lit(F16, 3)))):
            k.store(o[name], i, v)
    return built(k)


def arith_int(caps):
    k = KernelBuilder("arith_int", caps)
    n = k.dim("n", D(1, 100000))
    xi, yi = k.buffer("xi", R, I32, n), k.buffer("yi", R, I32, n)
    xu, yu = k.buffer("xu", R, U32, n), k.buffer("yu", R, U32, n)
    names_i = ["i_add", "i_sub", "i_mul", "i_neg", "i_abs", "i_min", "i_max", "i_div", "i_rem"]
    o = {nm: k.buffer(nm, W, I32, n) for nm in names_i}
    o["i_cmp"] = k.buffer("i_cmp", W, U32, n)
    for nm in ["u_add", "u_sub", "u_mul", "u_neg", "u_div", "u_rem", "u_min", "u_cmp"]:
        o[nm] = k.buffer(nm, W, U32, n)
    o["u_tof"] = k.buffer("u_tof", W, F32, n)
    o["i_lit"] = k.buffer("i_lit", W, I32, n)
    k.threads(64)
    k.groups(1)
    with k.strided("i", n) as i:
        a = k.let("a", k.load(xi, i))
        b = k.let("b", k.load(yi, i))
        p = k.let("p", k.load(xu, i))
        q = k.let("q", k.load(yu, i))
        k.store(o["i_add"], i, a + b)
        k.store(o["i_sub"], i, a - b)
        k.store(o["i_mul"], i, a * b)
        k.store(o["i_neg"], i, -a)
        k.store(o["i_abs"], i, abs(a))
        k.store(o["i_min"], i, min_e(a, b))
        k.store(o["i_max"], i, max_e(a, b))
        d = k.let("d", select(b.eq(0) | (b.eq(-lit(I32, 1)) & a.eq(-lit(I32, 2147483647) - 1)), lit(I32, 7), b))
        k.store(o["i_div"], i, quot(a, d))
        k.store(o["i_rem"], i, rem(a, d))
        k.store(o["i_cmp"], i, _cmp_bits(a, b))
        k.store(o["u_add"], i, p + q)
        k.store(o["u_sub"], i, p - q)
        k.store(o["u_mul"], i, p * q)
        k.store(o["u_neg"], i, -p)
        e = k.let("e", select(q.eq(0), u32(3), q))
        k.store(o["u_div"], i, quot(p, e))
        k.store(o["u_rem"], i, rem(p, e))
        k.store(o["u_min"], i, min_e(p, q) + max_e(p, q) * 3)
        k.store(o["u_cmp"], i, _cmp_bits(p, q))
        k.store(o["u_tof"], i, to_f32(p))
        # Haskell's -n is negate (fromInteger n): a negation in the IR.
        negated = k.let("negated", -(-lit(I32, 2147483647)))
        k.store(o["i_lit"], i, (a * (-lit(I32, 2147483647) - 1)) + (-lit(I32, 1)) - abs(-lit(I32, 5)) + negated)
    return built(k)


def conv(caps):
    k = KernelBuilder("conv", caps)
    n = k.dim("n", D(1, 100000))
    xb, xh = k.buffer("xb", R, BF16, n), k.buffer("xh", R, F16, n)
    xs, xc = k.buffer("xs", R, I8, n), k.buffer("xc", R, U8, n)
    o = {nm: k.buffer(nm, W, t, n) for nm, t in (("o_b", F32), ("o_h", F32), ("o_s", I32), ("o_c", U32),
                                                ("o_rb", BF16), ("o_rh", F16), ("o_pb", BF16))}
    k.threads(64)
    k.groups(1)
    with k.strided("i", n) as i:
        k.store(o["o_b"], i, widen(F32, k.load(xb, i)))
        k.store(o["o_h"], i, widen(F32, k.load(xh, i)))
        k.store(o["o_s"], i, widen(I32, k.load(xs, i)))
        k.store(o["o_c"], i, widen(U32, k.load(xc, i)))
        k.store(o["o_rb"], i, narrow(BF16, widen(F32, k.load(xb, i))))
        k.store(o["o_rh"], i, narrow(F16, widen(F32, k.load(xh, i))))
        k.store(o["o_pb"], i, k.load(xb, i))
    return built(k)


def flow(caps):
    """Divergent loops, SIMD-uniform branches, reductions, threadgroup memory
    (Cases.hs:424-454); 96 threads there, three 32-lane groups: here the
    threads are three SIMD groups of the target."""
    w = caps.simd_width
    threads = 3 * w
    k = KernelBuilder("flow", caps)
    n = k.dim("n", D(1, 4096))
    x = k.buffer("x", R, F32, n)
    cnt = k.buffer("cnt", R, U32, 3 * threads)
    y = k.buffer("y", W, F32, 3 * threads)
    z = k.buffer("z", W, F32, 3 * threads)
    wv = k.buffer("w", W, U32, 3 * threads)
    k.threads(threads)
    k.groups(3)
    tg = k.tg_array("tg", F32, threads)
    g = k.let("g", group_index * threads + thread_index)
    acc = k.var("acc", f32(0.0))
    hits = k.var("hits", u32(0))
    with k.for_step("j", rem(simd_lane, 3), k.load(cnt, g), 2) as j:
        k.assign(acc, acc.get + k.load(x, rem(j, n)))
        with k.when_lane(j.eq(4)):
            k.assign(acc, acc.get * 1.5)
            k.assign(hits, hits.get + 1)
    s = k.simd_sum("s", acc.get)
    mx = k.simd_max("mx", acc.get)
    hs = k.simd_sum("hs", hits.get)
    with k.when_simd(simd_group_index.eq(1)):
        t = k.simd_sum("t", acc.get * 3)
        with k.when_lane(simd_lane < 5):
            k.store(z, g, t)
    k.tg_store(tg, thread_index, s + mx)
    k.barrier()
    k.store(y, g, k.tg_load(tg, rem(thread_index + 1, threads)))
    k.store(wv, g, hs)
    k.barrier()
    tot = tg_reduce_sum(k, "total", tg, acc.get)
    with k.when_lane(thread_index.eq(0)):
        k.store(z, group_index * threads + threads - 1, tot)
    return built(k)


def simd_sums(caps):
    n = caps.simd_width * max(1, 64 // caps.simd_width)
    k = KernelBuilder("simd_sums", caps)
    x = k.buffer("x", R, F32, n)
    h = k.buffer("h", R, F16, n)
    y = k.buffer("y", W, F32, n)
    g = k.buffer("g", W, F16, n)
    k.threads(n)
    k.groups(1)
    s = k.simd_sum("s", k.load(x, thread_index))
    k.store(y, thread_index, s)
    t = k.simd_sum("t", k.load(h, thread_index))
    k.store(g, thread_index, t)
    return built(k)


def fma_case(caps, t: str):
    k = KernelBuilder("fma_" + t, caps)
    n = k.dim("n", D(1, 100000))
    a, b, c = (k.buffer(x, R, t, n) for x in "abc")
    o = k.buffer("o_fma", W, t, n)
    k.threads(64)
    k.groups(1)
    with k.strided("i", n) as i:
        k.store(o, i, fma_e(k.load(a, i), k.load(b, i), k.load(c, i)))
    return built(k)


def reductions(caps):
    k = KernelBuilder("reductions", caps)
    x = k.buffer("x", R, F32, 256)
    y = k.buffer("y", W, F32, 256)
    z = k.buffer("z", W, F32, 4)
    k.threads(64)
    k.groups(4)
    scratch = k.tg_array("scratch", F32, max(2, 64 // caps.simd_width))
    g = k.let("g", group_index * 64 + thread_index)
    v = k.let("v", k.load(x, g))
    m = k.simd_max("m", v)
    k.store(y, g, m)
    t = tg_reduce_max(k, "t", scratch, v)
    with k.when_lane(thread_index.eq(0)):
        k.store(z, group_index, t)
    return built(k)


def params(caps):
    k = KernelBuilder("params", caps)
    n = k.dim("n", D(1, 64))
    a = k.param("a", BOOL)
    b = k.param("b", F32)
    c = k.param("c", F16)
    d = k.param("d", I32)
    e = k.param("e", BF16)
    f = k.param("f", U8)
    g = k.param("g", I8)
    y = k.buffer("y", W, F32, n)
    yh = k.buffer("yh", W, F16, n)
    yi = k.buffer("yi", W, I32, n)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.when_lane(thread_index.eq(0)):
        k.store(y, 0, select(a, b, widen(F32, e)))
        k.store(y, 1, widen(F32, e) + to_f32(widen(U32, f)))
        k.store(yh, 0, (-c) * (-lit(F16, 2.5)) + 65504)
        k.store(yi, 0, d + widen(I32, g))
    return built(k)


def ranged(caps):
    k = KernelBuilder("ranged", caps)
    n = k.dim("n", D(8, 64, 8))
    y = k.buffer("y", W, F32, 64)
    k.threads(at_least(caps, 32))
    k.groups(1)
    with k.strided("i", n) as i:
        k.store(y, i, 1.0)
    return built(k)
