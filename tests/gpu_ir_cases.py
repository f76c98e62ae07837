"""The IR target's cases: test/cpu/Cases.hs's kernels and inputs (the CPU
target's checks), and InterpTest.hs's known-answer kernels, built for the
MI355X (64-lane SIMD groups).  The GPU tests run each case's kernel, lowered
to HIP and compiled by hipRTC, on the same inputs as the oracle's interpreter
and compare every output bit for bit; an output of arithmetic that is a NaN
is compared by class only (quiet or signalling), as Cases.hs:12-19 compares
the CPU target's.

The inputs are Cases.hs's: SplitMix's finaliser over a seed's sequence
(Cases.hs:1076-1086), values in [-2, 2) multiples of 2^-22, the special
values of each type and their pairs.  Where the reference's kernel is written
for 32-lane groups (thread counts, the GEMV variants' threads, flow's groups),
the MI355X's is the same kernel on 64-lane groups, its buffers sized to it.
"""

from __future__ import annotations

import functools
import math
from dataclasses import dataclass

import numpy as np

import ir_kernels as K
from furykernel_amd.ir import rocm
from furykernel_amd.ir.build import ROCM
from furykernel_amd.ir.gate import check
from furykernel_amd.program.graph import BF16, F16, F32
from oracle import interp

M64 = (1 << 64) - 1


def mix(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def randoms(seed: int, n: int) -> list:
    return [mix((seed * 0x9E3779B97F4A7C15 + i) & M64) for i in range(1, n + 1)]


def floats(seed: int, n: int) -> np.ndarray:
    return np.array([((w >> 40) - 2 ** 23) / 2 ** 22 for w in randoms(seed, n)], np.float32)


def f32s(seed, n):
    return floats(seed, n)


def bf16s(seed, n):
    return interp.narrow_bf16(floats(seed, n))


def f16s(seed, n):
    return interp.narrow_f16(floats(seed, n))


def zeros(n):
    return np.zeros(n, np.float32)


F32_SPECIALS = [0x00000000, 0x80000000, 0x3F800000, 0xBF800000, 0x3F000000, 0x40000000, 0x40400000, 0x00000001,
                0x007FFFFF, 0x00800000, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7FC00001, 0xFFC00000,
                0x7F800001, 0x7FA00000, 0xFF800001, 0x477FE000, 0x477FF000, 0x477FEFFF, 0x387FC000, 0x38800000,
                0x33800000, 0x33000000, 0x33000001, 0x3F808000, 0x3F818000, 0x3F808001, 0x7F7F8000, 0x3EAAAAAB,
                0x40490FDB, 0xC2C80000, 0x42C80000, 0x3F801000, 0x3F803000, 0xC1200000, 0x41200000, 0x3DCCCCCD]
F16_SPECIALS = [0x0000, 0x8000, 0x3C00, 0xBC00, 0x3800, 0x4000, 0x4200, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF,
                0x7C00, 0xFC00, 0x7E00, 0x7E01, 0xFE00, 0x7C01, 0x7D00, 0x3555, 0x4248, 0x5640, 0x1400, 0x0200,
                0x3C01, 0x7800, 0x5BFF, 0xC900]
I32_SPECIALS = [0, 1, -1, 2, -2, -2 ** 31, 2 ** 31 - 1, 7, -7, 3, 65536, -65536, 46341, -46341, 1000000007]
U32_SPECIALS = [0, 1, 2, 3, 0xFFFFFFFF, 0x80000000, 0x7FFFFFFF, 65536, 16777216, 16777217, 16777218, 16777219,
                33554433, 33554434, 33554435, 33554438, 0xFFFFFF80, 0xFFFFFF7F, 0xFFFFFF81, 0x7FFFFFC0, 0x7FFFFFBF]
BY_CLASS = ["o_add", "o_sub", "o_mul", "o_div", "o_min", "o_max", "o_sqrt", "o_rsqrt", "o_exp", "o_log", "o_tanh"]


def pairs(xs):
    return [(a, b) for a in xs for b in xs]


def as_i32(w):
    return np.array(w, np.uint32).view(np.int32)


@dataclass
class Case:
    id: str
    kernel: object
    runs: list  # (params, buffers, tables)
    by_class: tuple = ()
    transcendental: tuple = ()  # outputs the target computes within its stated bound, not bits


def _arith_f32():
    ps = pairs(F32_SPECIALS) + [(w & 0xFFFFFFFF, w >> 32) for w in randoms(50, 2000)]
    n = len(ps)
    x = np.array([a for a, _ in ps], np.uint32).view(np.float32)
    y = np.array([b for _, b in ps], np.uint32).view(np.float32)
    bufs = {"x": x, "y": y, "o_cmp": np.zeros(n, np.uint32), "o_bf": np.zeros(n, np.uint16),
            "o_h": np.zeros(n, np.uint16)}
    for o in BY_CLASS + ["o_abs", "o_neg", "o_sel"]:
        bufs[o] = zeros(n)
    return Case("arith_f32", K.arith_f32(ROCM), [({"n": n}, bufs, {})], tuple(BY_CLASS),
                ("o_rsqrt", "o_exp", "o_log", "o_tanh"))


def _arith_f16():
    ps = pairs(F16_SPECIALS) + [(w & 0xFFFF, (w >> 16) & 0xFFFF) for w in randoms(51, 3000)]
    n = len(ps)
    bufs = {"x": np.array([a for a, _ in ps], np.uint16), "y": np.array([b for _, b in ps], np.uint16),
            "o_cmp": np.zeros(n, np.uint32), "o_wide": zeros(n)}
    for o in BY_CLASS + ["o_abs", "o_neg", "o_lit"]:
        bufs[o] = np.zeros(n, np.uint16)
    return Case("arith_f16", K.arith_f16(ROCM), [({"n": n}, bufs, {})], tuple(["o_lit"] + BY_CLASS),
                ("o_rsqrt", "o_exp", "o_log", "o_tanh"))


def _arith_int():
    is_ = pairs(I32_SPECIALS) + [(((w & 0xFFFFFFFF) ^ 0x80000000) - 0x80000000,
                                  (((w >> 32) & 0xFFFFFFFF) ^ 0x80000000) - 0x80000000) for w in randoms(52, 500)]
    us_src = pairs(U32_SPECIALS) + [(w & 0xFFFFFFFF, (w >> 40) & 0xFFFFFFFF) for w in randoms(53, 500)]
    n = len(is_)
    us = [us_src[i % len(us_src)] for i in range(n)]
    bufs = {"xi": np.array([a for a, _ in is_], np.int32), "yi": np.array([b for _, b in is_], np.int32),
            "xu": np.array([a for a, _ in us], np.uint32), "yu": np.array([b for _, b in us], np.uint32)}
    for o in ["i_add", "i_sub", "i_mul", "i_neg", "i_abs", "i_min", "i_max", "i_div", "i_rem", "i_lit"]:
        bufs[o] = np.zeros(n, np.int32)
    for o in ["i_cmp", "u_add", "u_sub", "u_mul", "u_neg", "u_div", "u_rem", "u_min", "u_cmp"]:
        bufs[o] = np.zeros(n, np.uint32)
    bufs["u_tof"] = zeros(n)
    return Case("arith_int", K.arith_int(ROCM), [({"n": n}, bufs, {})])


def _conv():
    bs = [w & 0xFFFF for w in randoms(54, 4000)] + [0x7F81, 0xFF81, 0x7FC0, 0x7FFF, 0x7F80, 0x0001, 0x8000, 0x0000,
                                                    0xFFC1]
    n = len(bs)
    hsrc = F16_SPECIALS + [w & 0xFFFF for w in randoms(55, 3000)]
    bufs = {"xb": np.array(bs, np.uint16), "xh": np.array([hsrc[i % len(hsrc)] for i in range(n)], np.uint16),
            "xs": np.array([(i % 256) - 256 * ((i % 256) > 127) for i in range(n)], np.int8),
            "xc": np.array([i % 256 for i in range(n)], np.uint8), "o_b": zeros(n), "o_h": zeros(n),
            "o_s": np.zeros(n, np.int32), "o_c": np.zeros(n, np.uint32), "o_rb": np.zeros(n, np.uint16),
            "o_rh": np.zeros(n, np.uint16), "o_pb": np.zeros(n, np.uint16)}
    return Case("conv", K.conv(ROCM), [({"n": n}, bufs, {})])


def _fma_f32():
    addends = [0x00000000, 0x80000000, 0x3F800000, 0xBF800000, 0x00000001, 0x80000001, 0x00800000, 0x7F7FFFFF,
               0xFF7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000, 0x28800000, 0x33800000]
    edge = [(a, b, c) for a in F32_SPECIALS for b in F32_SPECIALS for c in addends]
    rand = [(w & 0xFFFFFFFF, w >> 32, v & 0xFFFFFFFF) for w, v in zip(randoms(56, 3000), randoms(57, 3000))]
    xs, ys = floats(58, 3000), floats(59, 3000)
    with np.errstate(all="ignore"):
        errs = [(int(a), int(b), int(c)) for a, b, c in zip(xs.view(np.uint32), ys.view(np.uint32),
                                                             (-(xs * ys)).astype(np.float32).view(np.uint32))]
    ties = [(0x3F800001, 0x3F7FFFFF, 0x28800000), (0x3F800001, 0x3F7FFFFF, 0xA8800000),
            (0x3F800001, 0x3F800001, 0xBF800002), (0x3F800800, 0x3F800800, 0xBF801000),
            (0x7F7FFFFF, 0x40000000, 0xFF7FFFFF), (0x1A000000, 0x1A400000, 0x00000000),
            (0x9A000000, 0x19800000, 0x00000000), (0x1A000000, 0x1A000000, 0x00000000)]
    t = edge + rand + errs + ties
    n = len(t)
    bufs = {k: np.array([x[i] for x in t], np.uint32).view(np.float32) for i, k in enumerate("abc")}
    bufs["o_fma"] = zeros(n)
    return Case("fma_f32", K.fma_case(ROCM, F32), [({"n": n}, bufs, {})], ("o_fma",))


def _fma_f16():
    addends = [0x0000, 0x8000, 0x3C00, 0xBC00, 0x0001, 0x8001, 0x0400, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00,
               0x1400, 0x3C02]
    edge = [(a, b, c) for a in F16_SPECIALS for b in F16_SPECIALS for c in addends]
    rand = [(w & 0xFFFF, (w >> 16) & 0xFFFF, (w >> 32) & 0xFFFF) for w in randoms(60, 6000)]
    xs, ys = interp.narrow_f16(floats(61, 3000)), interp.narrow_f16(floats(62, 3000))
    with np.errstate(all="ignore"):
        prod = interp.narrow_f16(interp.widen_f16(xs) * interp.widen_f16(ys))
    errs = [(int(a), int(b), int(c)) for a, b, c in zip(xs, ys, prod ^ np.uint16(0x8000))]
    ties = [(0x2740, 0x246A, 0x3C00), (0x2740, 0x246A, 0xBC00), (0x5BF8, 0x5C04, 0x0000), (0x5BF8, 0x5C04, 0xCC00),
            (0x3C01, 0x3C01, 0xBC02), (0x0C00, 0x0800, 0x0000), (0x0C00, 0x0A00, 0x0000), (0x8C00, 0x0400, 0x0000)]
    t = edge + rand + errs + ties
    n = len(t)
    bufs = {k: np.array([x[i] for x in t], np.uint16) for i, k in enumerate("abc")}
    bufs["o_fma"] = np.zeros(n, np.uint16)
    return Case("fma_f16", K.fma_case(ROCM, F16), [({"n": n}, bufs, {})], ("o_fma",))


def _simd_sums():
    xs = [16777216.0 if l == 0 else 1.0 for l in range(32)] + [math.ldexp(1 + l, l % 41 - 20) * (1 if l % 2 == 0 else -1)
                                                               for l in range(32)]
    hs = [2048.0 if l == 0 else 1.0 for l in range(32)] + [math.ldexp(1 + l, l % 15 - 8) * (1 if l % 2 == 0 else -1)
                                                          for l in range(32)]

    def order(big):
        return [big if l == 0 else (1.0 if l in (16, 17) else 0.0) for l in range(32)] * 2

    runs = []
    for a, b in ((xs, hs), (order(16777216.0), order(2048.0))):
        runs.append(({}, {"x": np.array(a, np.float32), "h": interp.narrow_f16(np.array(b, np.float32)),
                          "y": zeros(64), "g": np.zeros(64, np.uint16)}, {}))
    return Case("simd_sums", K.simd_sums(ROCM), runs)


def _narrowings():
    a = [-2 ** 31, -2 ** 31 + 1, -32768, -300, -129, -128, -127, -1, 0, 1, 126, 127, 128, 300, 65535, 2 ** 31 - 1]
    b = [0, 1, 127, 128, 254, 255, 256, 257, 300, 511, 512, 65535, 65536, 2147483648, 0xFFFFFFFE, 0xFFFFFFFF]
    bufs = {"a": np.array(a, np.int32), "b": np.array(b, np.uint32), "clamped_a": np.zeros(16, np.int8),
            "wrapped_a": np.zeros(16, np.int8), "clamped_b": np.zeros(16, np.uint8),
            "wrapped_b": np.zeros(16, np.uint8)}
    return Case("narrowings", K.narrowings(ROCM, 16), [({}, bufs, {})])


def _reductions():
    nans = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0xFF812345], np.uint32).view(np.float32)
    zs = np.array([0x00000000, 0x80000000], np.uint32).view(np.float32)
    xs = np.concatenate([np.resize(nans, 64),
                         np.array([nans[i % 4] if i % 2 == 0 else np.float32(i - 32) for i in range(64)], np.float32),
                         np.array([zs[(i // 3) % 2] for i in range(64)], np.float32),
                         floats(62, 63), np.array([np.inf], np.float32)])
    return Case("reductions", K.reductions(ROCM), [({}, {"x": xs, "y": zeros(256), "z": zeros(4)}, {})], ("y",))


def _params():
    outs = lambda: {"y": zeros(4), "yh": np.zeros(4, np.uint16), "yi": np.zeros(4, np.int32)}  # noqa: E731
    h = lambda v: int(interp.narrow_f16(np.array([v], np.float32))[0])  # noqa: E731
    b = lambda v: int(interp.narrow_bf16(np.array([v], np.float32))[0])  # noqa: E731
    return Case("params", K.params(ROCM), [
        ({"n": 4, "a": False, "b": 1.5, "c": h(0.75), "d": -123456, "e": b(-2.25), "f": 200, "g": -77}, outs(), {}),
        ({"n": 4, "a": True, "b": 1.5, "c": h(-1000.0), "d": 2 ** 31 - 1, "e": b(3.0), "f": 1, "g": -128}, outs(),
         {})])


def _flow():
    kern = K.flow(ROCM)
    size = 3 * kern.threads
    bufs = {"x": f32s(60, 50), "cnt": np.array([w % 13 for w in randoms(61, size)], np.uint32), "y": zeros(size),
            "z": zeros(size), "w": np.zeros(size, np.uint32)}
    return Case("flow", kern, [({"n": 50}, bufs, {})])


def _gemv_cases():
    shapes = [(K.GemvShape(64, 256, 1), K.GemvVariant(1, 64, 4, 1)), (K.GemvShape(64, 256, 3), K.GemvVariant(2, 128, 8, 2)),
              (K.GemvShape(128, 512, 2), K.GemvVariant(4, 256, 8, 4)), (K.GemvShape(64, 512, 3), K.GemvVariant(1, 512, 8, 8)),
              (K.GemvShape(32, 1024, 2), K.GemvVariant(8, 256, 8, 4)), (K.GemvShape(64, 512, 2), K.GemvVariant(2, 128, 4, 1))]
    out = []
    for i, (sh, v) in enumerate(shapes):
        name = f"gemv_{i}"
        bufs = {"x": bf16s(20, sh.batch * sh.inputs), "w": bf16s(21, sh.outputs * sh.inputs),
                "y": np.zeros(sh.batch * sh.outputs, np.uint16)}
        out.append(Case(name, K.gemv(ROCM, name, sh, v), [({}, bufs, {})]))
    return out


def _gemms():
    g = lambda a, b: ({"k": 64}, {"a": a(30, 16 * 64), "b": b(31, 16 * 64), "c": zeros(256)}, {})  # noqa: E731
    tile = lambda m, n, k: ({"m": m, "n": n, "k": k}, {"a": bf16s(40, m * k), "b": bf16s(41, n * k),  # noqa: E731
                                                      "c": zeros(m * n)}, {})
    return [
        Case("gemm_bf16", K.gemm(ROCM, BF16, "gemm_bf16"), [g(bf16s, bf16s)]),
        Case("gemm_f16", K.gemm(ROCM, F16, "gemm_f16"), [g(f16s, f16s)]),
        Case("gemm_f32", K.gemm(ROCM, F32, "gemm_f32"), [g(f32s, f32s)]),
        Case("staged", K.staged(ROCM), [({"k": 64}, {"a": bf16s(32, 1024), "b": bf16s(33, 1024), "c": zeros(256)}, {})]),
        Case("scaled_rows", K.scaled_rows(ROCM),
             [({"k": 64}, {"a": f32s(34, 1024), "b": bf16s(35, 1024), "c": zeros(256)}, {})]),
        Case("gemm_via", K.gemm_via(ROCM),
             [({"k": 32}, {}, {"ab": [None, bf16s(36, 512), bf16s(37, 512)], "cs": [None, zeros(256)]})]),
        Case("tiled", K.tiled(ROCM, K.GemmTile(64, 64, 16, 4), 1024, 1024, 4096), [tile(70, 72, 48)]),
        Case("tiled_narrow", K.tiled(ROCM, K.GemmTile(32, 64, 32, 1), 1024, 2048, 512, "tiled_narrow"),
             [tile(70, 72, 64)]),
    ]


def _known_answers():
    """InterpTest.hs's kernels, on the MI355X."""
    from test_ir import FMA16, FMA32, fma_buffers
    spot = [0xC19FDC5D, 0xC11967A1, 0x3E278700, 0x411F089A, 0x419FEA4A]
    xs = np.array(spot + [0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001]
                  + [k * 1048573 for k in range(4096)], np.uint32).view(np.float32)
    hs = np.arange(0x10000, dtype=np.uint16)
    fl32 = [(0x3F800000, 0x7F800001), (0x7F800001, 0x3F800000), (0, 0x80000000), (0x80000000, 0),
            (0x7FC00001, 0xFF800001), (0x3F800000, 0xBF800000), (0xFFC00001, 0), (0x80000000, 0)]
    fl16 = [(0x3C00, 0x7C01), (0x7C01, 0x3C00), (0, 0x8000), (0x8000, 0), (0x7E01, 0xFC01), (0x3C00, 0xBC00),
            (0xFD01, 0), (0x8000, 0)]
    arrays = [np.array([10 * e + i for i in range(8)], np.float32) for e in range(5)]
    ids = [3, 7, 1000, 4000]
    return [
        Case("lanes", K.lanes(ROCM), [({}, {"y": np.zeros(64, np.uint32)}, {})]),
        Case("count", K.count(ROCM), [({"n": 100}, {"y": np.zeros(100, np.uint32)}, {}),
                                      ({"n": 3}, {"y": np.zeros(5, np.uint32)}, {})]),
        Case("total", K.total(ROCM), [({}, {"y": np.zeros(1, np.uint32)}, {})]),
        Case("pairwise", K.pairwise(ROCM), [({}, {"y": zeros(64), "h": np.zeros(64, np.uint16)}, {})]),
        Case("neighbours", K.neighbours(ROCM), [({}, {"y": zeros(64), "h": np.zeros(64, np.uint16)}, {})]),
        Case("fmas", K.fmas(ROCM), [({"n": len(FMA32), "m": len(FMA16)}, fma_buffers(FMA32, FMA16), {})], ("y", "g")),
        Case("transcendentals", K.transcendentals(ROCM),
             [({"n": len(xs), "m": len(hs)}, {"x": xs, "h": hs, "y": zeros(4 * len(xs)),
                                              "g": np.zeros(4 * len(hs), np.uint16)}, {})], ("y", "g"), ("y", "g")),
        Case("floats", K.floats(ROCM),
             [({"n": 8}, {"x": np.array([a for a, _ in fl32], np.uint32).view(np.float32),
                          "y": np.array([b for _, b in fl32], np.uint32).view(np.float32),
                          "h": np.array([a for a, _ in fl16], np.uint16), "g": np.array([b for _, b in fl16], np.uint16),
                          "out": zeros(32), "out_h": np.zeros(32, np.uint16)}, {})]),
        Case("int32s", K.int32s(ROCM), [({"a": -2 ** 31, "b": -1}, {"y": np.zeros(5, np.int32)}, {}),
                                        ({"a": 2 ** 31 - 1, "b": 2}, {"y": np.zeros(5, np.int32)}, {})]),
        Case("int32_quotient", K.int32_quotient(ROCM), [({"a": -7, "b": 2}, {"y": np.zeros(2, np.int32)}, {})]),
        Case("pick", K.pick(ROCM), [({"entry": 1}, {"y": zeros(6)},
                                     {"arrays": [np.array([10 * e + i for i in range(4)], np.float32)
                                                 for e in range(3)]})]),
        Case("through_table", K.through_table(ROCM), [({"e": 2, "i": 3}, {"y": zeros(1)}, {"arrays": arrays})]),
        Case("eights", K.eights(ROCM), [({"n": 16}, {"y": np.zeros(64, np.uint32)}, {})]),
        Case("from_by", K.from_by(ROCM), [({"start": 4294967290, "step": 5}, {"y": np.zeros(1, np.uint32)}, {})]),
        Case("grid_less", K.grid_less(ROCM), [({"n": 3}, {"y": np.zeros(1, np.uint32)}, {}),
                                              ({"n": 1}, {"y": np.zeros(1, np.uint32)}, {})]),
        Case("through_blocks", K.through_blocks(ROCM),
             [({"entries": 2 ** 30}, {"ids": np.array(ids, np.uint32), "x": f32s(70, 256), "y": zeros(256)},
               {"blocks": [f32s(71 + e, 16384) if e in ids else None for e in range(4001)]})]),
        Case("sum_rows", K.sum_rows(ROCM), [({"n": 3}, {"x": f32s(3, 192), "y": zeros(3)},
                                             {"rows": [f32s(10 + i, 64) for i in range(3)]})]),
        Case("rmsnorm", K.rmsnorm(ROCM, 1000),
             [({"rows": 3, "eps": np.float32(1e-6)}, {"x": bf16s(1, 3000), "w": bf16s(2, 1000),
                                                     "y": np.zeros(3000, np.uint16)}, {})]),
        Case("scale", K.scale(ROCM), [({"n": 300, "s": np.float32(0.7)}, {"x": bf16s(4, 300),
                                                                         "y": np.zeros(300, np.uint16)}, {})]),
        Case("scale_packed", K.scale_packed(ROCM),
             [({"packs": 37, "s": np.float32(-1.3)}, {"x": bf16s(5, 296), "y": np.zeros(296, np.uint16)}, {})]),
        Case("ranged", K.ranged(ROCM), [({"n": 16}, {"y": zeros(64)}, {})]),
    ]


@functools.lru_cache(maxsize=1)
def all_cases() -> tuple:
    return tuple([_arith_f32(), _arith_f16(), _arith_int(), _conv(), _fma_f32(), _fma_f16(), _simd_sums(),
                  _narrowings(), _reductions(), _params(), _flow()] + _gemv_cases() + _gemms() + _known_answers())


class _Cases:
    def __iter__(self):
        return iter(all_cases())

    def __len__(self):
        return len(all_cases())


CASES = _Cases()


@functools.lru_cache(maxsize=1)
def lowered_unit():
    return rocm.lower([check(c.kernel, ROCM) for c in all_cases()])
