"""The kernel IR on the CPU: the builder renders the reference's golden IR
(test/Test/FuryKernel/BuildTest.hs) and its pinned hashes (AbiTest.hs:69-72);
the gate refuses what the MI355X target cannot run; the oracle's interpreter
gives the reference interpreter's known answers (InterpTest.hs) and the
mathematics' (closed forms, f64 within the accumulation bound); and the
backend lowers every case kernel to HIP that hipRTC compiles for gfx950, with
the launch tables the reference's Backend describes."""

import math
import struct
from fractions import Fraction

import numpy as np
import pytest

import ir_kernels as K
from furykernel_amd.ir import ir as I
from furykernel_amd.ir.abi import abi_description, abi_of
from furykernel_amd.ir.build import ROCM, BuildError, KernelBuilder, f32, lit, thread_index, u32
from furykernel_amd.ir.gate import GateError, check
from furykernel_amd.program.graph import BF16, F16, F32, I32, U32
from oracle import interp
from oracle.interp import RunError

T32 = K.T32


def golden(*lines):
    return "\n".join(lines) + "\n"


# ---------------------------------------------------------------------------
# The builder and the IR's text (BuildTest.hs)

def test_scale_renders_as_the_reference_golden():
    assert I.render_kernel(K.scale(T32)) == golden(
        "ir 1", "kernel scale threads 64 simd 32 groups 1u", "  param n : u32 dim 1..65536 multiple of 1",
        "  param s : f32", "  buffer x : read bf16[$n] align 16", "  buffer y : write bf16[$n] align 16", "{",
        "  for divergent i = @thread until $n step 64u {", "    let v : f32 = f32(x[i])",
        "    y[i] = bf16((v * $s))", "  }", "}")


def test_scale_packed_renders_with_its_width():
    body = ", ".join(f"bf16((f32(v_{i}) * $s))" for i in range(8))
    assert I.render_kernel(K.scale_packed(T32)) == golden(
        "ir 1", "kernel scale_packed threads 64 simd 32 groups 1u", "  param packs : u32 dim 1..8192 multiple of 1",
        "  param s : f32", "  buffer x : read bf16[($packs * 8u)] align 16",
        "  buffer y : write bf16[($packs * 8u)] align 16", "{", "  for divergent j = @thread until $packs step 64u {",
        "    let (v_0, v_1, v_2, v_3, v_4, v_5, v_6, v_7) : bf16 = x.pack8[j]", f"    y.pack8[j] = ({body})", "  }",
        "}")


def test_control_tables_fragments_literals_render():
    assert I.render_kernel(K.controlled(T32)) == golden(
        "ir 1", "kernel controlled threads 64 simd 32 groups 1u", "  buffer y : write f32[2u] align 16",
        "  threadgroup partial : f32[2]", "{", "  let s : f32 = simd_sum(f32:0x3f800000)",
        "  if divergent (@lane == 0u) {", "    partial[@simd_group] = s", "  }", "  barrier",
        "  if divergent (@thread < 2u) {", "    y[@thread] = partial[@thread]", "  }", "}")
    assert I.render_kernel(K.via_table(T32)) == golden(
        "ir 1", "kernel via_table threads 32 simd 32 groups 1u", "  param e : u32", "  buffer y : write f32[8u] align 16",
        "  table arrays : 4u x f32[8u] align 16", "{", "  if divergent (@thread < 8u) {",
        "    y[@thread] = arrays[$e][@thread]", "  }", "}")
    assert I.render_kernel(K.product8(T32)) == golden(
        "ir 1", "kernel product8 threads 32 simd 32 groups 1u", "  buffer a : read f32[64u] align 16",
        "  buffer b : read f32[64u] align 16", "  buffer c : write f32[64u] align 16", "{",
        "  fragment acc : f32[8x8] = 0", "  fragment fa : f32[8x8] = 0", "  fragment fb : f32[8x8] = 0",
        "  fa = a.fragment[0u, stride 8u]", "  fb = b.fragment[0u, stride 8u]", "  acc = fa * fb + acc",
        "  c.fragment[0u, stride 8u] = acc", "}")
    k = KernelBuilder("literals", T32)
    k.threads(32)
    k.groups(1)
    k.let("nan", f32(float("nan")))
    k.let("h", lit(F16, Fraction(1) + Fraction(1, 2048) + Fraction(1, 1073741824)))
    assert I.render_kernel(k.done()[0]) == golden(
        "ir 1", "kernel literals threads 32 simd 32 groups 1u", "{", "  let nan : f32 = f32:0x7fc00000",
        "  let h : f16 = f16:0x3c01", "}")


def test_locals_get_fresh_names_and_problems_are_noticed():
    k = KernelBuilder("twice", T32)
    v = k.param("v", F32)
    k.threads(32)
    k.groups(1)
    a = k.let("v", v)
    k.let("v", a + a)
    kernel, problems = k.done()
    assert problems == []
    assert I.render_kernel(kernel) == golden("ir 1", "kernel twice threads 32 simd 32 groups 1u", "  param v : f32",
                                             "{", "  let v_1 : f32 = $v", "  let v_2 : f32 = (v_1 + v_1)", "}")
    k = KernelBuilder("clash", T32)
    n = k.dim("x", I.DimRange(1, 8, 1))
    k.buffer("x", I.READ, U32, n)
    assert [p.message for p in k.done()[1]] == ["The name x is declared twice.",
                                                "No thread count: declare one with threads.",
                                                "No grid size: declare one with groups."]
    k = KernelBuilder("short", T32)
    y = k.buffer("y", I.WRITE, F32, 4)
    k.threads(32)
    k.groups(1)
    k.store_pack(y, 0, [1.0, 2.0, 3.0], n=4)
    assert [p.message for p in k.done()[1]] == ["A pack of 4 stored to y with 3 values."]


def test_expressions_and_literals_render():
    assert I.render_expr(I.ENarrowInt("clamp", "i8", I.EVar("x"))) == "i8_clamped(x)"
    assert I.render_expr(I.ENarrowInt("wrap", "i8", I.EVar("x"))) == "i8_wrapped(x)"
    from furykernel_amd.ir.build import fma_e
    assert I.render_expr(fma_e(lit(F32, 1), 2, 3).ir) == "fma(f32:0x3f800000, f32:0x40000000, f32:0x40400000)"
    with pytest.raises(BuildError, match="the literal 3000000000 is outside i32's range, -2147483648 to 2147483647"):
        lit(I32, 3000000000)
    with pytest.raises(BuildError, match="the literal 4294967296 is outside u32's range, 0 to 4294967295"):
        lit(U32, 4294967296)
    assert I.render_literal(lit(F32, -0.0).ir.lit) == "f32:0x80000000"


def test_the_pinned_ir_and_abi_hashes():
    """AbiTest.hs:69-72: what changes them changes every committed hash."""
    k = K.scale(T32)
    assert I.ir_hash(k) == 0x60C50BD78967A3D0
    assert abi_of(k).hash == 0xE99AD54061A304FF
    r = K.rmsnorm(T32, 2816)
    base = abi_of(r).hash
    renamed = I.Kernel(**{**r.__dict__, "buffers": tuple(I.Buffer("gamma" if b.name == "w" else b.name, b.access,
                                                                   b.type, b.align, b.extent) for b in r.buffers)})
    resized = I.Kernel(**{**r.__dict__, "buffers": tuple(I.Buffer(b.name, b.access, b.type, b.align,
                                                                   I.ELit(I.lit_u32(1))) for b in r.buffers)})
    assert abi_of(renamed).hash != base and abi_of(resized).hash == base
    assert abi_description(abi_of(k)).startswith("abi 1\nbuffer x read bf16 align 16\n")


def test_builder_refuses_what_the_types_refuse():
    k = KernelBuilder("bad", ROCM)
    x = k.buffer("x", I.READ, BF16, 64)
    k.threads(64)
    with pytest.raises(BuildError, match="no arithmetic"):
        _ = k.load(x, 0) + k.load(x, 1)
    with k.when_lane(thread_index < 3):
        with pytest.raises(BuildError, match="barrier"):
            k.barrier()
        with pytest.raises(BuildError, match="SIMD group"):
            k.simd_sum("s", f32(1.0))
    with pytest.raises(BuildError, match="threads"):
        KernelBuilder("t", ROCM).threads(96)


# ---------------------------------------------------------------------------
# The gate

def test_the_gate_takes_the_case_kernels_and_refuses_others():
    check(K.scale(ROCM), ROCM)
    with pytest.raises(GateError, match="built for SIMD groups of 32 lanes"):
        check(K.scale(T32), ROCM)
    body = (I.SIf("divergent", I.EBin("lt", I.EBuiltin("thread"), I.ELit(I.lit_u32(2))), (I.SBarrier(),)),)
    bad = I.Kernel("bad", 64, 64, I.ELit(I.lit_u32(1)), body=body)
    with pytest.raises(GateError, match="A barrier where not every thread"):
        check(bad, ROCM)
    typed = I.Kernel("typed", 64, 64, I.ELit(I.lit_u32(1)),
                     body=(I.SLet("a", F32, I.EBin("add", I.ELit(I.lit_f32(1.0)), I.ELit(I.lit_u32(1)))),))
    with pytest.raises(GateError, match="The operands of \\+ are f32 and u32"):
        check(typed, ROCM)
    big = I.Kernel("big", 64, 64, I.ELit(I.lit_u32(1)), tg_arrays=(I.TgArray("t", F32, 20000),))
    with pytest.raises(GateError, match="threadgroup memory"):
        check(big, ROCM)


# ---------------------------------------------------------------------------
# The oracle's interpreter against the reference interpreter's known answers

def run32(kernel, params, buffers, tables=None):
    return interp.run(kernel, 32, params, buffers, tables)[0]


def test_lanes_branch_and_reconverge_and_loops_visit_once():
    y = run32(K.lanes(T32), {}, {"y": np.zeros(64, np.uint32)})["y"]
    assert y.tolist() == [1 if l % 32 < 3 else 2 for l in range(64)]
    assert (run32(K.count(T32), {"n": 100}, {"y": np.zeros(100, np.uint32)})["y"] == 1).all()
    for caps in (K.T8, K.T16, K.T32, K.T64):
        assert interp.run(K.total(caps), caps.simd_width, {}, {"y": np.zeros(1, np.uint32)})[0]["y"][0] == 2016


def test_simd_sums_add_pairwise_neighbours_first():
    out = run32(K.pairwise(T32), {}, {"y": np.zeros(32, np.float32), "h": np.zeros(32, np.uint16)})
    assert (out["y"] == 16777246).all() and (out["h"] == 0x680F).all()
    out = run32(K.neighbours(T32), {}, {"y": np.zeros(32, np.float32), "h": np.zeros(32, np.uint16)})
    assert (out["y"] == 16777218).all() and (out["h"] == 0x6801).all()


FMA32 = [((0x3F800001, 0x3F800001, 0xBF800002), 0x28800000), ((0x3F800800, 0x3F800800, 0xBF801000), 0x33800000),
         ((0x7F7FFFFF, 0x40000000, 0xFF7FFFFF), 0x7F7FFFFF), ((0x3F800001, 0x3F7FFFFF, 0x28800000), 0x3F800001),
         ((0x1A000000, 0x1A400000, 0x00000000), 0x00000001), ((0x9A000000, 0x19800000, 0x00000000), 0x80000000),
         ((0x1A000000, 0x1A000000, 0x00000000), 0x00000000),
         # special cases (InterpTest.hs:555-572)
         ((0x7F800000, 0x00000000, 0x3F800000), 0x7FC00000), ((0x00000000, 0xFF800000, 0x7FC00000), 0x7FC00000),
         ((0x7F800000, 0x3F800000, 0xFF800000), 0x7FC00000), ((0x7F800000, 0x3F800000, 0x7F800000), 0x7F800000),
         ((0x7F800000, 0xBF800000, 0x40A00000), 0xFF800000), ((0x40000000, 0x40400000, 0x7F800000), 0x7F800000),
         ((0x7FC00001, 0x00000000, 0x7F800000), 0x7FC00000), ((0x00000000, 0x3F800000, 0x80000000), 0x00000000),
         ((0x80000000, 0x3F800000, 0x80000000), 0x80000000), ((0xBF800000, 0x00000000, 0x80000000), 0x80000000),
         ((0x3F800000, 0x3F800000, 0xBF800000), 0x00000000), ((0xBF800000, 0x3F800000, 0x3F800000), 0x00000000),
         ((0x80000000, 0x80000000, 0x80000000), 0x00000000)]
FMA16 = [((0x2740, 0x246A, 0x3C00), 0x3C01), ((0x5BF8, 0x5C04, 0x0000), 0x7C00), ((0x5BF8, 0x5C04, 0xCC00), 0x7BFF),
         ((0x3C01, 0x3C01, 0xBC02), 0x0010), ((0x0C00, 0x0C00, 0x0000), 0x0001), ((0x0C00, 0x0800, 0x0000), 0x0000),
         ((0x0C00, 0x0A00, 0x0000), 0x0001), ((0x8C00, 0x0400, 0x0000), 0x8000),
         ((0x7C00, 0x0000, 0x3C00), 0x7E00), ((0x7C00, 0x3C00, 0xFC00), 0x7E00), ((0xFC00, 0x3C00, 0xFC00), 0xFC00),
         ((0x7E01, 0x3C00, 0x3C00), 0x7E00), ((0x8000, 0x3C00, 0x8000), 0x8000), ((0x3C00, 0x3C00, 0xBC00), 0x0000)]


def fma_buffers(f32s, f16s):
    a, b, c = (np.array([t[0][i] for t in f32s], np.uint32).view(np.float32) for i in range(3))
    ah, bh, ch = (np.array([t[0][i] for t in f16s], np.uint16) for i in range(3))
    return {"a": a, "b": b, "c": c, "ah": ah, "bh": bh, "ch": ch, "y": np.zeros(len(f32s), np.float32),
            "g": np.zeros(len(f16s), np.uint16)}


def test_fma_rounds_once_and_its_special_cases():
    out = run32(K.fmas(T32), {"n": len(FMA32), "m": len(FMA16)}, fma_buffers(FMA32, FMA16))
    assert out["y"].view(np.uint32).tolist() == [w for _, w in FMA32]
    assert out["g"].tolist() == [w for _, w in FMA16]


def test_transcendentals_binary64_rounded_once():
    """InterpTest.hs:68-86: five spot values of exp where macOS's binary32 exp
    misrounds, and the binary16 exps and log that rounding through binary32
    would round twice."""
    spot = [0xC19FDC5D, 0xC11967A1, 0x3E278700, 0x411F089A, 0x419FEA4A]
    xs = np.array(spot + [0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001]
                  + [k * 1048573 for k in range(4096)], np.uint32).view(np.float32)
    hs = np.arange(0x10000, dtype=np.uint16)
    out = run32(K.transcendentals(T32), {"n": len(xs), "m": len(hs)},
                {"x": xs, "h": hs, "y": np.zeros(4 * len(xs), np.float32), "g": np.zeros(4 * len(hs), np.uint16)})
    y, g = out["y"].view(np.uint32), out["g"]
    assert [int(y[4 * i + 1]) for i in range(5)] == [0x311020AD, 0x388FC7EB, 0x3F96C052, 0x46A1FEE6, 0x4DE4E7BE]
    assert [int(g[4 * 0x1F79 + 1]), int(g[4 * 0x25CF + 1]), int(g[4 * 0x1D78 + 2])] == [0x3C07, 0x3C17, 0xC53B]
    with np.errstate(all="ignore"):
        x64 = xs.astype(np.float64)
        want = np.stack([1 / np.sqrt(x64), np.exp(x64), np.log(x64), np.tanh(x64)], 1).astype(np.float32)
    ok = (want.view(np.uint32).ravel() == y) | (np.isnan(want.ravel()) & np.isnan(out["y"]))
    assert ok.mean() > 0.999  # numpy's binary64 against the platform libm's: at most a rare last bit


def test_minimum_maximum_negation_magnitude():
    snan, qnan = 0x7F800001, 0x7FC00001
    f32p = [(0x3F800000, snan), (snan, 0x3F800000), (0x00000000, 0x80000000), (0x80000000, 0x00000000),
            (qnan, 0xFF800001), (0x3F800000, 0xBF800000), (0x7F800001, 0), (0xFFC00001, 0), (0x80000000, 0)]
    f16p = [(0x3C00, 0x7C01), (0x7C01, 0x3C00), (0x0000, 0x8000), (0x8000, 0x0000), (0x7E01, 0xFC01),
            (0x3C00, 0xBC00), (0x7D00, 0), (0xFD01, 0), (0x8000, 0)]
    n = len(f32p)
    out = run32(K.floats(T32), {"n": n},
                {"x": np.array([a for a, _ in f32p], np.uint32).view(np.float32),
                 "y": np.array([b for _, b in f32p], np.uint32).view(np.float32),
                 "h": np.array([a for a, _ in f16p], np.uint16), "g": np.array([b for _, b in f16p], np.uint16),
                 "out": np.zeros(4 * n, np.float32), "out_h": np.zeros(4 * n, np.uint16)})
    o, oh = out["out"].view(np.uint32).reshape(n, 4), out["out_h"].reshape(n, 4)

    def lee32(w):
        return 0x7FC00000 if (w & 0x7F800000) == 0x7F800000 and w & 0x7FFFFF else (0 if w == 0x80000000 else w)

    def lee16(w):
        return 0x7E00 if (w & 0x7C00) == 0x7C00 and w & 0x3FF else (0 if w == 0x8000 else w)
    assert [[lee32(int(w)) for w in r[:2]] for r in o[:6]] == [
        [0x3F800000] * 2, [0x3F800000] * 2, [0, 0], [0, 0], [0x7FC00000] * 2, [0xBF800000, 0x3F800000]]
    assert [[lee16(int(w)) for w in r[:2]] for r in oh[:6]] == [
        [0x3C00] * 2, [0x3C00] * 2, [0, 0], [0, 0], [0x7E00] * 2, [0xBC00, 0x3C00]]
    assert [r[2:].tolist() for r in o[6:]] == [[0xFF800001, 0x7F800001], [0x7FC00001, 0x7FC00001], [0, 0]]
    assert [r[2:].tolist() for r in oh[6:]] == [[0xFD00, 0x7D00], [0x7D01, 0x7D01], [0, 0]]


def test_integers_wrap_divide_and_narrow():
    def ints(a, b):
        return run32(K.int32s(T32), {"a": a, "b": b}, {"y": np.zeros(5, np.int32)})["y"].tolist()
    lo, hi = -2 ** 31, 2 ** 31 - 1
    assert ints(lo, -1) == [hi, lo + 1, lo, lo, lo]
    assert ints(hi, 2) == [lo + 1, hi - 2, -2, lo + 1, hi]
    q = run32(K.int32_quotient(T32), {"a": -7, "b": 2}, {"y": np.zeros(2, np.int32)})["y"].tolist()
    assert q == [-3, -1]
    with pytest.raises(RunError, match="DivideByZero"):
        run32(K.int32_quotient(T32), {"a": 7, "b": 0}, {"y": np.zeros(2, np.int32)})
    with pytest.raises(RunError, match="IntegerOverflow"):
        run32(K.int32_quotient(T32), {"a": lo, "b": -1}, {"y": np.zeros(2, np.int32)})
    out = run32(K.narrowings(T32), {}, {"a": np.array([300, -300, -129, 127], np.int32),
                                        "b": np.array([300, 255, 256, 65535], np.uint32),
                                        "clamped_a": np.zeros(4, np.int8), "wrapped_a": np.zeros(4, np.int8),
                                        "clamped_b": np.zeros(4, np.uint8), "wrapped_b": np.zeros(4, np.uint8)})
    assert [out[n].tolist() for n in ("clamped_a", "wrapped_a", "clamped_b", "wrapped_b")] == [
        [127, -128, -128, 127], [44, -44, 127, 127], [255, 255, 255, 255], [44, 255, 0, 255]]


def test_tables_elements_packs_and_unbound_entries():
    arrays = [np.array([10 * e + i for i in range(4)], np.float32) for e in range(3)]
    out = run32(K.pick(T32), {"entry": 1}, {"y": np.zeros(6, np.float32)}, {"arrays": arrays})
    assert out["y"].tolist() == [10, 11, 12, 13, 12, 13]
    with pytest.raises(RunError, match="OutOfBounds.*'arrays', 3, 3"):
        run32(K.pick(T32), {"entry": 3}, {"y": np.zeros(6, np.float32)}, {"arrays": arrays})
    ids = [3, 7, 1000, 4000]
    given = [np.zeros(16384, np.float32) if e in ids else None for e in range(4001)]
    xs = np.arange(256, dtype=np.float32)
    out, tabs = interp.run(K.through_blocks(T32), 32, {"entries": 2 ** 30},
                           {"ids": np.array(ids, np.uint32), "x": xs, "y": np.zeros(256, np.float32)},
                           {"blocks": given})
    assert out["y"].tolist() == (2 * xs).tolist()
    assert [tabs["blocks"][e][16320:].tolist() for e in ids] == [(2 * xs[g * 64:(g + 1) * 64]).tolist()
                                                                  for g in range(4)]
    assert not tabs["blocks"][7][:16320].any()
    with pytest.raises(RunError, match="UnboundEntry.*4001"):
        interp.run(K.through_blocks(T32), 32, {"entries": 2 ** 30},
                   {"ids": np.array([3, 7, 1000, 4001], np.uint32), "x": xs, "y": np.zeros(256, np.float32)},
                   {"blocks": given + [None]})


def test_errors_instead_of_undefined_behaviour():
    with pytest.raises(RunError, match="ShortBuffer.*'y', 100, 99"):
        run32(K.count(T32), {"n": 100}, {"y": np.zeros(99, np.uint32)})
    with pytest.raises(RunError, match="UninitializedRead.*'t', 1"):
        run32(K.uninitialised(T32), {}, {"y": np.zeros(1, np.uint32)})
    with pytest.raises(RunError, match="DivideByZero"):
        run32(K.divide(T32), {"d": 0}, {"y": np.zeros(1, np.uint32)})
    with pytest.raises(RunError, match="OutOfBounds.*'x', 7, 4"):
        run32(K.past_end(T32), {}, {"x": np.zeros(4, np.float32), "y": np.zeros(1, np.float32)})
    with pytest.raises(RunError, match=r"LaunchSizeOutOfRange.*\(\$n - 1u\).*-1"):
        run32(K.grid_less(T32), {"n": 0}, {"y": np.zeros(1, np.uint32)})
    assert run32(K.grid_less(T32), {"n": 3}, {"y": np.zeros(1, np.uint32)})["y"].tolist() == [1]
    with pytest.raises(RunError, match="NonTermination"):
        run32(K.from_by(T32), {"start": 0, "step": 0}, {"y": np.zeros(1, np.uint32)})
    with pytest.raises(RunError, match="NonTermination"):
        run32(K.from_by(T32), {"start": 4294967290, "step": 7}, {"y": np.zeros(1, np.uint32)})
    assert run32(K.from_by(T32), {"start": 4294967290, "step": 5}, {"y": np.zeros(1, np.uint32)})["y"][0] == 1
    assert run32(K.count(T32), {"n": 3}, {"y": np.zeros(5, np.uint32)})["y"].tolist() == [1, 1, 1, 0, 0]
    for n, ok in ((16, True), (12, False), (72, False), (0, False)):
        if ok:
            assert run32(K.eights(T32), {"n": n}, {"y": np.zeros(64, np.uint32)})["y"][:2].tolist() == [0, 1]
        else:
            with pytest.raises(RunError, match=f"DimOutOfRange.*'n', {n}"):
                run32(K.eights(T32), {"n": n}, {"y": np.zeros(64, np.uint32)})
    arrays = [np.array([10 * e + i for i in range(8)], np.float32) for e in range(5)]
    assert run32(K.through_table(T32), {"e": 2, "i": 3}, {"y": np.zeros(1, np.float32)},
                 {"arrays": arrays})["y"].tolist() == [23]
    with pytest.raises(RunError, match="OutOfBounds.*'arrays', 3, 3"):
        run32(K.through_table(T32), {"e": 3, "i": 0}, {"y": np.zeros(1, np.float32)}, {"arrays": arrays})
    with pytest.raises(RunError, match="OutOfBounds.*'arrays', 4, 4"):
        run32(K.through_table(T32), {"e": 1, "i": 4}, {"y": np.zeros(1, np.float32)}, {"arrays": arrays})


def widen_bf16(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def test_scale_is_its_spec_and_packs_are_elements():
    """InterpTest.hs:266-293: bit for bit narrowBF16(widen(x) * s), and the
    packed kernel the scalar one."""
    rng = np.random.default_rng(1)
    for n, s in ((300, np.float32(-1.3)), (8 * 37, np.float32(0.7))):
        xs = rng.integers(0, 0x10000, n).astype(np.uint16)
        y = run32(K.scale(T32), {"n": n, "s": s}, {"x": xs, "y": np.zeros(n, np.uint16)})["y"]
        with np.errstate(all="ignore"):
            want = interp.narrow_bf16(widen_bf16(xs) * s)
        assert np.array_equal(y, want)
        m = 8 * (n // 8)
        yp = run32(K.scale_packed(T32), {"packs": n // 8, "s": s}, {"x": xs, "y": np.zeros(n, np.uint16)})["y"]
        assert np.array_equal(yp[:m], y[:m]) and not yp[m:].any()


def noise(s, i):
    return ((s * 7919 + i * 104729) % 2001 - 1000) / 1000


@pytest.mark.parametrize("t", [BF16, F16, F32])
def test_fragment_products_are_their_f64_meaning(t):
    """FragmentTest.hs:33-41: C = A · Bᵀ within 1e-4 of binary64's."""
    kk = 64
    a = np.array([noise(1, i) for i in range(16 * kk)], np.float32)
    b = np.array([noise(2, i) for i in range(16 * kk)], np.float32)
    if t == BF16:
        a, b = interp.narrow_bf16(a), interp.narrow_bf16(b)
        wa, wb = widen_bf16(a), widen_bf16(b)
    elif t == F16:
        a, b = interp.narrow_f16(a), interp.narrow_f16(b)
        wa, wb = interp.widen_f16(a), interp.widen_f16(b)
    else:
        wa, wb = a, b
    c = run32(K.gemm(T32, t), {"k": kk}, {"a": a, "b": b, "c": np.zeros(256, np.float32)})["c"]
    exact = wa.astype(np.float64).reshape(16, kk) @ wb.astype(np.float64).reshape(16, kk).T
    assert np.abs(c.reshape(16, 16) - exact).max() < 1e-4


def test_scaled_rows_and_staged_tiles_agree_with_f64():
    kk = 64
    a = np.array([noise(1, i) for i in range(16 * kk)], np.float32)
    b = interp.narrow_bf16(np.array([noise(2, i) for i in range(16 * kk)], np.float32))
    exact = a.astype(np.float64).reshape(16, kk) @ widen_bf16(b).astype(np.float64).reshape(16, kk).T
    c = run32(K.scaled_rows(T32), {"k": kk}, {"a": a, "b": b, "c": np.zeros(256, np.float32)})["c"].reshape(16, 16)
    scale = np.array([2 ** (i % 8) * 0.3 for i in range(16)])[:, None]
    assert np.abs(c - exact * scale).max() / 2 ** 7 < 1e-4
    ab = interp.narrow_bf16(a)
    c = run32(K.staged(T32), {"k": kk}, {"a": ab, "b": b, "c": np.zeros(256, np.float32)})["c"].reshape(16, 16)
    exact = widen_bf16(ab).astype(np.float64).reshape(16, kk) @ widen_bf16(b).astype(np.float64).reshape(16, kk).T
    assert np.abs(c - exact).max() < 1e-4


@pytest.mark.parametrize("caps", [T32, ROCM], ids=["T32", "MI355X"])
def test_a_tiled_gemm_agrees_with_f64_and_its_order_is_the_tiles(caps):
    """Tile.hs: each element summed over k in order, eight at a time, so two
    tile shapes give one result, within the accumulation bound of f64's."""
    m, n, kk = 70, 72, 64
    rng = np.random.default_rng(3)
    a = interp.narrow_bf16(rng.standard_normal(m * kk).astype(np.float32))
    b = interp.narrow_bf16(rng.standard_normal(n * kk).astype(np.float32))
    outs = []
    for t, sizes in ((K.GemmTile(64, 64, 16, 4), (1024, 1024, 4096)), (K.GemmTile(32, 64, 32, 1), (1024, 2048, 512))):
        kern = K.tiled(caps, t, *sizes)
        outs.append(interp.run(kern, caps.simd_width, {"m": m, "n": n, "k": kk},
                               {"a": a, "b": b, "c": np.zeros(m * n, np.float32)})[0]["c"])
    exact = widen_bf16(a).astype(np.float64).reshape(m, kk) @ widen_bf16(b).astype(np.float64).reshape(n, kk).T
    bound = kk * 2.0 ** -24 * (np.abs(widen_bf16(a).reshape(m, kk)) @ np.abs(widen_bf16(b).reshape(n, kk)).T)
    assert np.all(np.abs(outs[0].reshape(m, n) - exact) <= bound)
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("caps", [T32, ROCM], ids=["T32", "MI355X"])
def test_gemv_variants_agree_and_are_within_f64s_bound(caps):
    """Gemv.hs:5-27: the pack width and the split fix the order; rows and
    threads do not.  Every variant within binary32's accumulation bound."""
    sh = K.GemvShape(64, 512, 2)
    rng = np.random.default_rng(5)
    x = interp.narrow_bf16(rng.standard_normal(sh.batch * sh.inputs).astype(np.float32))
    w = interp.narrow_bf16(rng.standard_normal(sh.outputs * sh.inputs).astype(np.float32))
    wide = caps.simd_width
    res = {}
    for v in (K.GemvVariant(1, 2 * wide, 8, 1), K.GemvVariant(2, 4 * wide, 8, 1), K.GemvVariant(1, 4 * wide, 8, 2),
              K.GemvVariant(4, 2 * wide, 8, 2)):
        kern = K.gemv(caps, "gemv", sh, v)
        res[v] = interp.run(kern, wide, {}, {"x": x, "w": w, "y": np.zeros(sh.batch * sh.outputs, np.uint16)})[0]["y"]
    vs = list(res)
    assert np.array_equal(res[vs[0]], res[vs[1]]) and np.array_equal(res[vs[2]], res[vs[3]])
    exact = widen_bf16(x).astype(np.float64).reshape(sh.batch, -1) @ widen_bf16(w).astype(np.float64).reshape(
        sh.outputs, -1).T
    got = widen_bf16(res[vs[0]]).reshape(sh.batch, sh.outputs)
    bound = sh.inputs * 2.0 ** -24 * (np.abs(widen_bf16(x).reshape(sh.batch, -1)) @ np.abs(
        widen_bf16(w).reshape(sh.outputs, -1)).T) + np.abs(exact) * 2.0 ** -8
    assert np.all(np.abs(got - exact) <= bound)


def test_rmsnorm_within_a_bf16_ulp_of_its_f64_spec():
    """ReduceTest.hs:97-108: RMSNorm within 1 bf16 ulp of the f64 spec."""
    hidden, rows = 1000, 3
    rng = np.random.default_rng(7)
    x = interp.narrow_bf16(rng.standard_normal(rows * hidden).astype(np.float32))
    w = interp.narrow_bf16((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))
    for caps in (T32, ROCM):
        y = interp.run(K.rmsnorm(caps, hidden), caps.simd_width, {"rows": rows, "eps": np.float32(1e-6)},
                       {"x": x, "w": w, "y": np.zeros(rows * hidden, np.uint16)})[0]["y"]
        xf = widen_bf16(x).astype(np.float64).reshape(rows, hidden)
        want = xf / np.sqrt((xf * xf).mean(1, keepdims=True) + 1e-6) * widen_bf16(w).astype(np.float64)
        got = widen_bf16(y).reshape(rows, hidden).astype(np.float64)
        ulp = 2.0 ** (np.floor(np.log2(np.abs(want))) - 7)
        assert np.all(np.abs(got - want) <= ulp)


# ---------------------------------------------------------------------------
# The backend

from gpu_ir_cases import CASES, lowered_unit  # noqa: E402


def test_every_case_lowers_to_hip_that_hiprtc_compiles_for_gfx950():
    from furykernel_amd.ir.runtime import compile_source
    low = lowered_unit()
    code = compile_source(low.source, "cases.hip")
    assert code[:4] == b"\x7fELF" and len(code) > 10000
    names = [lk.name for lk in low.kernels]
    assert len(set(names)) == len(names) == len({c.kernel.name for c in CASES})


def test_the_launch_tables():
    from furykernel_amd.ir import rocm
    low = lowered_unit()
    by = {lk.name: lk for lk in low.kernels}
    lk = by["through_blocks"]
    assert lk.bindings == (("ids", 0), ("x", 1), ("y", 2), ("blocks", 3)) and lk.params_binding == 4
    assert lk.threads == 64 and I.render_expr(lk.groups) == "4u" and lk.tg_memory == 0
    assert by["reductions"].params_binding is None and by["reductions"].tg_memory == 16
    assert by["scale"].abi.hash == abi_of(K.scale(ROCM)).hash and by["scale"].ir_hash == I.ir_hash(K.scale(ROCM))
    assert "extern \"C\" __global__ void __launch_bounds__(64) scale(" in low.source
    with pytest.raises(rocm.LoweringError, match="lowered 2 times"):
        rocm.lower([check(K.scale(ROCM), ROCM)] * 2)
    from furykernel_amd.ir.gate import Checked
    with pytest.raises(rocm.LoweringError, match="checked for T32"):
        rocm.lower([Checked(K.scale(T32), T32)])


def test_the_launch_contract_is_checked_on_the_host():
    from furykernel_amd.ir.runtime import LaunchError, launch_size, params_bytes
    low = lowered_unit()
    by = {lk.name: lk for lk in low.kernels}
    # the params struct in the ABI's layout: a bool, then f32, f16, i32, bf16, u8, i8
    raw = params_bytes(by["params"], {"n": 4, "a": True, "b": 1.5, "c": 0x3A00, "d": -123456, "e": 0xC010,
                                      "f": 200, "g": -77})
    f = {x.name: x.offset for x in by["params"].abi.params}
    assert struct.unpack_from("<I", raw, f["n"])[0] == 4 and raw[f["a"]] == 1
    assert struct.unpack_from("<f", raw, f["b"])[0] == 1.5 and struct.unpack_from("<i", raw, f["d"])[0] == -123456
    assert struct.unpack_from("<b", raw, f["g"])[0] == -77 and len(raw) == by["params"].abi.params_size
    assert launch_size({"m": 70, "n": 72}, by["tiled"].groups) == 4
    with pytest.raises(LaunchError, match="outside u32"):
        launch_size({"n": 0}, I.EBin("sub", I.EParam("n"), I.ELit(I.lit_u32(1))))
