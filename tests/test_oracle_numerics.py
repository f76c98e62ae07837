"""The oracle's numerics and reductions, pinned by the reference's own vectors
and by independent implementations (numpy's IEEE conversions, exact f64).

Sources: test/Test/FuryKernel/NumericsTest.hs, InterpTest.hs, ReduceTest.hs.
"""

import math
import struct

import numpy as np
import pytest

from oracle import fkref


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def f32_of(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b))[0]


def value_of(spec) -> float:
    """A fixture's number: a float, or a small expression in powers of two."""
    if isinstance(spec, (int, float)):
        return float(spec)
    table = {
        "2^-25+2^-60": 2.0**-25 + 2.0**-60,
        "-(2^-26)": -(2.0**-26),
        "inf": math.inf,
        "1+2^-11+2^-25": 1 + 2.0**-11 + 2.0**-25,
        "1+2^-8": 1 + 2.0**-8,
        "1+3*2^-8": 1 + 3 * 2.0**-8,
    }
    return table[spec]


def test_f16_edges(golden):
    g = golden("numerics.json")
    for x, want in g["f16_edges"]["cases"]:
        assert fkref.narrow_f16(float(np.float32(x))) == int(want, 16), x


def test_f16_from_f64_edges_round_once(golden):
    g = golden("numerics.json")
    for x, want in g["f16_f64_edges"]["cases"]:
        assert fkref.narrow_f16_f64(value_of(x)) == int(want, 16), x
    # Through binary32 the same value rounds twice, to the tie's even side.
    for x, want in g["f16_f64_edges"]["through_f32"]:
        assert fkref.narrow_f16(float(np.float32(value_of(x)))) == int(want, 16)
    # A NaN narrows to a quiet NaN of its sign.
    assert fkref.narrow_f16_f64(struct.unpack("<d", struct.pack("<Q", 0xFFF0000000000001))[0]) & 0xFE00 == 0xFE00


def test_bf16_ties_to_even(golden):
    g = golden("numerics.json")
    for x, want in g["bf16_ties"]["cases"]:
        assert fkref.narrow_bf16(value_of(x)) == int(want, 16)


def test_nan_widening_keeps_sign_and_payload(golden):
    g = golden("numerics.json")["nan_widening"]
    for h, want in g["bf16"]:
        assert f32_bits(fkref.widen_bf16(int(h, 16))) == int(want, 16)
    for h, want in g["f16"]:
        assert f32_bits(fkref.widen_f16(int(h, 16))) == int(want, 16)


def test_nans_narrow_quiet_with_their_sign():
    nan = f32_of(0xFF800001)
    assert fkref.narrow_bf16(nan) & 0x8040 == 0x8040
    assert fkref.narrow_f16(nan) & 0x8200 == 0x8200


def test_every_f16_and_bf16_round_trips():
    """NumericsTest.hs:27-30: 16 bits -> f32 -> 16 bits is the identity, NaNs aside;
    and widening agrees with numpy's IEEE conversion on every non-NaN value."""
    hs = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = hs.view(np.float16).astype(np.float32)
    for h in range(0, 1 << 16):
        w = fkref.widen_f16(h)
        if math.isnan(w):
            continue
        assert f32_bits(w) == int(ref.view(np.uint32)[h]), hex(h)
        assert fkref.narrow_f16(w) == h
        b = fkref.widen_bf16(h)
        if not math.isnan(b):
            assert fkref.narrow_bf16(b) == h


def test_f16_narrowing_matches_numpy_on_random_floats():
    """numpy's float32 -> float16 is IEEE round-to-nearest-even with subnormals:
    an independent implementation of narrowF16 (NumericsTest.hs:112-118)."""
    rng = np.random.default_rng(2026)
    xs = np.concatenate([
        rng.integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        rng.uniform(-70000, 70000, 5000).astype(np.float32),
        rng.uniform(-1e-4, 1e-4, 5000).astype(np.float32),
    ])
    xs = xs[~np.isnan(xs)]
    want = xs.astype(np.float16).view(np.uint16)
    for x, w in zip(xs.tolist(), want.tolist()):
        assert fkref.narrow_f16(x) == w, x


def test_f16_from_f64_at_every_midpoint():
    """NumericsTest.hs:87-90,188-199: each midpoint of neighbouring binary16 values
    goes to the even one, a binary64 ulp either side to the nearer."""
    for lo in range(0, 0x7BFF, 37):
        a = float(np.uint16(lo).view(np.float16))
        b = float(np.uint16(lo + 1).view(np.float16))
        mid = a + (b - a) / 2
        assert fkref.narrow_f16_f64(mid) == (lo if lo % 2 == 0 else lo + 1)
        up = struct.unpack("<d", struct.pack("<Q", struct.unpack("<Q", struct.pack("<d", mid))[0] + 1))[0]
        down = struct.unpack("<d", struct.pack("<Q", struct.unpack("<Q", struct.pack("<d", mid))[0] - 1))[0]
        assert fkref.narrow_f16_f64(up) == lo + 1
        assert fkref.narrow_f16_f64(down) == lo
        assert fkref.narrow_f16_f64(-mid) == 0x8000 | (lo if lo % 2 == 0 else lo + 1)


def test_simd_sums_are_pairwise_neighbours_first(golden):
    g = golden("numerics.json")["simd_pairwise"]
    lanes = [2.0**24] + [1.0] * 31
    assert fkref.simd_sum(lanes) == np.float32(g["cases"][0]["f32"])
    # In lane order every 1 rounds away.
    acc = np.float32(0)
    for v in lanes:
        acc = np.float32(acc + np.float32(v))
    assert acc == np.float32(2.0**24)
    lanes = [0.0] * 32
    lanes[0] = 2.0**24
    lanes[16] = lanes[17] = 1.0
    assert fkref.simd_sum(lanes) == np.float32(g["cases"][1]["f32"])


def test_reductions(golden):
    g = golden("numerics.json")["reduce"]
    for parts, want in zip(g["split_order"]["partials"], g["split_order"]["want"]):
        assert fkref.combine_splits(parts) == np.float32(want)
    t = g["max_of_thread_index"]
    assert fkref.tg_reduce_max(np.arange(t["threads"], dtype=np.float32), t["width"]) == np.float32(t["want"])
    neg = fkref.tg_reduce_sum(np.full(256, -0.0, np.float32), 32)
    pos = fkref.tg_reduce_sum(np.zeros(256, np.float32), 32)
    assert math.copysign(1, neg) == -1 and math.copysign(1, pos) == 1


def test_exp_is_binary64_rounded_once(golden):
    for x, want in golden("numerics.json")["transcendentals"]["exp_f32"]:
        assert f32_bits(fkref.lib().fkref_exp(f32_of(int(x, 16)))) == int(want, 16)


def test_min_max_are_minimum_and_maximum_number():
    """InterpTest.hs:167-175: a NaN gives way; -0 below +0."""
    snan = f32_of(0x7F800001)
    assert fkref.lib().fkref_max(1.0, snan) == 1.0
    assert fkref.lib().fkref_max(snan, 1.0) == 1.0
    assert f32_bits(fkref.lib().fkref_max(0.0, -0.0)) == 0
    assert f32_bits(fkref.lib().fkref_min(0.0, -0.0)) == 0x80000000
    assert f32_bits(fkref.lib().fkref_max(f32_of(0x7FC00001), f32_of(0xFF800001))) == 0x7FC00000


@pytest.mark.parametrize("width", [8, 32, 64])
def test_tg_reduce_sum_is_the_sum_of_slots(width):
    """Closed form: on integers the reduction is exact, whatever its order."""
    v = np.arange(256, dtype=np.float32)
    assert fkref.tg_reduce_sum(v, width) == np.float32(sum(range(256)))
