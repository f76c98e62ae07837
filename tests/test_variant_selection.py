"""Variant spaces and selections (furykernel_amd/variant.py, selection.py,
tuning.py) on the CPU: what the reference's tests hold of them
(test/Test/FuryKernel/VariantTest.hs, SelectionTest.hs) restated over this
target's GEMV families — points and axis keys, names that split back, the
spaces refused, pruning and why, duplicates, the selection format and
everything validation refuses — and the lowering's use of a pick, which
changes no bit the step computes."""

import dataclasses

import numpy as np
import pytest

from furykernel_amd import selection as S
from furykernel_amd import tuning as T
from furykernel_amd import variant as V

PROFILE = V.Profile(2)


def small_space():
    """The f32 standalone GEMV at n 8 × k 256, batches 1 and 2, on a GPU of 2 CUs."""
    return dataclasses.replace(T.gemv_space("f32"),
                               shapes=[(("n", 8), ("k", 256), ("m", 1)), (("n", 8), ("k", 256), ("m", 2))])


def test_points_first_axis_slowest():
    axes = [V.Axis("a", "a", (1, 2)), V.Axis("b", "b", (3, 4, 5), True)]
    assert [V.axis_key(p) for p in V.points(axes)] == ["a1_b3", "a1_b4", "a1_b5", "a2_b3", "a2_b4", "a2_b5"]


def test_axis_keys_read_back_and_say_what_is_wrong():
    axes = T.GEMV_AXES
    assert V.parse_axis_key(axes, "r2_t128") == (("r", 2), ("t", 128))
    for key, msg in [("r2", "The axis key r2 has 1 parts for 2 axes."),
                     ("r2_x128", "The axis key r2_x128 has x128 where threads (t) belongs."),
                     ("r3_t128", "The axis key r3_t128 gives rows_per_wave 3, which is not one of its values."),
                     ("r01_t128", "The axis key r01_t128 writes rows_per_wave 1 as 01.")]:
        with pytest.raises(ValueError) as e:
            V.parse_axis_key(axes, key)
        assert str(e.value) == msg
    assert V.parse_axis_key([], "") == ()


def test_names_split_back():
    space = small_space()
    shape = space.shapes[0]
    assert V.variant_name(space, shape, (("r", 1), ("t", 64))) == "gemv_f32_n8_k256_m1_x_r1_t64"
    assert V.variant_name(dataclasses.replace(space, axes=[]), shape, ()) == "gemv_f32_n8_k256_m1"
    assert V.variant_name(space, (), (("r", 1), ("t", 64))) == "gemv_f32_x_r1_t64"
    for s in space.shapes:
        for p in V.points(space.axes):
            assert V.variant_of_name(space, V.variant_name(space, s, p)) == (s, p)
    assert V.variant_of_name(space, "gemv_f32_n8_k256_m1_x_r3_t64") is None

    def bucket(r):
        return r.startswith("m") and r[1:].isdigit()
    assert V.split_join(bucket, "model_embed_x_s0_x_x_m1") == ("model_embed_x_s0_x", "m1")
    assert V.split_join(bucket, "a_x_b_x_m16") == ("a_x_b", "m16")
    assert V.split_join(bucket, "a_x_b") is None


def test_spaces_whose_names_would_not_read_back():
    space = small_space()
    assert V.check_space(space) == []
    assert V.check_space(dataclasses.replace(space, family="gemv_x_wide")) == [
        "The family gemv_x_wide holds _x_, which joins a variant's name to its axis key."]
    assert V.check_space(dataclasses.replace(space, axes=T.GEMV_AXES + [V.Axis("unused", "r", (1,))])) == [
        "The axes rows_per_wave and unused share the prefix r."]
    assert V.check_space(dataclasses.replace(space, axes=[V.Axis("rows", "r_", (1,)), V.Axis("none", "n", ())])) == [
        "The axis rows's prefix \"r_\" is not lowercase letters.", "The axis none has no values."]
    sh = space.shapes[0]
    assert V.check_space(dataclasses.replace(space, shapes=[(("n", 8), ("k_", 256), ("m", 1)),
                                                            (("n", 8), ("n", 16), ("m", 1)), sh, sh])) == [
        "The class n8_k_256_m1's dimension \"k_\" is not lowercase letters.",
        "The class n8_n16_m1 gives n 2 times.",
        "The class n8_k256_m1 is given 2 times."]
    assert V.check_space(dataclasses.replace(space, batch=["mm"])) == [
        "The batch dimension mm is not a dimension of the class n8_k256_m1.",
        "The batch dimension mm is not a dimension of the class n8_k256_m2."]


def describe(o):
    if isinstance(o, V.Kept):
        return f"kept, {o.variant.groups} groups"
    if isinstance(o, V.IllegalOutcome):
        return "illegal"
    if isinstance(o, V.Indivisible):
        return f"indivisible: {o.reasons}"
    if isinstance(o, V.TooFewGroups):
        return f"too few: {o.groups} groups"
    return f"same as {V.axis_key(o.point)}"


def test_pruning_and_why():
    space = small_space()
    shape = space.shapes[0]

    def outcome(key):
        return describe(V.consider(PROFILE, space, shape, V.parse_axis_key(space.axes, key)))
    assert outcome("r1_t64") == "kept, 8 groups"
    assert outcome("r2_t64") == "kept, 4 groups"
    assert outcome("r4_t64") == "too few: 2 groups"
    assert outcome("r4_t256") == "indivisible: ['n 8 is not a multiple of the 16 rows of a threadgroup.']"
    # the launch check's verdict: k not a multiple of the pack width is refused
    odd = dataclasses.replace(space, shapes=[(("n", 8), ("k", 258), ("m", 1))])
    o = V.consider(PROFILE, odd, odd.shapes[0], (("r", 1), ("t", 64)))
    assert isinstance(o, (V.IllegalOutcome, V.Indivisible))


def test_duplicates_the_first_point_of_a_launch_stays():
    space = small_space()
    twice = dataclasses.replace(space, axes=space.axes + [V.Axis("unused", "u", (1, 2))])
    shape = space.shapes[0]
    outcomes = V.enumerate_class(PROFILE, twice, shape)
    kept = [V.axis_key(v.point) for v in V.variants(PROFILE, space, shape)]
    assert [V.axis_key(p) for p, o in outcomes if isinstance(o, V.Kept)] == [k + "_u1" for k in kept]
    assert [(V.axis_key(p), V.axis_key(o.point)) for p, o in outcomes if isinstance(o, V.SameAs)] == \
        [(k + "_u2", k + "_u1") for k in kept]


def written(ps, family="gemv_f32", target="MI355X", profile=PROFILE):
    return S.Selection(family, target, profile, {c: S.Pick(a, h) for c, a, h in ps})


def hash_of(space, c, a):
    shape = [s for s in space.shapes if V.shape_key(s) == c][0]
    o = V.consider(PROFILE, space, shape, V.parse_axis_key(space.axes, a))
    return o.variant.ir_hash if isinstance(o, V.Kept) else 0


def test_the_format_classes_in_key_order():
    text = S.render(written([("n8_k256_m2", "r1_t64", 0x0123456789abcdef), ("n8_k256_m1", "r2_t64",
                                                                             0xfedcba9876543210)]))
    assert text == "\n".join([
        "{", '  "format": "furykernel-selection",', '  "version": 1,', '  "family": "gemv_f32",',
        '  "target": "MI355X",', '  "profile": {', '    "cores": 2', "  },", '  "classes": {',
        '    "n8_k256_m1": {', '      "variant": "r2_t64",', '      "ir_hash": "0xfedcba9876543210"', "    },",
        '    "n8_k256_m2": {', '      "variant": "r1_t64",', '      "ir_hash": "0x0123456789abcdef"', "    }",
        "  }", "}", ""])
    s = written([("n8_k256_m1", "r1_t64", 1), ("n8_k256_m2", "r2_t64", 2 ** 64 - 1)])
    assert S.parse(S.render(s)) == s


def field(name, value):
    base = [("format", '"furykernel-selection"'), ("version", "1"), ("family", '"gemv_f32"'),
            ("target", '"MI355X"'), ("profile", '{"cores": 2}'), ("classes", "{}")]
    return "{" + ", ".join(f'"{k}": {value if k == name else v}' for k, v in base) + "}"


@pytest.mark.parametrize("text,problem", [
    ("[]", "A selection is a JSON object."),
    (field("format", '"other"'), "The format is other, not furykernel-selection."),
    (field("version", "2"), "Version 2 of the format; this reads version 1."),
    ('{"format": "furykernel-selection", "version": 2, "extra": 1}', "Version 2 of the format; this reads version 1."),
    (field("classes", '{"n8_k256_m1": "r1_t64"}'), "The field classes has the wrong type."),
    (field("classes", '{"n8_k256_m1": {"variant": "r1_t64", "ir_hash": "0x12"}}'),
     "The field classes has the wrong type."),
    (field("profile", '{"cores": -1}'), "The field profile has the wrong type."),
    ('{"format": "furykernel-selection", "version": 1, "extra": 1}', "An unknown field: extra."),
    ('{"format": "furykernel-selection", "version": 1}', "The field family is missing."),
])
def test_the_format_is_checked(text, problem):
    with pytest.raises(S.SelectionError) as e:
        S.parse(text)
    assert e.value.problems == [problem]


def test_a_valid_selection_gives_a_variant_per_class():
    space = small_space()
    sel = written([(c, a, hash_of(space, c, a)) for c, a in (("n8_k256_m1", "r1_t64"), ("n8_k256_m2", "r2_t64"))])
    got = S.validate(PROFILE, space, sel)
    assert [(V.shape_key(v.shape), V.axis_key(v.point)) for v in got] == [("n8_k256_m1", "r1_t64"),
                                                                        ("n8_k256_m2", "r2_t64")]


def test_a_pick_is_the_launch_it_was_picked_as_on_the_profile_it_was_picked_on():
    space = small_space()
    stale = written([("n8_k256_m1", "r1_t64", 1), ("n8_k256_m2", "r2_t64", hash_of(space, "n8_k256_m2", "r2_t64"))])
    with pytest.raises(S.SelectionError) as e:
        S.validate(PROFILE, space, stale)
    now = hash_of(space, "n8_k256_m1", "r1_t64")
    assert e.value.problems == [f"gemv_f32_n8_k256_m1_x_r1_t64 was picked as the kernel of IR hash "
                                f"0x0000000000000001, and is now 0x{now:016x}."]
    good = written([(c, a, hash_of(space, c, a)) for c, a in (("n8_k256_m1", "r1_t64"), ("n8_k256_m2", "r2_t64"))])
    with pytest.raises(S.SelectionError) as e:
        S.validate(V.Profile(1), space, good)
    assert "The selection was made for a GPU of 2 cores, not 1." in e.value.problems


def test_everything_else_validation_refuses():
    space = small_space()
    with pytest.raises(S.SelectionError) as e:
        S.validate(PROFILE, space, S.Selection("gemm", "T64", PROFILE, {}))
    assert e.value.problems == ["The selection is for the family gemm, not gemv_f32.",
                                "The selection is for the target T64, not MI355X.",
                                "No variant for the class n8_k256_m1.", "No variant for the class n8_k256_m2."]
    sel = written([("n8_k256_m1", "r4_t256", 0), ("n8_k256_m2", "r4_t64", 0), ("n9_k256_m1", "r1_t64", 0)])
    with pytest.raises(S.SelectionError) as e:
        S.validate(PROFILE, space, sel)
    assert e.value.problems == [
        "The class n9_k256_m1 is not one of the family's.",
        "gemv_f32_n8_k256_m1_x_r4_t256 does not divide its class: n 8 is not a multiple of the 16 rows of a "
        "threadgroup.",
        "gemv_f32_n8_k256_m2_x_r4_t64 launches 2 threadgroups, fewer than twice the 2 cores."]
    with pytest.raises(S.SelectionError) as e:
        S.validate(PROFILE, space, written([("n8_k256_m1", "r1_t64", 0), ("n8_k256_m2", "r1_q64", 0)]))
    assert "The class n8_k256_m2's axis key r1_q64 has q64 where threads (t) belongs." in e.value.problems


def test_the_batch_sizes_of_a_class_share_the_order_of_its_reductions():
    """Were threads an order axis, two batches of a class picking different
    thread counts would be refused."""
    space = small_space()
    ordered = dataclasses.replace(space, axes=[T.GEMV_AXES[0], dataclasses.replace(T.GEMV_AXES[1], order=True)])
    sel = written([(c, a, hash_of(ordered, c, a)) for c, a in (("n8_k256_m1", "r1_t64"), ("n8_k256_m2", "r1_t128"))])
    with pytest.raises(S.SelectionError) as e:
        S.validate(PROFILE, ordered, sel)
    assert e.value.problems == ["The classes n8_k256_m1 and n8_k256_m2 differ only in batch size, and order "
                                "reductions differently: t64 against t128."]
    # the families here have no order axis: any picks of the two batches pass
    S.validate(PROFILE, space, written([(c, a, hash_of(space, c, a)) for c, a in
                                        (("n8_k256_m1", "r1_t64"), ("n8_k256_m2", "r1_t128"))]))


def test_the_step_family_keeps_the_classes_that_fill_the_gpu():
    space = T.step_space("f16")
    prof = V.Profile(256)
    for shape in space.shapes:
        kept = V.variants(prof, space, shape)
        assert kept and all(v.groups >= 512 for v in kept)
    # a 2048-row class cannot fill 512 threadgroups of 8 wavefronts
    small = T.step_space("f16", [(2048, 2048)])
    assert V.variants(prof, small, small.shapes[0]) == []
    # no step kernel of two rows a block at k 8192
    wide = T.step_space("f16", [(16384, 8192)])
    o = V.consider(prof, wide, wide.shapes[0], (("r", 2), ("g", 2)))
    assert isinstance(o, V.IllegalOutcome)


def test_committed_selections_validate():
    """Every selection committed under furykernel_amd/selections/ parses and
    validates against its family's space on this target's 256 CUs, every
    pick still the launch it was timed as: a stale pick (its kernel's code
    or its launch changed after tuning) fails here, so the committed picks
    are the ones the lowering and the bench use."""
    picks = T.validated(256)
    assert T.chooser_problems == {}
    assert sorted(picks) == sorted(s.family for s in T.spaces(256))


def test_a_pick_goes_stale_only_with_its_own_kernel(tmp_path):
    """A pick's hash covers its entry's defining header and what that
    includes: another kernel's header (the prefill's) leaves the step GEMV's
    hash as it is; its own header changes it."""
    from furykernel_amd import manifest as M
    entry = "fk_step_gemv_f16_k2048_r1_p0_e0"
    before = M.entry_source_hash(entry)
    assert "fk_prefill.h" not in M._include_closure("fk_step_gemv.h")
    assert "fk_step_gemv.h" in M._include_closure("fk_step_gemv.h")
    saved = M.KERNELS_DIR
    fake = tmp_path / "kernels"
    fake.mkdir()
    for f in saved.iterdir():
        if f.is_file():
            (fake / f.name).write_bytes(f.read_bytes())
    try:
        M.KERNELS_DIR = fake
        (fake / "fk_prefill.h").write_text((fake / "fk_prefill.h").read_text() + "\n// another kernel's change\n")
        assert M.entry_source_hash(entry) == before
        (fake / "fk_step_gemv.h").write_text((fake / "fk_step_gemv.h").read_text() + "\n// its own change\n")
        assert M.entry_source_hash(entry) != before
    finally:
        M.KERNELS_DIR = saved


# The lowering's use of a pick -------------------------------------------------

def test_a_pick_reshapes_the_launch_and_changes_no_bit():
    from furykernel_amd.lower import lower_plan
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import ONE_B, TINY, decoder_step
    from furykernel_amd.program.plan import PlanOptions, plan
    from test_lowering import seeded

    c = check_program(decoder_step(ONE_B, embed=True))
    pl = plan(PlanOptions(store_gelus=True), c)
    base = lower_plan(c, pl)
    picked = lower_plan(c, pl, choose=lambda L: (2, 3) if T.step_class(L) == (("n", 16384), ("k", 2048), ("m", 1))
                        else None)
    gu = [i for i, L in enumerate(base.launches)
          if L.entry.startswith("fk_step_gemv") and T.step_class(L) == (("n", 16384), ("k", 2048), ("m", 1))]
    assert len(gu) == 16
    for i in gu:
        assert picked.launches[i].groups == 768 and base.launches[i].groups == 512
        assert picked.launches[i].entry == base.launches[i].entry  # the SiLU pair epilogue at 2 rows a block
    # one row a block under the pair epilogue: each row of gate, then of up,
    # a block of its own (twice the rows in blocks)
    one = lower_plan(c, pl, choose=lambda L: (1, 4))
    for i in gu:
        L = one.launches[i]
        assert L.entry == base.launches[i].entry.replace("_r2_", "_r1_") and L.params["blocks"] == 2 * 8192
        assert L.groups == 1024
    # a pick a launch cannot take (two rows a block at an input row of 8192,
    # the down projection's) is passed over
    down = [i for i, L in enumerate(base.launches) if "_k8192_" in L.entry]
    assert len(down) == 16
    two = lower_plan(c, pl, choose=lambda L: (2, 2))
    for i in down:
        assert two.launches[i].entry == base.launches[i].entry and two.launches[i].groups == base.launches[i].groups

    # the tiny step under every launch's (1, 4) and (2, 1) against the default: the same bits
    tiny = check_program(decoder_step(dataclasses.replace(TINY, context=32), embed=False))
    tp = plan(PlanOptions(), tiny)
    ref = seeded(lower_plan(tiny, tp), 3, 9)
    ref.run()
    changed = 0
    for pick in ((1, 4), (2, 1)):
        low = lower_plan(tiny, tp, choose=lambda L, pick=pick: pick)
        changed += sum(L.entry != R.entry or L.groups != R.groups for L, R in zip(low.launches, ref.lowered.launches))
        got = seeded(low, 3, 9)
        got.run()
        # every buffer but the greedy token's per-threadgroup candidates (one
        # a threadgroup of the logits' step) holds the same bits
        for name in low.buffers:
            if not name.startswith("argmax:"):
                assert np.array_equal(got.read(name).view(np.uint8), ref.read(name).view(np.uint8)), (pick, name)
        assert int(got.read("value:token")[0]) == int(ref.read("value:token")[0])
    assert changed > 0
