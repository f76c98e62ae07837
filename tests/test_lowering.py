"""The lowering of planned steps to launches, on the CPU: which launches a
decoder step becomes, and that the attention launch which folds in the KV
store before it computes, in the oracle's CPU target, exactly what the
plan's separate store and attention steps compute."""

import dataclasses
import zlib

import numpy as np
import pytest

from furykernel_amd.lower import LoweringError, lower_plan, rope_table
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import ONE_B, TINY, decoder_step
from furykernel_amd.program.plan import PlanOptions, plan
from oracle.cpu_target import CpuTarget

TINY32 = dataclasses.replace(TINY, context=32)


def lowered(dims, options=PlanOptions(), fuse=True, embed=False, layers=None, wide=False):
    checked = check_program(decoder_step(dims, embed=embed, layers=layers))
    return lower_plan(checked, plan(options, checked), fuse=fuse, wide=wide)


def seeded(low, seed, position, width=64):
    """A CPU target with every buffer the step reads drawn from a stream
    seeded by `seed` and the buffer's name: weights 0.02 N(0, 1) (norm gains 1), caches N(0, 1), inputs
    0.02 N(0, 1)."""
    cpu = CpuTarget(low, width)
    for name, spec in sorted(low.buffers.items()):
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])  # a buffer's draws its own
        buf = cpu.buffers[name]
        if name.startswith("weight:"):
            if "norm" in name:
                buf[:] = 1
            else:
                buf[:] = (rng.standard_normal(spec.count) * 0.02).astype(buf.dtype)
        elif name.startswith("cache:"):
            buf[:] = rng.standard_normal(spec.count).astype(np.float16).view(buf.dtype)
        elif name.startswith("value:"):
            buf[:] = (rng.standard_normal(spec.count) * 0.02).astype(buf.dtype)
    for name, what in low.constants.items():
        if what[0] == "rope":
            cpu.write(name, rope_table(*what[1:]))
    cpu.write("ints:position", [position])
    return cpu


def test_a_1b_layer_in_wide_splits_is_five_launches():
    """The QKV GEMV with RoPE on its rows, the attention in wide splits with
    the KV store folded in, the O GEMV whose prologue combines the splits,
    gate/up, down."""
    low = lowered(ONE_B, embed=True, wide=True)
    entries = [launch.entry for launch in low.launches]
    assert len(entries) == 16 * 5 + 2
    assert entries[:5] == ["fk_step_gemv_f16_k2048_r1_p3_e0", "fk_step_attend_wide",
                           "fk_step_gemv_f16_k2048_r1_p5_e2", "fk_step_gemv_f16_k2048_r2_p1_e0",
                           "fk_step_gemv_f16_k8192_r1_p4_e1"]
    assert entries[5:10] == ["fk_step_gemv_f16_k2048_r1_p1_e0", "fk_step_attend_wide",
                             "fk_step_gemv_f16_k2048_r1_p5_e1", "fk_step_gemv_f16_k2048_r2_p1_e0",
                             "fk_step_gemv_f16_k8192_r1_p4_e1"]
    attend, o = low.launches[1], low.launches[2]
    assert attend.step == "s1_store+s2_attend"
    assert (attend.params["store"], attend.params["krope"]) == (1, 1)
    # 4096 positions in 8 splits of 512: 8 wavefronts of 64 positions
    assert (attend.params["splits"], attend.params["split"], attend.threads) == (8, 512, 512)
    assert attend.groups == ONE_B.kv_heads * attend.params["splits"]
    assert o.bind["src"] == attend.bind["partials"] and o.params["splits"] == 8 and o.params["head_dim"] == 64
    # The greedy token folds into the logits' GEMV step, then a token launch.
    head, token = low.launches[-2:]
    assert head.entry == "fk_step_gemv_f16_k2048_r2_p1_e4" and head.bind["arg"] == "argmax:token"
    assert low.buffers["argmax:token"].count == head.groups == token.params["slots"]
    assert token.entry == "fk_step_token" and token.bind["out"] == "value:token"


def test_a_1b_layer_is_six_launches():
    """The default, narrow splits: 32 splits of 128 positions, more than the
    GEMV step's combine prologue takes, so the combine is a launch."""
    low = lowered(ONE_B, embed=True)
    entries = [launch.entry for launch in low.launches]
    assert len(entries) == 16 * 6 + 2
    assert entries[:6] == ["fk_step_gemv_f16_k2048_r1_p3_e0", "fk_step_attend", "fk_step_combine",
                           "fk_step_gemv_f16_k2048_r1_p0_e2", "fk_step_gemv_f16_k2048_r2_p1_e0",
                           "fk_step_gemv_f16_k8192_r1_p4_e1"]
    assert low.launches[1].params["splits"] == 32
    head, token = low.launches[-2:]
    assert head.entry == "fk_step_gemv_f16_k2048_r2_p1_e4" and token.entry == "fk_step_token"


def test_a_stored_silu_mul_folds_into_the_gate_and_up_step():
    low = lowered(ONE_B, PlanOptions(store_gelus=True), embed=True)
    assert len(low.launches) == 16 * 6 + 2
    gu, down = low.launches[4], low.launches[5]
    assert gu.step.endswith("_act") and gu.params["epi_mode"] == 3 and gu.bind["epi_out"] == "value:l0_act"
    assert gu.entry == "fk_step_gemv_f16_k2048_r2_p1_e3" and gu.params["blocks"] == ONE_B.ffn
    assert down.entry == "fk_step_gemv_f16_k8192_r1_p0_e1" and down.bind["src"] == "value:l0_act"


def test_unfused_lowering_keeps_the_plans_steps():
    low = lowered(ONE_B, embed=True, fuse=False)
    assert [launch.entry for launch in low.launches[:7]] == [
        "fk_step_gemv_f16_k2048_r1_p3_e0", "fk_step_store", "fk_step_attend", "fk_step_combine",
        "fk_step_gemv_f16_k2048_r1_p0_e2", "fk_step_gemv_f16_k2048_r2_p1_e0", "fk_step_gemv_f16_k8192_r1_p4_e1"]
    assert low.launches[-1].entry == "fk_step_argmax"


@pytest.mark.parametrize("wide", [False, True], ids=["narrow", "wide"])
@pytest.mark.parametrize("position", [0, 5, 31])
@pytest.mark.parametrize("options", [PlanOptions(), PlanOptions(store_gelus=True)])
def test_fused_launches_compute_the_plans_steps(position, options, wide):
    """Each layer's KV store folded into its attention, its combine into the
    O GEMV step's prologue (and, when the plan stores the SiLU·mul, that
    light step folded into the gate/up GEMV step); the greedy token folded
    into the logits' step and a token launch.  Every buffer the fused step
    writes holds the same bits as the unfused step's."""
    fused, apart = lowered(TINY32, options, wide=wide), lowered(TINY32, options, fuse=False, wide=wide)
    per_layer = (2 if options.store_gelus else 1) + 1
    assert len(apart.launches) - len(fused.launches) == TINY32.layers * per_layer
    same_bits(fused, apart, 7, position)


def same_bits(fused, apart, seed, position):
    """Runs both lowerings from the same seeded buffers: the buffers the
    fused step writes hold the unfused step's bits, and the ones it no
    longer writes are only the combined attention rows its GEMV prologues
    keep in registers."""
    from test_bounds import written

    a, b = seeded(fused, seed, position), seeded(apart, seed, position)
    a.run()
    b.run()
    skipped = written(apart) - written(fused)
    combined = {L.bind["out"] for L in apart.launches if L.entry == "fk_step_combine"}
    assert skipped <= combined, skipped - combined
    assert set(apart.buffers) - set(fused.buffers) == skipped
    for name in apart.buffers:
        if name not in skipped:
            assert np.array_equal(a.read(name).view(np.uint8), b.read(name).view(np.uint8)), name


def test_every_lowered_entry_is_in_the_launch_table():
    from furykernel_amd.kernels import ABIS

    for dims, opts in [(ONE_B, PlanOptions()), (ONE_B, PlanOptions(store_gelus=True)), (TINY32, PlanOptions()),
                       (TINY32, PlanOptions(store_gelus=True))]:
        for fuse in (True, False):
            for launch in lowered(dims, opts, fuse=fuse, embed=True).launches:
                assert launch.entry in ABIS, launch.entry


def test_bf16_caches_fuse_the_same_way():
    dims = dataclasses.replace(TINY32, cache_elem="bf16")
    try:
        fused, apart = lowered(dims), lowered(dims, fuse=False)
    except (LoweringError, ValueError) as e:  # a program the gate refuses needs no lowering test
        pytest.skip(f"bf16 caches: {e}")
    same_bits(fused, apart, 9, 17)


def _residual_gather_program(table_type):
    from furykernel_amd.program.build import program
    from furykernel_amd.program.graph import F16, F32, whole_row

    def body(b):
        tokens = b.row_ints("tokens", 1, 16)
        table = b.weight("embed", [16, 64], table_type)
        s = b.input("s", whole_row(64), F32)
        w = b.weight("w", [64, 64], F16)
        x0 = b.gather("x0", table, tokens, 1.0)
        y = b.linear("y", w, 0, s)
        b.output("out", b.add("out", x0, y))
    return program("residual_gather", body)


def test_a_residual_gathered_from_a_table_of_another_type_is_gathered_apart():
    """The GEMV step's epilogue reads the gathered residual's table as the
    weights' element type: the same table in f16 lowers to the
    gathered-residual epilogue; an f32 table under f16 weights is refused
    there, so its gather is a launch of its own and the epilogue adds the
    stored row."""
    from furykernel_amd.program.graph import F16, F32
    ok = check_program(_residual_gather_program(F16))
    low = lower_plan(ok, plan(PlanOptions(), ok))
    assert [L.entry for L in low.launches] == ["fk_step_gemv_f16_k2048_r1_p0_e2"]
    apart = check_program(_residual_gather_program(F32))
    low = lower_plan(apart, plan(PlanOptions(), apart))
    assert [L.entry for L in low.launches] == ["fk_step_gather_f32", "fk_step_gemv_f16_k2048_r1_p0_e1"]
    assert low.launches[1].bind["res"] == low.launches[0].bind["y"]
