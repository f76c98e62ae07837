"""The prefill path on the host: the vectorised f64 evaluator pinned to the
exact one, and the lowering of a step of many rows (furykernel_amd/prefill.py)."""

import dataclasses

import numpy as np
import pytest

from furykernel_amd.layout import pack, pair, unpack
from furykernel_amd.lower import LoweringError
from furykernel_amd.prefill import check_rows, lower_prefill, weight_image
from furykernel_amd.program.check import check_program
from furykernel_amd.program.decoder import ONE_B_PREFILL, SMALL_PREFILL, TINY, decoder_step
from furykernel_amd.program.plan import PlanOptions, plan
from oracle.eval import Bindings, evaluate, evaluate_fast


def tiny_rows_bindings(checked, rows, seed=11):
    rng = np.random.default_rng(seed)
    weights = {}
    for src in checked.program.sources:
        if type(src.kind).__name__ == "SWeight":
            n = int(np.prod(src.kind.dims))
            weights[src.name] = 1 + 0.1 * rng.standard_normal(n) if len(src.kind.dims) == 1 else \
                0.1 * rng.standard_normal(n)
    caches = {}
    for src in checked.program.sources:
        if type(src.kind).__name__ == "SCache":
            lay = src.kind.layout
            caches[src.name] = {s: np.zeros(lay.kv_heads * lay.length * lay.head_dim) for s in range(lay.slots)}
    return Bindings(rows, inputs={"x": rng.standard_normal((rows, TINY.d_model)).tolist()}, weights=weights,
                    row_ints={"position": [[p] for p in range(rows)], "slot": [[0]] * rows}, caches=caches)


def test_fast_evaluator_agrees_with_the_exact_one_over_several_rows():
    """Six rows of one sequence at positions 0..5, causal: the two evaluators
    differ only in the order of each binary64 sum."""
    checked = check_program(decoder_step(TINY, embed=False))
    b = tiny_rows_bindings(checked, 6)
    ex, fa = evaluate(checked, b), evaluate_fast(checked, b)
    want = np.array(ex.outputs["logits"])
    got = fa.outputs["logits"]
    assert np.max(np.abs(got - want)) <= 1e-12 * np.max(np.abs(want))
    for name, units in ex.caches.items():
        assert np.max(np.abs(fa.caches[name][0] - units[0])) <= 1e-12 * max(1e-300, np.max(np.abs(units[0])))
    assert [int(t[0]) for t in ex.outputs["token"]] == [int(t) for t in fa.outputs["token"][:, 0]]


def small_lowered(seq_rows=128, seqs=2, **kw):
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=seq_rows, **kw))
    return c, lower_prefill(c, plan(PlanOptions(sequence_rows=seq_rows), c), seqs * seq_rows)


def test_prefill_lowering_of_the_small_decoder():
    _, low = small_lowered()
    entries = [l.entry for l in low.launches]
    norm = "fk_prefill_norm_pack"     # rows of 256: the two-pass kernel
    # the QKV GEMM RoPEs and stores in its epilogue: no RoPE launch, no f32 q, k, v
    # f16 rings, no staged rows: the attention loads its blocks straight into LDS
    per_layer = [norm, "fk_gemm_f16_qkv_rope", "fk_prefill_attend_f16_g2",
                 "fk_gemm_f16_add", norm, "fk_gemm_f16_silu_mul", "fk_gemm_f16_add"]
    # the head's GEMM leaves the greedy token's keys, 128 columns a key
    assert entries == ["fk_prefill_gather"] + per_layer * 2 + [norm, "fk_gemm_f16_store_keys",
                                                               "fk_prefill_argmax_keys"]
    head, token = low.launches[-2:]
    assert head.bind["keys"] == token.bind["keys"] and head.bind["c0"] == "value:logits"
    assert token.params == {"rows": 256, "parts": SMALL_PREFILL.vocab // 128}
    assert low.buffers[head.bind["keys"]].dtype == "u64"
    assert low.buffers[head.bind["keys"]].count == 256 * SMALL_PREFILL.vocab // 128
    qkv = low.launches[2]
    assert qkv.params["first_col"] == [0, 512, 768, 1024] and qkv.groups == 1 * 4
    att = low.launches[3]
    assert att.entry == "fk_prefill_attend_f16_g2" and att.threads == 128 and att.groups == (256 // 32) * 4
    assert (qkv.bind["c0"], qkv.bind["c1"], qkv.bind["c2"]) == (att.bind["qr"], att.bind["kc"], att.bind["vc"])
    assert (qkv.params["kv_heads"], qkv.params["length"], qkv.params["slots"]) == (4, 256, 2)
    assert not any(b.startswith(("value:l0_q", "value:l0_k", "value:l0_v")) for b in low.buffers)
    silu = low.launches[6]
    assert silu.bind["b0"] == "pair:l0_gate_proj|l0_up_proj" and silu.bind["c0"] == "tiled:l0_act"
    assert low.launches[7].bind["a"] == "tiled:l0_act"
    # the o projection reads the attention's tiled output, adds the gathered rows
    o = low.launches[4]
    assert o.bind["a"] == "tiled:l0_attn" and o.bind["r0"] == "value:x0"


def test_prefill_keeps_the_rope_launch_when_only_some_pairs_turn():
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128, rope_rotated=16))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256)
    entries = [l.entry for l in low.launches]
    assert "fk_prefill_rope_store" in entries and "fk_gemm_f16_qkv_rope" not in entries


def test_prefill_lowering_of_the_1b_decoder():
    c = check_program(decoder_step(ONE_B_PREFILL, name="prefill", position_bound=2048))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=2048), c), 8192)
    assert len(low.launches) == 1 + 16 * 7 + 3
    gu = [l for l in low.launches if l.entry == "fk_gemm_f16_silu_mul"][0]
    assert gu.groups == 32 * (8192 // 128)
    att = [l for l in low.launches if l.entry.startswith("fk_prefill_attend")][0]
    assert att.entry == "fk_prefill_attend_f16_g4" and att.threads == 256 and att.groups == 256 * 8
    assert low.buffers["cache:l0_k_cache"].count == 4 * 8 * 4096 * 64
    assert low.launches[1].entry == "fk_prefill_norm_pack_w2048"   # the one-pass norm of rows of 2048


def test_staged_stores_lower_to_staging_rows_reads_and_lands():
    """Positions up to the ring's length leave no room for a step's rows
    (Plan.hs:41-50): the plan stages the stores, the QKV epilogue writes the
    staging rows, the attention reads them, and the combine step lands them."""
    from furykernel_amd import kernels as K, runtime
    from furykernel_amd.engine import check_launch, params_struct
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill"))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256, run_rows=128)
    entries = [l.entry for l in low.launches]
    assert entries.count("fk_prefill_land") == SMALL_PREFILL.layers
    qkv = [l for l in low.launches if l.entry == "fk_gemm_f16_qkv_rope"]
    att = [l for l in low.launches if l.entry.startswith("fk_prefill_attend")]
    lands = [l for l in low.launches if l.entry == "fk_prefill_land"]
    for q, a, land in zip(qkv, att, lands):
        assert q.params["staged"] == 1 and q.bind["c1"].startswith("staged:") and q.bind["c2"].startswith("staged:")
        assert a.params["staged"] == 1 and a.params["run_rows"] == 128
        assert (a.bind["ks"], a.bind["vs"]) == (q.bind["c1"], q.bind["c2"])
        assert (land.bind["ks"], land.bind["vs"], land.bind["kc"], land.bind["vc"]) == \
            (a.bind["ks"], a.bind["vs"], a.bind["kc"], a.bind["vc"])
        assert entries.index("fk_prefill_land", entries.index(a.entry)) > entries.index(a.entry)
    assert low.buffers["staged:l0_k_cache"].count == 256 * SMALL_PREFILL.kv_heads * 64
    # every launch through the engine's and the launch table's checks on the host
    at, addr = 1 << 40, {}
    for name, spec in low.buffers.items():
        addr[name] = at
        at += (spec.nbytes + 4095) // 4096 * 4096
    for L in low.launches:
        check_launch(L, low.buffers)
        spans = [(0, 0) if L.bind.get(b) is None else (addr[L.bind[b]], low.buffers[L.bind[b]].nbytes)
                 for b in K.ABIS[L.entry].buffers]
        runtime.launch_check(L.entry, L.groups, L.threads, L.lds_bytes, spans, params_struct(L))
    # in place, nothing is staged
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256, run_rows=128)
    assert "fk_prefill_land" not in [l.entry for l in low.launches]
    assert not any(n.startswith("staged:") for n in low.buffers)
    with pytest.raises(LoweringError, match="runs of 96"):
        lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256, run_rows=96)


def test_prefill_refuses_what_its_kernels_do_not_take():
    with pytest.raises(LoweringError):   # rows not a multiple of 256
        c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128))
        lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 128)
    with pytest.raises(LoweringError):   # anchors narrower than a tile
        c = check_program(decoder_step(dataclasses.replace(TINY, weight_type="f16"), name="prefill", position_bound=8))
        lower_prefill(c, plan(PlanOptions(sequence_rows=8), c), 256)


def test_weight_images_are_the_layouts():
    c, low = small_lowered()
    rng = np.random.default_rng(3)
    g = rng.standard_normal((512, 256)).astype(np.float16)
    u = rng.standard_normal((512, 256)).astype(np.float16)
    q = rng.standard_normal((512, 256)).astype(np.float16)
    img = weight_image(low, "pair:l0_gate_proj|l0_up_proj", {"l0_gate_proj": g, "l0_up_proj": u})
    back = unpack(img, 1024, 256)
    assert np.array_equal(back[:128], g[:128]) and np.array_equal(back[128:256], u[:128])
    assert np.array_equal(weight_image(low, "tiled:l0_q_proj", {"l0_q_proj": q}), pack(q))


def test_check_rows_takes_blocks_of_one_sequence():
    pos = np.tile(np.arange(64), 2)
    check_rows(pos, np.repeat([0, 1], 64))
    with pytest.raises(LoweringError):   # sequences of 16 rows: a block of 32 spans two
        check_rows(np.tile(np.arange(16), 8), np.repeat(np.arange(8), 16))
    with pytest.raises(LoweringError):   # a block's rows from two sequences
        check_rows(pos, np.arange(128) % 2)
    with pytest.raises(LoweringError):
        bad = pos.copy()
        bad[5] = 7
        check_rows(bad, np.repeat([0, 1], 64))


def _windowed_attention_program(window):
    from furykernel_amd.program.build import program
    from furykernel_amd.program.graph import AttnSpec, F32, Ring, RopeSpec, whole_row

    def body(b):
        pos = b.row_ints("position", 1, 16)
        slot = b.row_ints("slot", 1, 2)
        x = b.input("x", whole_row(32), F32)
        wq = b.weight("wq", [32, 32], F32)
        wk = b.weight("wk", [16, 32], F32)
        wv = b.weight("wv", [16, 32], F32)
        kc = b.cache("kc", Ring(2, 2, 16, 8), "f16")
        vc = b.cache("vc", Ring(2, 2, 16, 8), "f16")
        q = b.rope("qr", RopeSpec(10000.0, 4), pos, b.linear("q", wq, 8, x))
        k = b.rope("kr", RopeSpec(10000.0, 4), pos, b.linear("k", wk, 8, x))
        b.kv_store("sk", kc, pos, slot, k)
        b.kv_store("sv", vc, pos, slot, b.linear("v", wv, 8, x))
        b.output("o", b.attend("o", AttnSpec(4, 2, 8, window, 0.35), q, kc, vc, pos, slot))
    return program("windowed", body)


@pytest.mark.parametrize("window", [None, 3])
def test_fast_evaluator_agrees_over_interleaved_sequences_and_windows(window):
    """Two sequences' rows interleaved (slot 1's rows between slot 0's), GQA 2,
    with and without a window of 3: the by-sequence masked attention of the
    fast evaluator is the exact evaluator's per-row sums."""
    checked = check_program(_windowed_attention_program(window))
    rng = np.random.default_rng(5)
    rows = 10
    slots = [0, 1, 0, 1, 1, 0, 0, 1, 0, 1]
    positions = [0, 0, 1, 1, 2, 2, 3, 3, 4, 4]
    weights = {"wq": rng.standard_normal(32 * 32), "wk": rng.standard_normal(16 * 32),
               "wv": rng.standard_normal(16 * 32)}
    caches = {n: {s: rng.standard_normal(2 * 16 * 8) for s in range(2)} for n in ("kc", "vc")}
    b = Bindings(rows, inputs={"x": rng.standard_normal((rows, 32)).tolist()}, weights=weights,
                 row_ints={"position": [[p] for p in positions], "slot": [[s] for s in slots]}, caches=caches)
    ex, fa = evaluate(checked, b), evaluate_fast(checked, b)
    want = np.array(ex.outputs["o"])
    assert np.max(np.abs(fa.outputs["o"] - want)) <= 1e-12 * np.max(np.abs(want))


def prefill_head(cap=None):
    """A head of many rows: RMSNorm, the logits over f16 weights, an optional
    softcap, the greedy token."""
    from furykernel_amd.program.build import program
    from furykernel_amd.program.graph import F16, F32, whole_row

    def body(b):
        x = b.input("x", whole_row(256))
        norm = b.weight("final_norm", [256], F32)
        embed = b.weight("embed", [512, 256], F16)
        logits = b.linear("logits", embed, 0, b.rmsnorm("normed", 1e-6, norm, 1, x))
        out = logits if cap is None else b.softcap("capped", cap, logits)
        b.output("logits", out)
        b.output("token", b.argmax("token", out))
    return check_program(program("prefill_head", body))


def test_the_token_folds_into_the_heads_gemm_only_without_a_softcap():
    plain = prefill_head()
    low = lower_prefill(plain, plan(PlanOptions(), plain), 512)
    assert [l.entry for l in low.launches][-2:] == ["fk_gemm_f16_store_keys", "fk_prefill_argmax_keys"]
    assert low.launches[-1].params == {"rows": 512, "parts": 4}
    # a softcap between the logits and the token: the token reads the capped
    # rows, so the plain argmax stays
    capped = prefill_head(30.0)
    low = lower_prefill(capped, plan(PlanOptions(), capped), 512)
    assert [l.entry for l in low.launches][-3:] == ["fk_gemm_f16_store", "fk_prefill_softcap", "fk_prefill_argmax"]
    assert low.launches[-1].bind["x"] == low.launches[-2].bind["y"]


def test_paged_pools_lower_to_the_paged_qkv_epilogue_and_attention():
    """Caches as paged pools (Graph.hs:144-152): the QKV GEMM's epilogue
    stores through each row's block table, the attention reads through it."""
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128, paging=(64, 8)))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256, run_rows=128)
    entries = [l.entry for l in low.launches]
    # f16 pools: the attention's blocks straight into LDS
    assert entries.count("fk_gemm_f16_qkv_rope_paged") == entries.count("fk_prefill_attend_paged_f16_g2") == 2
    assert "fk_prefill_rope_store" not in entries and "fk_prefill_attend_g2" not in entries
    qkv, att = low.launches[2], low.launches[3]
    assert qkv.bind["table"] == att.bind["table"] == "ints:blocks"
    assert low.buffers["ints:blocks"].count == 256 * 4
    assert (qkv.bind["c1"], qkv.bind["c2"]) == (att.bind["kc"], att.bind["vc"])
    assert low.buffers[att.bind["kc"]].count == 8 * 4 * 64 * 64
    for L in (qkv, att):
        assert (L.params["block_size"], L.params["table_len"], L.params["blocks"], L.params["length"]) == (64, 4, 8, 256)


def test_paged_pools_with_rope_on_some_pairs_store_through_the_rope_kernel():
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128, paging=(64, 8), rope_rotated=16))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256, run_rows=128)
    entries = [l.entry for l in low.launches]
    assert entries.count("fk_prefill_rope_store_paged") == 2 and "fk_gemm_f16_qkv_rope_paged" not in entries
    rs = low.launches[entries.index("fk_prefill_rope_store_paged")]
    assert rs.bind["table"] == "ints:blocks" and rs.params["rotated"] == 16
    assert (rs.params["block_size"], rs.params["table_len"], rs.params["blocks"]) == (64, 4, 8)


def test_a_pool_has_room_for_any_steps_rows():
    # Plan.hs:276-281 stages only ring stores: positions up to the table's
    # reach store in place
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", paging=(64, 8)))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256, run_rows=128)
    assert not any(l.entry == "fk_prefill_land" for l in low.launches)
