"""The programs of the reference's program-layer tests
(test/Test/FuryKernel/ProgramTest.hs), written with this repository's builder,
for the planner's and the evaluator's known answers."""

from __future__ import annotations

import math

from furykernel_amd.program.build import ProgramBuilder, program
from furykernel_amd.program.graph import (
    AttnSpec, CACHE_F16, F32, Paged, Reach, Ring, RopeSpec, Shape, U32, whole_row)


def layer(k_eq_v: bool = False):
    """ProgramTest.hs:488-557: hidden 32, four query heads of 8 over two KV
    heads, 8 experts of 16 of which a row takes 2."""
    hidden, eps = 32, 1e-6

    def body(b: ProgramBuilder):
        x = b.input("x", whole_row(hidden), F32)
        pos = b.row_ints("position", 1, 64)
        slot = b.row_ints("slot", 1, 2)
        pre_attn = b.weight("pre_attn_norm", [hidden])
        wq = b.weight("q_proj", [4 * 8, hidden])
        wk = b.weight("k_proj", [2 * 8, hidden])
        wv = b.weight("v_proj", [2 * 8, hidden])
        q_norm = b.weight("q_norm", [8])
        k_norm = b.weight("k_norm", [8])
        wo = b.weight("o_proj", [hidden, 4 * 8])
        post_attn = b.weight("post_attn_norm", [hidden])
        pre_mlp = b.weight("pre_mlp_norm", [hidden])
        gate_w = b.weight("gate_proj", [48, hidden])
        up_w = b.weight("up_proj", [48, hidden])
        down = b.weight("down_proj", [hidden, 48])
        post_mlp = b.weight("post_mlp_norm", [hidden])
        router_scale = b.weight("router_scale", [hidden])
        router = b.weight("router_proj", [8, hidden])
        expert_scale = b.weight("expert_scale", [8])
        pre_moe = b.weight("pre_moe_norm", [hidden])
        experts_gate_up = b.table("experts_gate_up", 8, [2 * 16, hidden])
        experts_down = b.table("experts_down", 8, [hidden, 16])
        post_moe = b.weight("post_moe_norm", [hidden])
        post_ffn = b.weight("post_ffn_norm", [hidden])
        scalar = b.weight("layer_scalar", [1])
        k_cache = b.cache("k_cache", Ring(2, 2, 12, 8))
        v_cache = b.cache("v_cache", Ring(2, 2, 12, 8))
        a = b.rmsnorm("attn_in", eps, pre_attn, 1, x)
        q = b.linear("q", wq, 8, a)
        k = b.linear("k", wk, 8, a)
        v = k if k_eq_v else b.linear("v", wv, 8, a)
        qn = b.rmsnorm("q_normed", eps, q_norm, 1, q)
        kn = b.rmsnorm("k_normed", eps, k_norm, 1, k)
        vn = b.rmsnorm("v_normed", eps, None, 1, v)
        qr = b.rope("q_rotated", RopeSpec(10000, 4), pos, qn)
        kr = b.rope("k_rotated", RopeSpec(10000, 4), pos, kn)
        b.kv_store("store_k", k_cache, pos, slot, kr)
        b.kv_store("store_v", v_cache, pos, slot, vn)
        o = b.attend("attended", AttnSpec(4, 2, 8, 6, 1), qr, k_cache, v_cache, pos, slot)
        out = b.linear("attn_out", wo, 0, o)
        out_normed = b.rmsnorm("attn_out_normed", eps, post_attn, 1, out)
        x1 = b.add("x1", x, out_normed)
        bb = b.rmsnorm("mlp_in", eps, pre_mlp, 1, x1)
        gate = b.linear("gate", gate_w, 0, bb)
        up = b.linear("up", up_w, 0, bb)
        r = b.rmsnorm("router_in", eps, router_scale, 1 / math.sqrt(32), x1)
        logits = b.linear("router_logits", router, 0, r)
        g = b.gelu_mul("mlp_act", gate, up)
        ids, ws = b.route("route", 2, expert_scale, logits)
        c = b.rmsnorm("moe_in", eps, pre_moe, 1, x1)
        d = b.linear("mlp_out", down, 0, g)
        gue = b.linear_routed("experts_gate_up_out", experts_gate_up, ids, c)
        ge = b.gated_gelu("experts_act", gue)
        de = b.linear_routed("experts_out", experts_down, ids, ge)
        h1 = b.rmsnorm("mlp_out_normed", eps, post_mlp, 1, d)
        s = b.combine_ranks("experts_sum", ws, de)
        h2 = b.rmsnorm("moe_out_normed", eps, post_moe, 1, s)
        hs = b.add("ffn_sum", h1, h2)
        f = b.rmsnorm("ffn_out", eps, post_ffn, 1, hs)
        x2 = b.add("x2_unscaled", x1, f)
        y = b.scale_by("x2", scalar, x2)
        b.output("x", y)

    return program("layer_kv" if k_eq_v else "layer", body)


def head_program():
    """ProgramTest.hs:643-653."""
    def body(b):
        x = b.input("x", whole_row(32))
        norm = b.weight("final_norm", [32])
        embed = b.weight("embed", [64, 32])
        n = b.rmsnorm("final_normed", 1e-6, norm, 1, x)
        logits = b.linear("logits", embed, 0, n)
        capped = b.softcap("capped", 30, logits)
        token = b.argmax("token", capped)
        b.output("token", token)
    return program("head", body)


def two_tiles():
    def body(b):
        x = b.input("x", whole_row(32))
        wa = b.weight("wa", [16, 32])
        wb = b.weight("wb", [16, 32])
        a = b.linear("a", wa, 0, x)
        bb = b.linear("b", wb, 0, x)
        b.output("c", b.add("c", a, bb))
    return program("two_tiles", body)


def attending(name: str, rest):
    """ProgramTest.hs:703-718: attention over two stored positions of a ring."""
    def body(b):
        q = b.input("q", Shape(4, 2))
        pos = b.row_ints("position", 1, 4)
        slot = b.row_ints("slot", 1, 2)
        k = b.cache("k", Ring(2, 1, 4, 2))
        v = b.cache("v", Ring(2, 1, 4, 2))
        kv = b.input("kv", Shape(2, 2))
        vv = b.input("vv", Shape(2, 2))
        b.kv_store("store_k", k, pos, slot, kv)
        b.kv_store("store_v", v, pos, slot, vv)
        o = b.attend("o", AttnSpec(2, 1, 2, None, 1), q, k, v, pos, slot)
        rest(b, o)
    return program(name, body)


def attn_out():
    return attending("attn_out", lambda b, o: b.output("o", o))


def attn_capped():
    return attending("attn_capped", lambda b, o: b.output("y", b.softcap("capped", 50, o)))


def attn_stored():
    def rest(b, o):
        c = b.cache("o_cache", Ring(2, 2, 4, 2))
        pos = b.row_ints("o_position", 1, 64)
        slot = b.row_ints("o_slot", 1, 2)
        b.kv_store("store_o", c, pos, slot, o)
        b.output("o", o)
    return attending("attn_stored", rest)


def attn_normed():
    def rest(b, o):
        w = b.weight("o_proj", [4, 4])
        n = b.rmsnorm("o_normed", 1e-6, None, 1, o)
        b.output("out", b.linear("out", w, 0, n))
    return attending("attn_normed", rest)


def attn_mixed():
    def rest(b, o):
        s = b.weight("attn_scale", [1])
        w = b.weight("o_proj", [4, 4])
        y = b.scale_by("scaled", s, o)
        n = b.rmsnorm("sub_norm", 1e-6, None, 1, o)
        out = b.linear("out", w, 0, n)
        b.output("y", y)
        b.output("out", out)
    return attending("attn_mixed", rest)


def attn_kept():
    def rest(b, o):
        w = b.weight("o_proj", [4, 4])
        n = b.rmsnorm("sub_norm", 1e-6, None, 1, o)
        out = b.linear("out", w, 0, n)
        c = b.cache("o_cache", Ring(2, 2, 4, 2))
        pos = b.row_ints("o_position", 1, 64)
        slot = b.row_ints("o_slot", 1, 2)
        b.kv_store("store_o", c, pos, slot, o)
        b.output("out", out)
    return attending("attn_kept", rest)


def predicting():
    def body(b):
        x = b.input("x", whole_row(32))
        router = b.weight("router_proj", [8, 32])
        ahead = b.weight("ahead_proj", [8, 32])
        experts = b.table("experts", 8, [16, 32])
        logits = b.linear("router_logits", router, 0, x)
        ahead_logits = b.linear("ahead_logits", ahead, 0, x)
        ids, ws = b.route("route", 2, None, logits)
        ahead_ids, _ = b.route("ahead", 2, None, ahead_logits)
        y = b.linear_routed("experts_out", experts, ids, x)
        s = b.combine_ranks("experts_sum", ws, y)
        b.output("y", s)
        b.output("ahead", ahead_ids)
    return program("predicting", body)


def embed_program():
    def body(b):
        tokens = b.row_ints("tokens", 1, 64)
        embed = b.weight("embed", [64, 32])
        b.output("x", b.gather("x", embed, tokens, 5.65625))
    return program("embed", body)


def ring_program(scaled: bool = False):
    """ProgramTest.hs:1294-1327."""
    def body(b):
        q = b.input("q", Shape(4, 2))
        pos = b.row_ints("position", 1, 64)
        slot = b.row_ints("slot", 1, 2)
        k = b.cache("k", Ring(2, 1, 4, 2))
        v = b.cache("v", Ring(2, 1, 4, 2))
        if scaled:
            one = b.weight("one", [1])
            kv = b.scale_by("kv_scaled", one, b.input("kv", Shape(2, 2)))
            vv = b.scale_by("vv_scaled", one, b.input("vv", Shape(2, 2)))
        else:
            kv = b.input("kv", Shape(2, 2))
            vv = b.input("vv", Shape(2, 2))
        b.kv_store("store_k", k, pos, slot, kv)
        b.kv_store("store_v", v, pos, slot, vv)
        b.output("o", b.attend("o", AttnSpec(2, 1, 2, 2, 1), q, k, v, pos, slot))
    return program("ring_scaled" if scaled else "ring", body)


def pooled():
    def body(b):
        t = b.weight("table", [6, 4])
        tok = b.row_ints("rows", 3, 6)
        w = b.weight("w", [2, 4])
        rows = b.gather("pooled", t, tok, 1 / 3)
        b.output("out", b.linear("out", w, 0, rows))
    return program("pooled", body)


def small():
    def body(b):
        x = b.input("x", whole_row(4))
        w = b.weight("w", [4, 4])
        y = b.linear("y", w, 0, x)
        b.output("n", b.rmsnorm("n", 1e-6, None, 1, y))
    return program("small", body)


def planned():
    """ProgramTest.hs:676-692: the programs the planner's tests plan."""
    return [layer(False), layer(True), head_program(), two_tiles(), embed_program(), attn_out(), attn_capped(),
            attn_stored(), attn_normed(), attn_mixed(), attn_kept(), predicting(), ring_program(), pooled()]


def routed_over(logits: int, entries: int):
    def body(b):
        x = b.input("x", whole_row(4))
        router = b.weight("router", [logits, 4])
        experts = b.table("experts", entries, [2, 4])
        ids, weights = b.route("route", 2, None, b.linear("router_logits", router, 0, x))
        y = b.linear_routed("experts_out", experts, ids, x)
        b.output("y", b.combine_ranks("experts_sum", weights, y))
    return program("routed", body)


def stored_into(layout, sequences: int, positions: int):
    def body(b):
        x = b.input("x", Shape(2, 2))
        pos = b.row_ints("position", 1, positions)
        sq = b.row_ints("slot", 1, sequences) if isinstance(layout, Ring) else b.row_ints("blocks", 2, sequences)
        k = b.cache("k", layout)
        b.kv_store("store_k", k, pos, sq, x)
    return program("stored_into", body)


def over_ring(length: int, window, bound: int):
    def body(b):
        q = b.input("q", Shape(2, 2))
        pos = b.row_ints("position", 1, bound)
        slot = b.row_ints("slot", 1, 1)
        k = b.cache("k", Ring(1, 1, length, 2))
        v = b.cache("v", Ring(1, 1, length, 2))
        b.output("o", b.attend("o", AttnSpec(1, 1, 2, window, 1), q, k, v, pos, slot))
    return program("over_ring", body)


def reaching(length: int, window, ahead, position_bound: int, reach_bound: int):
    """ProgramTest.hs:1571-1583."""
    def body(b):
        q = b.input("q", Shape(4, 2))
        pos = b.row_ints("position", 1, position_bound)
        slot = b.row_ints("slot", 1, 1)
        reach = None if ahead is None else Reach(b.row_ints("reach", 1, reach_bound).id, ahead)
        k = b.cache("k", Ring(1, 1, length, 2))
        v = b.cache("v", Ring(1, 1, length, 2))
        kv = b.input("kv", Shape(2, 2))
        b.kv_store("store_k", k, pos, slot, kv)
        b.kv_store("store_v", v, pos, slot, kv)
        b.output("o", b.attend("o", AttnSpec(2, 1, 2, window, 1, reach), q, k, v, pos, slot))
    return program("reach", body)


def paged_attention(blocks: int, positions: int, with_reach: bool):
    def body(b):
        q = b.input("q", Shape(4, 2))
        pos = b.row_ints("position", 1, positions)
        table = b.row_ints("blocks", 2, blocks)
        reach = Reach(b.row_ints("reach", 1, positions).id, positions) if with_reach else None
        k = b.cache("k", Paged(4, 2, 1, 2))
        v = b.cache("v", Paged(4, 2, 1, 2))
        b.output("o", b.attend("o", AttnSpec(2, 1, 2, None, 1, reach), q, k, v, pos, table))
    return program("paged", body)


def stored_dot_in(elem: str, k: int):
    """ProgramTest.hs:1147-1157: a linear layer of one output stored into a one-element cache."""
    def body(b):
        x = b.input("x", whole_row(k))
        w = b.weight("w", [1, k])
        pos = b.row_ints("position", 1, 1)
        slot = b.row_ints("slot", 1, 1)
        c = b.cache("c", Ring(1, 1, 1, 1), elem)
        y = b.linear("y", w, 0, x)
        b.kv_store("store", c, pos, slot, y)
        b.output("y", y)
    return program("stored_dot", body)
