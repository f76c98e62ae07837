"""Decode attention over paged pools and with a reach, the cases the CPU and
GPU tests share: a program of one decode row (queries and new key/value rows
as inputs, RoPE on queries and keys, the KV stores, the attention), in a
paged-pool form and the ring form holding the same keys and values, with
seeded state; and their runs on the oracle's CPU target."""

from __future__ import annotations

import math

import numpy as np

from furykernel_amd.lower import lower_plan, rope_table
from furykernel_amd.program.build import program
from furykernel_amd.program.check import check_program
from furykernel_amd.program.graph import CACHE_BF16, CACHE_F16, AttnSpec, F32, Paged, Reach, Ring, RopeSpec, Shape
from furykernel_amd.program.plan import PlanOptions, plan
from oracle.cpu_target import CpuTarget

# heads, kv heads, head width, block size, pool blocks, table length, window, bf16 caches
CASES = [
    (8, 2, 64, 16, 64, 16, None, 0),
    (32, 8, 64, 64, 48, 16, None, 0),   # the 1B shape's heads, a table of 1024 positions
    (4, 4, 32, 8, 40, 12, 40, 1),       # a window across blocks, bf16
]


def case_id(c) -> str:
    return "h{}_kv{}_d{}_bs{}_pool{}_t{}_w{}_bf{}".format(*[x if x is not None else 0 for x in c])


def decode_attention(heads, kv, d, layout, seq_count, seq_bound, window=None, bf16=0, reach_bound=None):
    """One row: RoPE'd queries over the caches after storing the row's
    RoPE'd key and its value."""
    positions = layout.block_size * seq_count if isinstance(layout, Paged) else layout.length

    def body(b):
        q = b.input("q", Shape(heads * d, d), F32)
        k = b.input("k", Shape(kv * d, d), F32)
        v = b.input("v", Shape(kv * d, d), F32)
        pos = b.row_ints("position", 1, positions)
        sq = b.row_ints("blocks" if isinstance(layout, Paged) else "slot", seq_count, seq_bound)
        reach = None if reach_bound is None else Reach(b.row_ints("reach", 1, reach_bound).id, reach_bound)
        kc = b.cache("kc", layout, CACHE_BF16 if bf16 else CACHE_F16)
        vc = b.cache("vc", layout, CACHE_BF16 if bf16 else CACHE_F16)
        spec = RopeSpec(10000.0, d // 2)
        qr = b.rope("qr", spec, pos, q)
        kr = b.rope("kr", spec, pos, k)
        b.kv_store("store_k", kc, pos, sq, kr)
        b.kv_store("store_v", vc, pos, sq, v)
        o = b.attend("o", AttnSpec(heads, kv, d, window, 1.0 / math.sqrt(d), reach), qr, kc, vc, pos, sq)
        b.output("o", o)
    return check_program(program("decode_attention", body))


def paged_program(c, reach_bound=None):
    heads, kv, d, bs, blocks, tl, window, bf16 = c
    return decode_attention(heads, kv, d, Paged(blocks, bs, kv, d), tl, blocks, window, bf16, reach_bound)


def ring_program(c, reach_bound=None):
    heads, kv, d, bs, blocks, tl, window, bf16 = c
    return decode_attention(heads, kv, d, Ring(1, kv, bs * tl, d), 1, 1, window, bf16, reach_bound)


def state(c, position, seed=7):
    """Inputs, a block table (distinct blocks in a scrambled order), and a
    pool whose blocks hold N(0, 1) keys and values, with the ring that holds
    the same rows."""
    heads, kv, d, bs, blocks, tl, window, bf16 = c
    rng = np.random.default_rng(seed)
    table = rng.permutation(blocks)[:tl].astype(np.uint32)
    x = {"q": (rng.standard_normal(heads * d) * 0.5).astype(np.float32),
         "k": (rng.standard_normal(kv * d) * 0.5).astype(np.float32),
         "v": rng.standard_normal(kv * d).astype(np.float32)}
    vals = rng.standard_normal((2, blocks, kv, bs, d)).astype(np.float32)
    if bf16:
        pool = (vals.view(np.uint32) >> 16).astype(np.uint16)
    else:
        pool = vals.astype(np.float16).view(np.uint16)
    # ring[h, t] = block table[t // bs], row (h, t % bs)
    ring = np.stack([pool[j][table[np.arange(bs * tl) // bs], :, np.arange(bs * tl) % bs, :].transpose(1, 0, 2)
                     for j in range(2)])
    return x, table, pool, ring


def lowered(checked, wide=False):
    return lower_plan(checked, plan(PlanOptions(), checked), wide=wide)


def run_cpu(low, x, position, table=None, pool=None, ring=None, reach=None):
    cpu = CpuTarget(low, 64)
    for name, what in low.constants.items():
        if what[0] == "rope":
            cpu.write(name, rope_table(*what[1:]))
    for name, val in x.items():
        cpu.write(f"value:{name}", val)
    cpu.write("ints:position", [position])
    def bits(name, a):  # the cache's elements as their bits
        cpu.write(name, np.ascontiguousarray(a).ravel().view(cpu.buffers[name].dtype))

    if table is not None:
        cpu.write("ints:blocks", table)
        bits("cache:kc", pool[0])
        bits("cache:vc", pool[1])
    else:
        cpu.write("ints:slot", [0])
        bits("cache:kc", ring[0])
        bits("cache:vc", ring[1])
    if reach is not None:
        cpu.write("ints:reach", [reach])
    cpu.run()
    return cpu
