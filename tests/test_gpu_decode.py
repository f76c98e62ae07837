"""A planned decode step on the GPU against the oracle's CPU target running the
same launch list, bit for bit; and the device state it leaves (KV caches,
every stored value).  Configurations: the tiny f32 decode and the 1B-class f16
decode (d_model 2048, 16 layers, 32/8 heads of 64, FFN 8192, vocab 32000,
context 4096)."""

import dataclasses

import numpy as np
import pytest

from furykernel_amd.decode import DecodeSession
from furykernel_amd.program.decoder import ONE_B, TINY, TINY_GQA
from furykernel_amd.program.plan import PlanOptions
from oracle.cpu_target import CpuTarget

pytestmark = pytest.mark.gpu

TINY32 = dataclasses.replace(TINY, context=32)


def mirror(session: DecodeSession, width: int = 64, cpu: CpuTarget | None = None) -> CpuTarget:
    """The CPU target with every buffer the device holds (given a CPU target
    that has the weights already, every other buffer)."""
    fresh = cpu is None
    cpu = CpuTarget(session.lowered, width) if fresh else cpu
    for name in session.lowered.buffers:
        if fresh or not name.startswith("weight:"):
            cpu.write(name, session.engine.read(name))
    return cpu


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def compare_all(session, cpu, names=None):
    bad = []
    for name in names or session.lowered.buffers:
        g, c = session.engine.read(name), cpu.read(name)
        if not np.array_equal(bits(g), bits(c)):
            bad.append((name, int(np.sum(bits(g) != bits(c))), g.size))
    return bad


@pytest.mark.parametrize("position,fuse", [(0, True), (16, True), (31, True), (0, False), (31, False)])
def test_tiny_decode_step_bit_exact(device, kernels, position, fuse):
    """With the KV store folded into the attention launch (fuse), and as the
    plan's separate store and attention steps."""
    s = DecodeSession(device, kernels, TINY32, PlanOptions(), embed=False, fuse=fuse)
    try:
        s.init_synthetic()
        s.set_position(position)
        cpu = mirror(s)
        print(f"tiny decode at position {position} (fuse {fuse}): {len(s.lowered.launches)} launches", flush=True)
        s.step()
        device.sync()
        cpu.run()
        assert compare_all(s, cpu) == []
    finally:
        s.close()


def test_tiny_decode_graph_replays_agree_with_eager(device, kernels):
    s = DecodeSession(device, kernels, TINY32, PlanOptions(store_gelus=True), embed=False)
    try:
        s.init_synthetic()
        s.set_position(5)
        s.step()
        device.sync()
        eager = s.logits()
        g = s.graph()
        for _ in range(3):
            g.replay()
            device.sync()
            assert np.array_equal(bits(s.logits()), bits(eager))
        g.destroy()
    finally:
        s.close()


@pytest.mark.parametrize("store_gelus,tuned", [(False, False), (True, False), (True, True)])
def test_1b_decode_step_bit_exact(device, kernels, store_gelus, tuned):
    """The 1B-class step's real shapes (2 of its 16 layers, and the head) at the
    full context: position 4095 reads all 4096 positions of every cache.  With
    the plan's SiLU·mul recomputed in the down projection's prologue, and
    stored (folded into the gate/up step's epilogue); and with the GEMV steps
    shaped as the committed selections pick (tuned)."""
    layers = 2
    s = DecodeSession(device, kernels, ONE_B, PlanOptions(store_gelus=store_gelus), embed=True, layers=layers,
                      tuned=tuned)
    try:
        s.init_synthetic()
        s.set_position(4095, token=31999)
        cpu = mirror(s)
        print(f"1B decode ({layers} layers, store_gelus {store_gelus}) at position 4095: "
              f"{len(s.lowered.launches)} launches", flush=True)
        s.step()
        device.sync()
        cpu.run()
        skip = {n for n in s.lowered.buffers if n.startswith("weight:")}
        assert compare_all(s, cpu, [n for n in s.lowered.buffers if n not in skip]) == []
    finally:
        s.close()


@pytest.mark.parametrize("pick", [(1, 3), (1, 4), (2, 3)])
def test_1b_decode_step_bit_exact_in_every_block_shape(device, kernels, pick):
    """Two layers of the 1B step with every GEMV step shaped as the pick
    says (rows a block, threadgroups a CU) where it can be: at one row a
    block the gate/up step's SiLU·mul meets each row of gate and of up
    across two wavefronts; every stored buffer the CPU target's."""
    s = DecodeSession(device, kernels, ONE_B, PlanOptions(store_gelus=True), embed=True, layers=2,
                      choose=lambda L: pick)
    try:
        gu = [L for L in s.lowered.launches if L.params.get("epi_mode") == 3]
        assert gu and all(f"_r{pick[0]}_" in L.entry for L in gu)
        s.init_synthetic()
        s.set_position(4095, token=31999)
        cpu = mirror(s)
        print(f"1B decode (2 layers) with GEMV blocks {pick}: {len(s.lowered.launches)} launches", flush=True)
        s.step()
        device.sync()
        cpu.run()
        assert compare_all(s, cpu, [n for n in s.lowered.buffers if not n.startswith("weight:")]) == []
    finally:
        s.close()


def test_tiny_decode_bit_exact_at_one_row_a_block(device, kernels):
    """The tiny f32 step (SiLU·mul folded into gate/up) with every GEMV step
    at one row a block, two threadgroups a CU: bit for bit the CPU target's."""
    s = DecodeSession(device, kernels, TINY32, PlanOptions(store_gelus=True), embed=False, choose=lambda L: (1, 2))
    try:
        assert any(L.params.get("epi_mode") == 3 and "_r1_" in L.entry for L in s.lowered.launches)
        s.init_synthetic()
        s.set_position(20)
        cpu = mirror(s)
        print("tiny decode, one row a block", flush=True)
        s.step()
        device.sync()
        cpu.run()
        assert compare_all(s, cpu) == []
    finally:
        s.close()


def test_1b_full_decode_greedy_tokens_via_graph(device, kernels):
    """All 16 layers, planned as the benchmark plans them: three greedy tokens by
    graph replay, each step's token the CPU target's for the same state."""
    s = DecodeSession(device, kernels, ONE_B, PlanOptions(store_gelus=True), embed=True)
    try:
        s.init_synthetic()
        s.set_position(4000, token=7)
        g = s.graph()
        cpu = None
        for i in range(3):
            cpu = mirror(s, cpu=cpu)
            print(f"1B decode token {i}", flush=True)
            g.replay()
            device.sync()
            cpu.run()
            assert s.token() == int(cpu.read("value:token")[0])
            assert np.array_equal(bits(s.logits()), bits(cpu.read("value:logits")))
            assert int(s.engine.read("ints:tokens")[0]) == s.token()
            assert int(s.engine.read("ints:position")[0]) == 4001 + i
        g.destroy()
    finally:
        s.close()


def test_tiny_decode_on_the_gpu_within_1e4_of_the_f64_evaluator(device, kernels):
    """The tiny configuration (d_model 64, 2 layers, 4 heads of 16, FFN 256
    SiLU-gated, vocab 256; weights, caches and input N(0, 0.02); 16 cached
    positions before the token) on the GPU: its logits within 1e-4 (of the
    row's largest magnitude) of the f64 program evaluator, and bit for bit the
    CPU target's."""
    from test_evaluator import rel, run_cpu_target, run_evaluator, tiny_state

    checked, w, c, x, position = tiny_state()
    s = DecodeSession(device, kernels, TINY32, PlanOptions(), embed=False)
    try:
        for name, v in w.items():
            if f"weight:{name}" in s.lowered.buffers:
                s.engine.write(f"weight:{name}", v)
        for name, v in c.items():
            s.engine.write(f"cache:{name}", v)
        s.engine.write("value:x", x)
        s.set_position(position)
        print(f"tiny decode vs the f64 evaluator at position {position}", flush=True)
        s.step()
        device.sync()
        logits = s.logits()
        ev = run_evaluator(checked, w, c, x, position)
        assert rel(logits, ev.outputs["logits"][0]) <= 1e-4
        cpu = run_cpu_target(checked, w, c, x, position, 64)
        assert np.array_equal(bits(logits), bits(cpu.read("value:logits")))
        assert s.token() == int(cpu.read("value:token")[0])
    finally:
        s.close()


@pytest.mark.parametrize("position", [130, 255])
def test_tiny_gqa_decode_on_the_gpu_in_two_splits(device, kernels, position):
    """Grouped queries (4 heads over 2 kv heads, ring of 256) at positions
    whose attention runs in two splits: the GPU's logits within 1e-4 of the
    f64 evaluator, and logits, caches and token bit for bit the CPU target's."""
    from test_evaluator import rel, run_cpu_target, run_evaluator, tiny_state

    checked, w, c, x, _ = tiny_state(position=position, dims=TINY_GQA)
    s = DecodeSession(device, kernels, TINY_GQA, PlanOptions(), embed=False)
    try:
        for name, v in w.items():
            if f"weight:{name}" in s.lowered.buffers:
                s.engine.write(f"weight:{name}", v)
        for name, v in c.items():
            s.engine.write(f"cache:{name}", v)
        s.engine.write("value:x", x)
        s.set_position(position)
        print(f"tiny GQA decode vs the f64 evaluator at position {position}", flush=True)
        s.step()
        device.sync()
        logits = s.logits()
        ev = run_evaluator(checked, w, c, x, position)
        assert rel(logits, ev.outputs["logits"][0]) <= 1e-4
        cpu = run_cpu_target(checked, w, c, x, position, 64)
        assert np.array_equal(bits(logits), bits(cpu.read("value:logits")))
        for name in c:
            assert np.array_equal(s.engine.read(f"cache:{name}").view(np.uint16),
                                  cpu.read(f"cache:{name}").view(np.uint16)), name
        assert s.token() == int(cpu.read("value:token")[0])
    finally:
        s.close()


def test_tiny_decode_on_the_gpu_within_the_element_bounds(device, kernels):
    """The tiny configuration on the GPU against the evaluator's per-element
    bounds (Eval.hs:686-966): every value the step stores within its
    element's bound of the exact value, every new cache element one a kernel
    may store, the token the evaluator's where its arg-max is decided."""
    from oracle import bounds as B
    from test_bounds import bindings, check_tiny
    from test_evaluator import run_evaluator, tiny_state

    checked, w, c, x, position = tiny_state()
    s = DecodeSession(device, kernels, TINY32, PlanOptions(), embed=False)
    try:
        for name, v in w.items():
            if f"weight:{name}" in s.lowered.buffers:
                s.engine.write(f"weight:{name}", v)
        for name, v in c.items():
            s.engine.write(f"cache:{name}", v)
        s.engine.write("value:x", x)
        s.set_position(position)
        print(f"tiny decode on the GPU against the element bounds at position {position}", flush=True)
        s.step()
        device.sync()
        ev = run_evaluator(checked, w, c, x, position)
        bd = B.evaluate_bounds(checked, bindings(w, c, x, position), ev)

        class Read:
            lowered = s.lowered

            @staticmethod
            def read(name):
                return s.engine.read(name)
        assert check_tiny(Read, ev, bd, checked, c) == []
        if bd.values["token"][0][0] == 0:
            assert s.token() == int(ev.values["token"][0][0])
        # evaluateStored: the evaluation given the caches the kernels left
        # (each new element checked against its bound), and the step's values
        # within their bounds of it.
        from test_bounds import kept_of
        ev2, bd2 = B.evaluate_stored(checked, bindings(w, c, x, position), kept_of(Read, checked))
        assert check_tiny(Read, ev2, bd2, checked, c) == []
        # and anchored at every value the launches stored: each launch from
        # its stored inputs, both layers held to finite bounds
        from test_bounds import check_anchored
        _, _, rel = check_anchored(Read, checked, w, c, x, position)
        assert any(n.startswith("l1_") for n in rel)
        assert max(v for n, v in rel.items() if n != "token") < 1e-4
    finally:
        s.close()


def test_paged_decode_step_is_the_ring_step_bit_for_bit(device, kernels):
    """Two layers of the 1B-shape step at position 4095 with the caches as
    paged pools (blocks of 64 positions in a pool of 80, a scrambled table):
    the pools hold the ring's rows through the table, and the step's logits,
    token and the row it stores are the ring step's bit for bit."""
    import dataclasses

    from furykernel_amd.program.decoder import ONE_B
    dims = dataclasses.replace(ONE_B)
    bs, pool = 64, 80
    table = np.random.default_rng(4).permutation(pool)[:dims.context // bs].astype(np.uint32)
    ring = DecodeSession(device, kernels, dims, PlanOptions(store_gelus=True), embed=True, layers=2)
    paged = DecodeSession(device, kernels, dims, PlanOptions(store_gelus=True), embed=True, layers=2,
                          paging=(bs, pool))
    try:
        assert any(l.entry == "fk_step_attend_paged" for l in paged.lowered.launches)
        ring.init_synthetic()
        paged.init_synthetic()
        names = [n for n in ring.lowered.buffers if n.startswith("cache:")]
        for n in names:   # the ring's rows scattered into the pool's blocks by the table
            r = ring.engine.read(n).reshape(dims.kv_heads, dims.context // bs, bs, dims.head_dim)
            p = np.zeros((pool, dims.kv_heads, bs, dims.head_dim), r.dtype)
            p[table] = r.transpose(1, 0, 2, 3)
            paged.engine.write(n, p.reshape(-1))
        ring.set_position(4095, token=7)
        paged.set_position(4095, token=7, table=table)
        print("1B shapes, two layers: ring and paged decode steps at position 4095", flush=True)
        ring.step()
        paged.step()
        device.sync()
        assert np.array_equal(ring.logits().view(np.uint32), paged.logits().view(np.uint32))
        assert ring.token() == paged.token()
        for n in names:
            r = ring.engine.read(n).reshape(dims.kv_heads, dims.context // bs, bs, dims.head_dim)
            p = paged.engine.read(n).reshape(pool, dims.kv_heads, bs, dims.head_dim)
            assert np.array_equal(p[table].transpose(1, 0, 2, 3).view(np.uint16), r.view(np.uint16)), n
    finally:
        ring.close()
        paged.close()


def test_tiny_embed_decode_on_the_gpu_within_1e4_of_the_f64_evaluator(device, kernels):
    """The tiny decode with the token's embedding row gathered and scaled by
    5.65625 (the reference's embedding program, ProgramTest.hs:785-789) on
    the GPU: every buffer the step stores (the layer-0 QKV step's gathered
    prologue, the gathered residual, caches, logits, token) bit for bit the
    CPU target's, and the logits within 1e-4 of the f64 evaluator."""
    from furykernel_amd.program.decoder import TINY_EMBED
    from test_embed_decode import POSITION, TOKEN, embed_state, rel, run_cpu, run_eval

    checked, w, c = embed_state()
    s = DecodeSession(device, kernels, TINY_EMBED, PlanOptions(), embed=True)
    try:
        for name, v in w.items():
            if f"weight:{name}" in s.lowered.buffers:
                s.engine.write(f"weight:{name}", v)
        for name, v in c.items():
            s.engine.write(f"cache:{name}", v)
        s.set_position(POSITION, token=TOKEN)
        cpu = mirror(s)
        print(f"tiny decode, embedding row scaled by 5.65625, token {TOKEN} at position {POSITION}", flush=True)
        s.step()
        device.sync()
        cpu.run()
        assert compare_all(s, cpu, [n for n in s.lowered.buffers if not n.startswith("weight:")]) == []
        # the mirrored state is the CPU tests' state
        assert np.array_equal(bits(s.logits()), bits(run_cpu(checked, w, c).read("value:logits")))
        ev = run_eval(checked, w, c)
        assert rel(s.logits(), ev.outputs["logits"][0]) <= 1e-4
    finally:
        s.close()
