"""Staged KV stores on the GPU (src/FuryKernel/Program/Plan.hs:41-50): a
prefill whose positions may reach the ring's length stores each row's keys
and values into staging rows, the attention reads the step's own positions
from there and earlier ones from the ring, and the combine step lands them.

- From position 0 the staged prefill is the in-place one bit for bit:
  logits, tokens and every cache (the staged rows hold what the cache would,
  and the attention reads the same values from them).
- A second step continuing the sequences (positions 128..255) reads the
  first step's rows from the ring and its own from the staging rows: its
  logits and the caches it fills within the f16 bar (2e-3) of the binary64
  evaluator started from the caches the first step left.
- At the 1B shape (4 sequences of 2048 rows, positions bounded by the ring's
  4096), staged and in place agree bit for bit on the tokens, on sampled
  rows' logits and on two layers' caches.
"""

import numpy as np
import pytest

from furykernel_amd.program.decoder import ONE_B_PREFILL, SMALL_PREFILL
from oracle.eval import Bindings, evaluate_fast
from test_gpu_prefill import BAR, SEQ_ROWS, SEQS, rel, small_state

pytestmark = pytest.mark.gpu


def session(device, kernels, dims, seqs, rows, bound=None, rotated=None):
    from furykernel_amd.prefill import PrefillSession
    s = PrefillSession(device, kernels, dims, seqs, rows, position_bound=bound, rope_rotated=rotated)
    for name in s.lowered.buffers:
        if name.startswith("cache:"):
            s.engine.zero(name)
    return s


def caches_of(s):
    return {n: s.engine.read(n).copy() for n in s.lowered.buffers if n.startswith("cache:")}


@pytest.mark.parametrize("rotated", [None, 16], ids=["qkv-epilogue-stores", "rope-kernel-stores"])
def test_staged_prefill_is_the_in_place_one_bit_for_bit(device, kernels, rotated):
    """With every pair turned the QKV GEMM's epilogue writes the staging
    rows; with 16 of 32 the RoPE kernel does."""
    a = session(device, kernels, SMALL_PREFILL, SEQS, SEQ_ROWS, rotated=rotated)
    b = session(device, kernels, SMALL_PREFILL, SEQS, SEQ_ROWS, bound=SMALL_PREFILL.context, rotated=rotated)
    try:
        assert not a.staged and b.staged
        weights, tokens = small_state(a.checked)
        for s in (a, b):
            s.write_weights(weights)
            s.set_tokens(tokens)
            print(f"small prefill, staged {s.staged}: {len(s.lowered.launches)} launches", flush=True)
            s.run()
            device.sync()
        assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))
        assert np.array_equal(a.tokens(), b.tokens())
        ca, cb = caches_of(a), caches_of(b)
        assert ca.keys() == cb.keys() and all(np.array_equal(ca[n], cb[n]) for n in ca)
    finally:
        a.close()
        b.close()


def test_a_second_staged_step_reads_the_ring_and_its_staging_rows(device, kernels):
    s = session(device, kernels, SMALL_PREFILL, SEQS, SEQ_ROWS, bound=SMALL_PREFILL.context)
    try:
        weights, tokens = small_state(s.checked)
        s.write_weights(weights)
        s.set_tokens(tokens)
        s.run()
        device.sync()
        before = caches_of(s)
        rng = np.random.default_rng(5)
        tokens2 = rng.integers(0, SMALL_PREFILL.vocab, SEQS * SEQ_ROWS)
        positions2 = np.tile(np.arange(SEQ_ROWS, 2 * SEQ_ROWS, dtype=np.uint32), SEQS)
        slots = np.repeat(np.arange(SEQS, dtype=np.uint32), SEQ_ROWS)
        from furykernel_amd.prefill import check_rows
        check_rows(positions2, slots, SEQ_ROWS)
        s.engine.set_ints("position", positions2, SMALL_PREFILL.context)
        s.set_tokens(tokens2)
        print("small prefill, second staged step at positions 128..255", flush=True)
        s.run()
        device.sync()
        lay = SMALL_PREFILL
        per_slot = lay.kv_heads * lay.context * lay.head_dim
        caches = {}
        for src in s.checked.program.sources:
            if type(src.kind).__name__ == "SCache":
                raw = before[f"cache:{src.name}"].astype(np.float64)
                caches[src.name] = {u: raw[u * per_slot:(u + 1) * per_slot].copy() for u in range(lay.slots)}
        ev = evaluate_fast(s.checked, Bindings(
            SEQS * SEQ_ROWS, weights={k: np.asarray(v, np.float64) for k, v in weights.items()},
            row_ints={"tokens": tokens2[:, None], "position": positions2[:, None], "slot": slots[:, None]},
            caches=caches))
        assert rel(s.logits(), np.array(ev.outputs["logits"])) <= BAR
        after = caches_of(s)
        for src in s.checked.program.sources:
            if type(src.kind).__name__ == "SCache":
                got = after[f"cache:{src.name}"].astype(np.float64)
                want = np.concatenate([np.asarray(ev.caches[src.name][u]) for u in range(lay.slots)])
                assert rel(got, want) <= BAR
                # the first step's rows are untouched by the second
                g = got.reshape(lay.slots, lay.kv_heads, lay.context, lay.head_dim)
                w = before[f"cache:{src.name}"].astype(np.float64).reshape(g.shape)
                assert np.array_equal(g[:, :, :SEQ_ROWS], w[:, :, :SEQ_ROWS])
    finally:
        s.close()


def test_staged_1b_prefill_is_the_in_place_one(device, kernels):
    seqs, rows = 4, 2048
    a = session(device, kernels, ONE_B_PREFILL, seqs, rows)
    try:
        a.init_synthetic(seed=2026)
        tokens = np.random.default_rng(9).integers(0, ONE_B_PREFILL.vocab, seqs * rows)
        a.set_tokens(tokens)
        print("1B prefill in place", flush=True)
        a.run()
        device.sync()
        tok_a = a.tokens().copy()
        pick = np.arange(0, seqs * rows, 977)
        lg_a = a.logits()[pick].copy()
        names = ["cache:l0_k_cache", "cache:l15_v_cache"]
        ca = {n: a.engine.read(n).copy() for n in names}
    finally:
        a.close()
    b = session(device, kernels, ONE_B_PREFILL, seqs, rows, bound=ONE_B_PREFILL.context)
    try:
        assert b.staged
        b.init_synthetic(seed=2026)
        b.set_tokens(tokens)
        print("1B prefill staged", flush=True)
        b.run()
        device.sync()
        assert np.array_equal(tok_a, b.tokens())
        assert np.array_equal(lg_a.view(np.uint32), b.logits()[pick].view(np.uint32))
        for n in names:
            assert np.array_equal(ca[n], b.engine.read(n))
    finally:
        b.close()


def _pool_as_rings(pool, tables, kv_heads, block_size, d):
    """A pool [blocks][kv_heads][block_size][d] read through each sequence's
    table as rings [sequences][kv_heads][table_len block_size][d]."""
    p = pool.reshape(-1, kv_heads, block_size, d)
    return np.stack([np.concatenate([p[b] for b in t], axis=1) for t in tables])


@pytest.mark.parametrize("dims,seqs,rows,layers,paging,rotated", [
    (SMALL_PREFILL, SEQS, SEQ_ROWS, None, (64, 11), None),
    (SMALL_PREFILL, SEQS, SEQ_ROWS, None, (32, 20), 16),
    (ONE_B_PREFILL, 4, 2048, 2, (64, 300), None),
], ids=["small", "small-rope-kernel", "1b-two-layers"])
def test_paged_prefill_is_the_ring_prefill_bit_for_bit(device, kernels, dims, seqs, rows, layers, paging, rotated):
    """The caches as paged pools, each sequence's rows through a scrambled
    block table: logits and tokens are the ring prefill's bit for bit, and
    the pool read through the tables holds the ring's rows.  With every pair
    turned the QKV GEMM's epilogue stores into the pools; with 16 of 32 the
    RoPE kernel does."""
    from furykernel_amd.prefill import PrefillSession
    tokens = np.random.default_rng(33).integers(0, dims.vocab, seqs * rows)
    out = {}
    for paged in (False, True):
        s = PrefillSession(device, kernels, dims, seqs, rows, layers=layers, paging=paging if paged else None,
                           rope_rotated=rotated)
        try:
            entries = {l.entry for l in s.lowered.launches}
            store = "fk_prefill_rope_store_paged" if rotated else "fk_gemm_f16_qkv_rope_paged"
            assert (store in entries) == paged
            for name in s.lowered.buffers:
                if name.startswith("cache:"):
                    s.engine.zero(name)
            s.init_synthetic(seed=41)
            s.set_tokens(tokens)
            print(f"prefill {dims.d_model} x {seqs * rows} rows, paged {paged}", flush=True)
            s.run()
            device.sync()
            pick = np.arange(0, seqs * rows, 37)
            caches = {n: s.engine.read(n).copy() for n in s.lowered.buffers if n.startswith("cache:")}
            out[paged] = (s.logits()[pick].copy(), s.tokens().copy(), caches,
                          s.tables if paged else None)
        finally:
            s.close()
    (la, ta, ca, _), (lb, tb, cb, tables) = out[False], out[True]
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)) and np.array_equal(ta, tb)
    bs = paging[0]
    for name, ring in ca.items():
        ring = ring.reshape(dims.slots, dims.kv_heads, dims.context, dims.head_dim)[:seqs]
        got = _pool_as_rings(cb[name], tables, dims.kv_heads, bs, dims.head_dim)
        assert np.array_equal(got.view(np.uint16), ring.view(np.uint16)), name
