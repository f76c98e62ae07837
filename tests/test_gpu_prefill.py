"""Prefill on the GPU against the f64 evaluator.

The small decoder (d 256, 8 heads of 64 over 4 kv heads, FFN 512, vocab 512,
2 layers, f16 weights) over two sequences of 128 rows, through the planned
prefill (furykernel_amd/prefill.py): every row's logits and the KV caches it
fills within the f16 bar, 2e-3 of the largest magnitude, of the vectorised
binary64 evaluator (oracle/eval.py, pinned to the exact one).  The GEMM
operands and the attention's probabilities are f16 on this path; the
evaluator rounds only the cache stores.  With every pair of the heads turned
the QKV GEMM RoPEs and stores in its epilogue; with 16 of the 32 the RoPE
kernel does (both run); and the same decoder with a GELU-tanh MLP (the gate/up
GEMM's other activation).
"""

import dataclasses

import numpy as np
import pytest

from furykernel_amd.program.decoder import SMALL_PREFILL
from oracle.eval import Bindings, evaluate_fast

pytestmark = pytest.mark.gpu

SEQS, SEQ_ROWS = 2, 128
BAR = 2e-3


def small_state(checked, seed=31):
    rng = np.random.default_rng(seed)
    weights = {}
    for src in checked.program.sources:
        if type(src.kind).__name__ != "SWeight":
            continue
        dims = src.kind.dims
        if len(dims) == 1:
            weights[src.name] = (1 + 0.1 * rng.standard_normal(dims[0])).astype(np.float32)
        elif src.name == "embed":
            weights[src.name] = (0.5 * rng.standard_normal(dims)).astype(np.float16)
        else:
            weights[src.name] = (0.05 * rng.standard_normal(dims)).astype(np.float16)
    tokens = rng.integers(0, SMALL_PREFILL.vocab, SEQS * SEQ_ROWS)
    return weights, tokens


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.fixture(scope="module", params=[(None, "silu"), (16, "silu"), (None, "gelu_tanh")],
                ids=["rope-all-pairs", "rope-16-pairs", "gelu-tanh"])
def run(request, device, kernels):
    from furykernel_amd.prefill import PrefillSession

    rotated, act = request.param
    dims = dataclasses.replace(SMALL_PREFILL, act=act)
    s = PrefillSession(device, kernels, dims, SEQS, SEQ_ROWS, rope_rotated=rotated)
    entries = {l.entry for l in s.lowered.launches}
    fused = "fk_gemm_f16_qkv_rope" in entries
    assert fused == (rotated is None) and fused != ("fk_prefill_rope_store" in entries)
    acts = {l.params["act"] for l in s.lowered.launches if l.entry == "fk_gemm_f16_silu_mul"}
    assert acts == {1 if act == "gelu_tanh" else 0}
    weights, tokens = small_state(s.checked)
    s.write_weights(weights)
    for name in s.lowered.buffers:
        if name.startswith("cache:"):
            s.engine.zero(name)
    s.set_tokens(tokens)
    print(f"prefill small, rotated {rotated}, {act}: {len(s.lowered.launches)} launches", flush=True)
    s.run()
    device.sync()
    lay = SMALL_PREFILL
    caches = {}
    for src in s.checked.program.sources:
        if type(src.kind).__name__ == "SCache":
            caches[src.name] = {u: np.zeros(lay.kv_heads * lay.context * lay.head_dim) for u in range(lay.slots)}
    positions = np.tile(np.arange(SEQ_ROWS), SEQS)
    slots = np.repeat(np.arange(SEQS), SEQ_ROWS)
    ev = evaluate_fast(s.checked, Bindings(
        SEQS * SEQ_ROWS, weights={k: np.asarray(v, np.float64) for k, v in weights.items()},
        row_ints={"tokens": tokens[:, None], "position": positions[:, None], "slot": slots[:, None]},
        caches=caches))
    yield s, ev
    s.close()


def test_prefill_logits_within_the_f16_bar_of_the_f64_evaluator(run):
    s, ev = run
    got = s.logits()
    want = ev.outputs["logits"]
    assert got.shape == want.shape
    assert rel(got, want) <= BAR
    # and row by row, against each row's own scale
    for r in range(0, got.shape[0], 17):
        assert rel(got[r], want[r]) <= 4 * BAR


def test_prefill_fills_the_caches_the_decode_step_reads(run):
    s, ev = run
    lay = SMALL_PREFILL
    for layer in range(lay.layers):
        for kv in ("k", "v"):
            name = f"l{layer}_{kv}_cache"
            got = s.cache(name).astype(np.float64).reshape(lay.slots, lay.kv_heads, lay.context, lay.head_dim)
            want = np.stack([ev.caches[name][u] for u in range(lay.slots)]).reshape(got.shape)
            # the rows written: positions 0..127 of both slots
            assert rel(got[:, :, :SEQ_ROWS], want[:, :, :SEQ_ROWS]) <= BAR
            assert np.all(got[:, :, SEQ_ROWS:] == 0)


def test_prefill_tokens_are_each_rows_greedy_choice(run):
    s, ev = run
    logits = s.logits()
    assert np.array_equal(s.tokens(), np.argmax(logits, axis=1))
    want = ev.outputs["logits"]
    top2 = np.sort(want, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 8 * BAR * np.max(np.abs(want))
    assert np.array_equal(s.tokens()[clear], np.argmax(want, axis=1)[clear])


def test_prefill_graph_replays_equal_the_eager_run(run, device):
    s, _ = run
    eager = s.logits().copy()
    g = s.graph()
    for _ in range(3):
        g.replay()
        device.sync()
        assert np.array_equal(s.logits(), eager)
    g.destroy()


def test_prefill_attention_with_a_window_against_f64(device, kernels):
    """fk_prefill_attend alone: 256 rows (4 sequences of 64 at positions 16..79
    of their slots), 8 heads over 2 kv heads, a window of 48, random f16
    caches; against binary64 softmax attention of the same f16 values."""
    rng = np.random.default_rng(9)
    rows, heads, kvh, length, slots, window = 256, 8, 2, 128, 4, 48
    scale = 0.125
    q = (rng.standard_normal((rows, heads * 64))).astype(np.float16)
    kc = rng.standard_normal((slots, kvh, length, 64)).astype(np.float16)
    vc = rng.standard_normal((slots, kvh, length, 64)).astype(np.float16)
    positions = np.tile(np.arange(16, 80), 4).astype(np.uint32)
    seqs = np.repeat(np.arange(4), 64).astype(np.uint32)
    bufs = [device.upload(x) for x in (q, kc, vc, positions, seqs)]
    out = device.alloc(rows * heads * 64 * 2)
    kernels.prefill_attend(*bufs, out, rows, heads, kvh, length, slots, scale, window=window,
                           positions=positions, seqs=seqs)
    device.sync()
    from furykernel_amd.layout import unpack

    got = unpack(out.read(np.float16, rows * heads * 64), rows, heads * 64).astype(np.float64)
    want = np.empty((rows, heads, 64))
    for r in range(rows):
        p, sl = int(positions[r]), int(seqs[r])
        ts = np.arange(max(0, p - window + 1), p + 1)
        for h in range(heads):
            g = h // (heads // kvh)
            sc = scale * (kc[sl, g, ts].astype(np.float64) @ q[r, h * 64:(h + 1) * 64].astype(np.float64))
            e = np.exp(sc - sc.max())
            want[r, h] = (e / e.sum()) @ vc[sl, g, ts].astype(np.float64)
    assert rel(got, want.reshape(rows, -1)) <= BAR
    for b in bufs + [out]:
        b.free()


@pytest.mark.parametrize("width", [512, 2048, 768])
def test_prefill_norm_pack_against_f64(device, kernels, width):
    """The one-pass entries (rows of 512 and 2048 held in registers) and the
    two-pass kernel (768)."""
    from furykernel_amd.layout import unpack

    rng = np.random.default_rng(4)
    x = rng.standard_normal((256, width)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    bx, bg, by = device.upload(x), device.upload(g), device.alloc(256 * width * 2)
    kernels.prefill_norm_pack(bx, bg, by, 256, width, eps=1e-5)
    device.sync()
    got = unpack(by.read(np.float16, 256 * width), 256, width).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd * (np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) ** -0.5 * g
    # one f16 rounding: within half an f16 ulp of the value, up to f32 noise
    assert np.all(np.abs(got - want) <= np.abs(want) * (2.0**-11 + 2.0**-20) + 2.0**-25)
    for b in (bx, bg, by):
        b.free()


@pytest.mark.parametrize("staged", [False, True], ids=["in-place", "staged"])
def test_prefill_with_bf16_caches_against_the_f64_evaluator(device, kernels, staged):
    """The small decoder with bf16 KV caches: the QKV epilogue rounds k and v
    to bf16 (into the ring, or into staging rows that fk_prefill_land copies),
    the attention widens them to f16 for the matrix cores.  Logits within the
    f16 bar of the evaluator (which rounds its cache stores to bf16 too); each
    cache element within the bar plus one bf16 unit in the last place of
    itself, since an element next to a rounding boundary may round either way
    from values that agree to the bar; tokens each row's argmax."""
    from furykernel_amd.prefill import PrefillSession
    from furykernel_amd.program.graph import CACHE_BF16

    dims = dataclasses.replace(SMALL_PREFILL, cache_elem=CACHE_BF16)
    s = PrefillSession(device, kernels, dims, SEQS, SEQ_ROWS, position_bound=dims.context if staged else None)
    try:
        assert s.staged == staged
        assert all(l.params.get("cache_bf16") == 1 for l in s.lowered.launches if "cache_bf16" in l.params)
        weights, tokens = small_state(s.checked)
        s.write_weights(weights)
        for name in s.lowered.buffers:
            if name.startswith("cache:"):
                s.engine.zero(name)
        s.set_tokens(tokens)
        print(f"prefill small, bf16 caches, staged {staged}", flush=True)
        s.run()
        device.sync()
        lay = dims
        caches = {}
        for src in s.checked.program.sources:
            if type(src.kind).__name__ == "SCache":
                caches[src.name] = {u: np.zeros(lay.kv_heads * lay.context * lay.head_dim) for u in range(lay.slots)}
        positions = np.tile(np.arange(SEQ_ROWS), SEQS)
        slots = np.repeat(np.arange(SEQS), SEQ_ROWS)
        ev = evaluate_fast(s.checked, Bindings(
            SEQS * SEQ_ROWS, weights={k: np.asarray(v, np.float64) for k, v in weights.items()},
            row_ints={"tokens": tokens[:, None], "position": positions[:, None], "slot": slots[:, None]},
            caches=caches))
        got = s.logits()
        assert rel(got, ev.outputs["logits"]) <= BAR
        assert np.array_equal(s.tokens(), np.argmax(got, axis=1))
        for layer in range(lay.layers):
            for kv in ("k", "v"):
                name = f"l{layer}_{kv}_cache"
                bits = s.engine.read(f"cache:{name}").view(np.uint16).astype(np.uint32)
                g = (bits << 16).view(np.float32).astype(np.float64).reshape(lay.slots, lay.kv_heads, lay.context,
                                                                             lay.head_dim)
                w = np.stack([ev.caches[name][u] for u in range(lay.slots)]).reshape(g.shape)
                gw, ww = g[:, :, :SEQ_ROWS], w[:, :, :SEQ_ROWS]
                assert np.all(np.abs(gw - ww) <= BAR * np.max(np.abs(ww)) + 2.0 ** -7 * np.abs(ww)), name
                assert np.all(g[:, :, SEQ_ROWS:] == 0)
    finally:
        s.close()
