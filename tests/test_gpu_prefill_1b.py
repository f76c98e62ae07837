"""The 1B-class prefill at its real shapes (4 sequences of 2048 rows into
rings of 4096, d 2048, 32 heads of 64 over 8 kv heads, FFN 8192, vocab 32000,
f16) on the GPU against the binary64 evaluator (src/FuryKernel/Program/
Eval.hs, restated in oracle/eval.py; the plan: Plan.hs:270-300, the ring
fitting in place at position bound 2048).

* The planned prefill of two layers of the 1B model (every kernel at its 1B
  shape: the QKV GEMM with RoPE and the KV store in its epilogue, the causal
  attention over 2048-row sequences, the O / gate-up / down GEMMs, the
  logits GEMM over 32000 columns and the per-row argmax): the logits of every
  row of sequences 0 and 3 and the KV rows of their slots within the f16 bar,
  2e-3 of the largest magnitude, of the evaluator over those sequences'
  rows; each row's token the argmax of its logits.
* The causal attention alone (fk_prefill_attend_g4) over 4 x 2048 rows with
  f16 and bf16 caches: sampled rows against binary64 attention of the same
  values.
"""

import numpy as np
import pytest

from furykernel_amd.program.decoder import ONE_B_PREFILL
from oracle.eval import Bindings, evaluate_fast

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(300)]

SEQS, SEQ_ROWS, LAYERS = 4, 2048, 2
BAR = 2e-3
EVALUATED = (0, 3)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.fixture(scope="module")
def run(device, kernels):
    from furykernel_amd.prefill import PrefillSession

    s = PrefillSession(device, kernels, ONE_B_PREFILL, SEQS, SEQ_ROWS, layers=LAYERS)
    rng = np.random.default_rng(2026)
    weights = {}
    for src in s.checked.program.sources:
        if type(src.kind).__name__ != "SWeight":
            continue
        dims = src.kind.dims
        if len(dims) == 1:
            weights[src.name] = (1 + 0.1 * rng.standard_normal(dims[0])).astype(np.float32)
        elif src.name == "embed":
            weights[src.name] = (0.5 * rng.standard_normal(dims)).astype(np.float16)
        else:
            weights[src.name] = (0.02 * rng.standard_normal(dims)).astype(np.float16)
    tokens = rng.integers(0, ONE_B_PREFILL.vocab, SEQS * SEQ_ROWS)
    s.write_weights(weights)
    for name in s.lowered.buffers:
        if name.startswith("cache:"):
            s.engine.zero(name)
    s.set_tokens(tokens)
    print(f"prefill 1B shapes, {LAYERS} layers, {SEQS}x{SEQ_ROWS} rows: {len(s.lowered.launches)} launches",
          flush=True)
    s.run()
    device.sync()
    V = ONE_B_PREFILL.vocab
    logits_buf = s.engine.buffers["value:logits"]
    got = {u: logits_buf.read(np.float32, SEQ_ROWS * V, u * SEQ_ROWS * V * 4).reshape(SEQ_ROWS, V)
           for u in EVALUATED}
    lay = ONE_B_PREFILL
    evals = {}
    for u in EVALUATED:
        print(f"evaluating sequence {u} in binary64", flush=True)
        caches = {src.name: {u: np.zeros(lay.kv_heads * lay.context * lay.head_dim)}
                  for src in s.checked.program.sources if type(src.kind).__name__ == "SCache"}
        rows = slice(u * SEQ_ROWS, (u + 1) * SEQ_ROWS)
        evals[u] = evaluate_fast(s.checked, Bindings(
            SEQ_ROWS, weights={k: np.asarray(v, np.float64) for k, v in weights.items()},
            row_ints={"tokens": tokens[rows, None], "position": np.arange(SEQ_ROWS)[:, None],
                      "slot": np.full((SEQ_ROWS, 1), u)},
            caches=caches))
    yield s, got, evals
    s.close()


def test_1b_prefill_logits_within_the_f16_bar(run):
    s, got, evals = run
    for u in EVALUATED:
        want = evals[u].outputs["logits"]
        assert rel(got[u], want) <= BAR, u
        for r in (0, 1, 31, 32, 1000, 2047):
            assert rel(got[u][r], want[r]) <= 4 * BAR, (u, r)


def test_1b_prefill_fills_the_rings_within_the_f16_bar(run):
    s, got, evals = run
    lay = ONE_B_PREFILL
    for layer in range(LAYERS):
        for kv in ("k", "v"):
            name = f"l{layer}_{kv}_cache"
            ring = s.cache(name).astype(np.float64).reshape(lay.slots, lay.kv_heads, lay.context, lay.head_dim)
            for u in EVALUATED:
                want = evals[u].caches[name][u].reshape(lay.kv_heads, lay.context, lay.head_dim)
                assert rel(ring[u, :, :SEQ_ROWS], want[:, :SEQ_ROWS]) <= BAR, (name, u)
            assert np.all(ring[:, :, SEQ_ROWS:] == 0), name


def test_1b_prefill_tokens_are_each_rows_argmax(run):
    s, got, evals = run
    tokens = s.tokens()
    for u in EVALUATED:
        mine = tokens[u * SEQ_ROWS:(u + 1) * SEQ_ROWS]
        assert np.array_equal(mine, np.argmax(got[u], axis=1)), u
        want = evals[u].outputs["logits"]
        top2 = np.sort(want, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 8 * BAR * np.max(np.abs(want))
        assert clear.sum() > SEQ_ROWS // 2
        assert np.array_equal(mine[clear], np.argmax(want, axis=1)[clear]), u


@pytest.mark.parametrize("bf16", [0, 1], ids=["f16-caches", "bf16-caches"])
def test_causal_attention_over_2048_row_sequences_against_f64(device, kernels, bf16):
    """fk_prefill_attend_g4 over 4 sequences of 2048 rows (positions 0..2047
    of slots 0..3), 32 heads over 8, a ring of 4096; sampled rows of each
    sequence against binary64 attention of the same cache values (bf16 caches
    are read into f16 in the kernel: values this test draws are far inside
    f16's range)."""
    from furykernel_amd.layout import unpack

    rng = np.random.default_rng(77 + bf16)
    rows, heads, kvh, length, slots, d = SEQS * SEQ_ROWS, 32, 8, 4096, 4, 64
    scale = 0.125
    q = rng.standard_normal((rows, heads * d)).astype(np.float16)
    kf = rng.standard_normal((slots, kvh, length, d)).astype(np.float32)
    vf = rng.standard_normal((slots, kvh, length, d)).astype(np.float32)
    if bf16:
        kc, vc = ((x.view(np.uint32) >> 16).astype(np.uint16) for x in (kf, vf))
        widen = lambda c: (c.astype(np.uint32) << 16).view(np.float32).astype(np.float64)  # noqa: E731
    else:
        kc, vc = (x.astype(np.float16).view(np.uint16) for x in (kf, vf))
        widen = lambda c: c.view(np.float16).astype(np.float64)  # noqa: E731
    positions = np.tile(np.arange(SEQ_ROWS), SEQS).astype(np.uint32)
    seqs = np.repeat(np.arange(SEQS), SEQ_ROWS).astype(np.uint32)
    bufs = [device.upload(x) for x in (q, kc, vc, positions, seqs)]
    out = device.alloc(rows * heads * d * 2)
    print(f"prefill attention g4 over {SEQS}x{SEQ_ROWS} rows, bf16 {bf16}", flush=True)
    kernels.prefill_attend(*bufs, out, rows, heads, kvh, length, slots, scale, cache_bf16=bool(bf16),
                           positions=positions, seqs=seqs)
    device.sync()
    got = unpack(out.read(np.float16, rows * heads * d), rows, heads * d).astype(np.float64)
    K, V = widen(kc).reshape(kf.shape), widen(vc).reshape(vf.shape)
    sample = [r + u * SEQ_ROWS for u in range(SEQS) for r in (0, 1, 31, 32, 63, 64, 500, 1023, 1024, 2046, 2047)]
    for r in sample:
        p, sl = int(positions[r]), int(seqs[r])
        want = np.empty((heads, d))
        for h in range(heads):
            g = h // (heads // kvh)
            sc = scale * (K[sl, g, :p + 1] @ q[r, h * d:(h + 1) * d].astype(np.float64))
            e = np.exp(sc - sc.max())
            want[h] = (e / e.sum()) @ V[sl, g, :p + 1]
        assert rel(got[r], want.reshape(-1)) <= BAR, (r, rel(got[r], want.reshape(-1)))
    for b in bufs + [out]:
        b.free()
