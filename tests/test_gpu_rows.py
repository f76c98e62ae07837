"""Steps of any number of rows on the GPU, through the prefill kernels,
against the f64 evaluator (the f16 bar, 2e-3 of the largest magnitude):

- a ragged prefill: one sequence of 100 rows, and two of 100 (runs of 128,
  the step filled out to 256 rows in the caches' scratch slot): every real
  row's logits, the KV rows it fills, the ring past them untouched;
- a decode step of four rows (Eval.hs:126-140), four sequences at positions
  5, 40, 200 and 255 of slots 0, 3, 1, 2 over caches holding earlier keys:
  each row's logits, the one KV row each stores, every other cache row
  untouched (the small decoder, and two layers of the 1B shapes at
  positions up to 4095)."""

import dataclasses

import numpy as np
import pytest

from furykernel_amd.program.decoder import ONE_B, SMALL_PREFILL
from oracle.eval import Bindings, evaluate_fast
from test_gpu_prefill import BAR, rel, small_state

pytestmark = pytest.mark.gpu


def caches_of(s, dims):
    """The program's caches as the device holds them (the real slots)."""
    out = {}
    for src in s.checked.program.sources:
        if type(src.kind).__name__ == "SCache":
            per = dims.kv_heads * dims.context * dims.head_dim
            a = s.cache(src.name).astype(np.float64)
            out[src.name] = {u: a[u * per:(u + 1) * per] for u in range(dims.slots)}
    return out


@pytest.mark.parametrize("seqs", [1, 2])
def test_a_ragged_prefill_of_100_rows(device, kernels, seqs):
    from furykernel_amd.prefill import PrefillSession

    rows = 100
    dims = SMALL_PREFILL
    s = PrefillSession(device, kernels, dims, seqs, rows)
    try:
        assert s.rows == 256 and s.run_rows == 128 and len(s.real) == seqs * rows
        weights, tokens = small_state(s.checked)
        tokens = tokens[:seqs * rows]
        s.write_weights(weights)
        for name in s.lowered.buffers:
            if name.startswith("cache:"):
                s.engine.zero(name)
        s.set_tokens(tokens)
        print(f"ragged prefill: {seqs} x {rows} rows in a step of {s.rows}", flush=True)
        s.run()
        device.sync()
        zero = {n: {u: np.zeros(dims.kv_heads * dims.context * dims.head_dim) for u in range(dims.slots)}
                for n in caches_of(s, dims)}
        ev = evaluate_fast(s.checked, Bindings(
            seqs * rows, weights={k: np.asarray(v, np.float64) for k, v in weights.items()},
            row_ints={"tokens": tokens[:, None], "position": np.tile(np.arange(rows), seqs)[:, None],
                      "slot": np.repeat(np.arange(seqs), rows)[:, None]}, caches=zero))
        got = s.logits()
        assert got.shape == ev.outputs["logits"].shape
        assert rel(got, ev.outputs["logits"]) <= BAR
        held = caches_of(s, dims)
        for name in held:
            for u in range(dims.slots):
                g = held[name][u].reshape(dims.kv_heads, dims.context, dims.head_dim)
                w = ev.caches[name][u].reshape(g.shape)
                if u < seqs:
                    assert rel(g[:, :rows], w[:, :rows]) <= BAR, (name, u)
                assert np.all(g[:, rows:] == 0) if u < seqs else np.all(g == 0), (name, u)
    finally:
        s.close()


def host_weights(checked, std, seed=31):
    """Weights for any decoder program: gains 1 + 0.1 N(0, 1) in f32, the
    embedding 0.5 N(0, 1) and every other weight std N(0, 1) in f16."""
    rng = np.random.default_rng(seed)
    out = {}
    for src in checked.program.sources:
        if type(src.kind).__name__ != "SWeight":
            continue
        dims = src.kind.dims
        if len(dims) == 1:
            out[src.name] = (1 + 0.1 * rng.standard_normal(dims[0])).astype(np.float32)
        else:
            out[src.name] = ((0.5 if src.name == "embed" else std) * rng.standard_normal(dims)).astype(np.float16)
    return out


@pytest.mark.parametrize("which", ["small", "1b"])
def test_a_decode_step_of_four_rows(device, kernels, which):
    from furykernel_amd.prefill import DecodeRows

    if which == "small":
        dims, layers, std = dataclasses.replace(SMALL_PREFILL, slots=4), None, 0.05
        positions = [5, 40, 200, 255]
    else:
        dims, layers, std = dataclasses.replace(ONE_B, slots=4), 2, 0.02
        positions = [5, 1000, 4094, 4095]
    slots = [0, 3, 1, 2]
    s = DecodeRows(device, kernels, dims, positions, slots, layers=layers)
    try:
        rng = np.random.default_rng(3)
        weights = host_weights(s.checked, std)
        s.write_weights(weights)
        for i, name in enumerate(sorted(n for n in s.lowered.buffers if n.startswith("cache:"))):
            s.engine.init_normal(name, 2027 + 7919 * i, 0.5)
        device.sync()
        before = caches_of(s, dims)
        tokens = rng.integers(0, dims.vocab, 4)
        s.set_tokens(tokens)
        print(f"decode step of 4 rows ({which}): {len(s.lowered.launches)} launches in a step of {s.rows}",
              flush=True)
        s.run()
        device.sync()
        ev = evaluate_fast(s.checked, Bindings(
            4, weights={k: np.asarray(v, np.float64) for k, v in weights.items()},
            row_ints={"tokens": np.asarray(tokens)[:, None], "position": np.asarray(positions)[:, None],
                      "slot": np.asarray(slots)[:, None]}, caches=before))
        got = s.logits()
        assert got.shape == (4, dims.vocab)
        assert rel(got, ev.outputs["logits"]) <= BAR
        for r in range(4):
            assert rel(got[r], ev.outputs["logits"][r]) <= 4 * BAR
        after = caches_of(s, dims)
        for name in after:
            for u in range(dims.slots):
                g = after[name][u].reshape(dims.kv_heads, dims.context, dims.head_dim)
                b = before[name][u].reshape(g.shape)
                w = ev.caches[name][u].reshape(g.shape)
                p = positions[slots.index(u)]
                assert rel(g[:, p], w[:, p]) <= BAR, (name, u)   # the row it stored
                assert np.array_equal(np.delete(g, p, axis=1), np.delete(b, p, axis=1)), (name, u)
    finally:
        s.close()
