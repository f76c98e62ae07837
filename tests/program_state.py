"""Seeded state for any program of the program layer, the oracle's CPU
target run of its lowering, and the f64 evaluator on the same state: the
harness of the reference programs' tests (tests/programs.py).

Weights N(0, std) (one-dimensional ones, gains and scales, 1 + 0.1 N(0, 1)),
rounded to their type (bf16 as its bits); tables likewise; caches
N(0, 0.5) rounded to their element; inputs N(0, 1); row integers uniform
below their bounds unless given."""

from __future__ import annotations

import numpy as np

from furykernel_amd.lower import lower_plan, rope_table
from furykernel_amd.program.graph import BF16, F16, F32, Paged, SCache, SInput, SRowInts, STable, SWeight
from furykernel_amd.program.plan import PlanOptions, plan
from oracle.cpu_target import CpuTarget
from oracle.eval import Bindings, evaluate


def bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def widen(t: str, a) -> np.ndarray:
    """A type's stored elements as f32 (bf16 bits widened exactly)."""
    if t == BF16:
        return (np.asarray(a, np.uint32) << 16).view(np.float32)
    return np.asarray(a).astype(np.float32)


def rounded(t: str, x) -> np.ndarray:
    if t == BF16:
        return bf16_bits(x)
    return np.asarray(x, np.float16 if t == F16 else np.float32)


class State:
    """Every source's host values: ``weights`` (as stored: bf16 bits,
    f16, f32), ``tables`` [entries, ...], ``caches`` (flat, as stored),
    ``inputs`` (f32 rows), ``ints`` (u32)."""

    def __init__(self, checked, seed: int = 7, std: float = 0.3, ints: dict | None = None):
        rng = np.random.default_rng(seed)
        self.checked = checked
        self.weights, self.tables, self.caches, self.inputs, self.ints = {}, {}, {}, {}, {}
        ints = ints or {}
        for src in checked.program.sources:
            k = src.kind
            if isinstance(k, SWeight):
                n = int(np.prod(k.dims))
                v = 1 + 0.1 * rng.standard_normal(n) if len(k.dims) == 1 else std * rng.standard_normal(n)
                self.weights[src.name] = (k.type, rounded(k.type, v))
            elif isinstance(k, STable):
                n = int(np.prod(k.dims))
                self.tables[src.name] = (k.type, rounded(k.type, std * rng.standard_normal((k.entries, n))))
            elif isinstance(k, SCache):
                lay = k.layout
                n = (lay.blocks * lay.block_size if isinstance(lay, Paged) else lay.slots * lay.length) \
                    * lay.kv_heads * lay.head_dim
                elem = BF16 if k.elem == "bf16" else F16
                self.caches[src.name] = (elem, rounded(elem, 0.5 * rng.standard_normal(n)))
            elif isinstance(k, SInput):
                width = [v for v in checked.program.values if v.name == src.name][0].shape.width
                self.inputs[src.name] = rng.standard_normal(width).astype(np.float32)
            elif isinstance(k, SRowInts):
                self.ints[src.name] = np.asarray(ints.get(src.name, rng.integers(0, k.bound, k.count)), np.uint32)

    def bindings(self) -> Bindings:
        caches = {}
        for name, (t, v) in self.caches.items():
            src = self.checked.program.source_named(name)
            lay = src.kind.layout
            per = v.size // (lay.blocks if isinstance(lay, Paged) else lay.slots)
            flat = widen(t, v).astype(np.float64)
            n = lay.blocks if isinstance(lay, Paged) else lay.slots
            caches[name] = {s: flat[s * per:(s + 1) * per] for s in range(n)}
        return Bindings(
            1, inputs={n: [v.astype(np.float64)] for n, v in self.inputs.items()},
            weights={n: widen(t, v).astype(np.float64) for n, (t, v) in self.weights.items()},
            row_ints={n: [[int(i) for i in v]] for n, v in self.ints.items()},
            caches=caches,
            tables={n: [widen(t, e).astype(np.float64) for e in v] for n, (t, v) in self.tables.items()})

    def evaluate(self):
        return evaluate(self.checked, self.bindings())

    def load(self, target, lowered) -> None:
        """Writes the state into a CPU target or an engine (``write``)."""
        for name, (t, v) in self.weights.items():
            if f"weight:{name}" in lowered.buffers:
                target.write(f"weight:{name}", v)
            if f"widen:{name}" in lowered.buffers:
                target.write(f"widen:{name}", widen(t, v))
        for name, (t, v) in self.tables.items():
            if f"table:{name}" in lowered.buffers:
                target.write(f"table:{name}", v.reshape(-1))
        for name, (t, v) in self.caches.items():
            target.write(f"cache:{name}", v)
        for name, v in self.inputs.items():
            target.write(f"value:{name}", v)
        for name, v in self.ints.items():
            target.write(f"ints:{name}", v)

    def cpu(self, lowered, width: int = 64) -> CpuTarget:
        cpu = CpuTarget(lowered, width)
        for name, what in lowered.constants.items():
            if what[0] == "rope":
                cpu.write(name, rope_table(*what[1:]))
            elif what[0] == "ones":
                cpu.write(name, np.ones(lowered.buffers[name].count, np.float32))
        self.load(cpu, lowered)
        return cpu


def lowered(checked, gated: bool = False, store_gelus: bool = False):
    return lower_plan(checked, plan(PlanOptions(gated=gated, store_gelus=store_gelus), checked))


def output_buffers(checked) -> dict:
    """Each program output's name -> the value buffer holding it."""
    p = checked.program
    return {o.name: f"value:{p.value(o.value).name}" for o in p.outputs}


def rel(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    scale = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / scale) if scale else float(np.max(np.abs(a - b)))
