"""The IR target on the GPU: every case kernel (test/cpu/Cases.hs's and
InterpTest.hs's, built for 64-lane SIMD groups) lowered to HIP by
furykernel_amd/ir/rocm.py, compiled by hipRTC through the C ABI
(fk_rtc_compile), launched through its launch table, and every output
compared with the oracle's interpreter on the same inputs: bit for bit; an
output of arithmetic that is a NaN by class (quiet or signalling); rsqrt,
exp, log and tanh within one unit in the last place of the operand's type,
the bound the target states (binary64's functions rounded once: the device
library's binary64 and the host's libm can differ in a last binary64 bit,
which moves the rounded result only next to a midpoint).

The interpreter runs first: its bounds checks hold every access of the
launch inside the buffers the GPU is given."""

import numpy as np
import pytest

from furykernel_amd.ir.runtime import Unit
from gpu_ir_cases import CASES, lowered_unit
from oracle import interp

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def unit(device):
    print("compiling the IR cases' unit with hipRTC", flush=True)
    return Unit(device, lowered_unit(), "cases.hip")


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view({4: np.uint32, 2: np.uint16, 1: np.uint8}[a.dtype.itemsize]).astype(np.int64)


def _ordered(bits, width):
    sign = 1 << (width - 1)
    return np.where(bits & sign, -(bits & (sign - 1)), bits)


def _nan(bits, width):
    if width == 32:
        return ((bits & 0x7F800000) == 0x7F800000) & ((bits & 0x7FFFFF) != 0)
    return ((bits & 0x7C00) == 0x7C00) & ((bits & 0x3FF) != 0)


def _quiet(bits, width):
    return (bits & (0x400000 if width == 32 else 0x200)) != 0


def compare(name, got, want, by_class: bool, within_ulp: bool):
    """The mismatching elements' count."""
    g, w = _bits(got), _bits(want)
    width = 8 * np.asarray(want).dtype.itemsize
    same = g == w
    if by_class and width in (16, 32) and np.asarray(want).dtype != np.uint32:
        both = _nan(g, width) & _nan(w, width) & (_quiet(g, width) == _quiet(w, width))
        same |= both
    if within_ulp and width in (16, 32):
        close = np.abs(_ordered(g, width) - _ordered(w, width)) <= 1
        off = close & ~same & ~_nan(w, width) & ~_nan(g, width)
        print(f"  {name}: {int(off.sum())} of {len(w)} one unit in the last place from the host's", flush=True)
        assert off.sum() <= max(1, len(w) // 1000), "more than one in a thousand off the host's bits"
        same |= off
    bad = int((~same).sum())
    if bad:
        i = int(np.flatnonzero(~same)[0])
        print(f"  {name}: {bad} of {len(w)} differ, first at {i}: {int(g[i]):#x} against {int(w[i]):#x}", flush=True)
    return bad


@pytest.mark.parametrize("case", list(CASES), ids=lambda c: c.id)
def test_case_on_the_gpu_is_the_interpreters(device, unit, case):
    k = case.kernel
    for r, (params, buffers, tables) in enumerate(case.runs):
        want, want_tables = interp.run(k, 64, params, buffers, tables)
        print(f"IR case {case.id} run {r}: {k.threads} threads", flush=True)
        bufs = {n: device.upload(np.ascontiguousarray(a)) for n, a in buffers.items()}
        entries, tabs = {}, {}
        for t in k.tables:
            arrays = [None if a is None else device.upload(np.ascontiguousarray(a)) for a in tables[t.name]]
            entries[t.name] = arrays
            addrs = np.array([0 if a is None else a.ptr for a in arrays], np.uint64)
            tabs[t.name] = device.upload(addrs)
        try:
            unit.launch(k.name, params, bufs, tabs)
            device.sync()
            bad = 0
            for b in k.buffers:
                if b.access == "read":
                    continue
                got = bufs[b.name].read(want[b.name].dtype, len(want[b.name]))
                bad += compare(b.name, got, want[b.name], b.name in case.by_class, b.name in case.transcendental)
            for t in k.tables:
                if t.access == "read":
                    continue
                for e, a in enumerate(entries[t.name]):
                    if a is not None:
                        w = want_tables[t.name][e]
                        bad += compare(f"{t.name}[{e}]", a.read(w.dtype, len(w)), w, False, False)
            assert bad == 0
        finally:
            for x in list(bufs.values()) + list(tabs.values()) + [a for v in entries.values() for a in v if a]:
                x.free()
