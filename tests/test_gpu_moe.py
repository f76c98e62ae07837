"""Routed experts on the GPU: the lowered MoE step (the norm, the router's
GEMV step, fk_step_route, the routed GEMVs over tables of experts, the gated
GELU over the ranks' rows, the combine of the ranks and its residual) through
the engine, every buffer bit for bit the oracle's CPU target's, at small
shapes and at a 1B-class width (16 experts of 1024, 2 a row); and the route
kernel alone against the oracle over ties and NaNs."""

import numpy as np
import pytest

from furykernel_amd import kernels as K
from furykernel_amd import runtime
from furykernel_amd.engine import Engine
from moe_cases import CASES, ONE_B_MOE, case_id, lowered, moe_program, run_cpu, state
from oracle import fkref

pytestmark = pytest.mark.gpu


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view({4: np.uint32, 2: np.uint16, 8: np.uint64}[a.dtype.itemsize])


@pytest.mark.parametrize("case", CASES + [ONE_B_MOE], ids=case_id)
def test_moe_step_bit_exact(device, kernels, case):
    checked = moe_program(case)
    low = lowered(checked)
    w, x = state(case)
    print(f"moe step {case_id(case)}: {[L.entry for L in low.launches]}", flush=True)
    eng = Engine(device, kernels, low)
    try:
        eng.write_weights({k: v.ravel() for k, v in w.items()})
        eng.write("value:x", x)
        eng.enqueue()
        device.sync()
        cpu = run_cpu(low, w, x)
        bad = [n for n in low.buffers if not n.startswith(("tableaddr:", "addr:"))
               and not np.array_equal(bits(eng.read(n)), bits(cpu.read(n)))]
        assert bad == []
    finally:
        eng.close()


@pytest.mark.parametrize("n,k,scaled", [(64, 8, True), (16, 4, False), (2048, 2, False), (8, 8, True)])
def test_route_kernel_against_the_oracle(device, kernels, n, k, scaled):
    rng = np.random.default_rng(n * 10 + k)
    L = fkref.lib()
    for trial in range(6):
        x = rng.standard_normal(n).astype(np.float32)
        if trial == 1:
            x[: n // 2] = x[0]  # ties: the lower index first
        if trial == 2:
            x[1] = np.nan  # a NaN ranked last
        if trial == 3:
            x[:] = 0.0
            x[n // 2] = -0.0
        s = (1 + 0.3 * rng.standard_normal(n)).astype(np.float32)
        bx, bs = device.upload(x), device.upload(s)
        bi, bw = device.alloc(k * 4), device.alloc(k * 4)
        params = K.RouteParams(n, k, int(scaled))
        spans = [(bx.ptr, bx.size), (bs.ptr, bs.size), (bi.ptr, bi.size), (bw.ptr, bw.size)]
        runtime.launch_check("fk_step_route", 1, 64, 0, spans, params)
        print(f"route n {n} k {k} trial {trial}", flush=True)
        kernels.launch("fk_step_route", 1, 64, {"x": bx.ptr, "scale": bs.ptr, "ids": bi.ptr, "ws": bw.ptr}, params)
        device.sync()
        ids, ws = bi.read(np.uint32, k), bw.read(np.float32, k)
        want_i, want_w = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        assert L.fkref_route(x.ctypes.data, s.ctypes.data if scaled else None, want_i.ctypes.data,
                             want_w.ctypes.data, n, k, int(scaled)) == 0
        assert ids.tolist() == want_i.tolist()
        assert np.array_equal(bits(ws), bits(want_w))
        for b in (bx, bs, bi, bw):
            b.free()
