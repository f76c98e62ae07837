"""The reference's own program-layer test programs on the GPU through the C
ABI (tests/test_reference_programs.py runs them on the CPU target): every
buffer a launch writes bit for bit the oracle's CPU target's from the same
device state, and every output within 1e-4 of the f64 evaluator.  layer
and its k = v form, two_tiles, embed (gather scaled by 5.65625), pooled
(three rows summed, a linear layer over rows of 4), and predicting, ungated and gated (bf16 expert tables)."""

import numpy as np
import pytest

from furykernel_amd.engine import Engine
from furykernel_amd.program.check import check_program
from oracle.cpu_target import CpuTarget
from program_state import State, lowered
from test_reference_programs import CASES, check_outputs

pytestmark = pytest.mark.gpu


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("gated", [False, True], ids=["ungated", "gated"])
@pytest.mark.parametrize("name", sorted(CASES))
def test_reference_program_on_the_gpu(device, kernels, name, gated):
    make, ints = CASES[name]
    checked = check_program(make())
    low = lowered(checked, gated=gated)
    st = State(checked, seed=7, ints=ints)
    eng = Engine(device, kernels, low)
    try:
        st.load(eng, low)
        device.sync()
        cpu = CpuTarget(low, 64)
        for n in low.buffers:
            cpu.write(n, eng.read(n))
        print(f"{name} ({'gated' if gated else 'ungated'}): {len(low.launches)} launches "
              f"{sorted({L.entry for L in low.launches})}", flush=True)
        eng.enqueue()
        device.sync()
        cpu.run()
        bad = [(n, int(np.sum(bits(eng.read(n)) != bits(cpu.read(n))))) for n in low.buffers
               if not np.array_equal(bits(eng.read(n)), bits(cpu.read(n)))]
        assert bad == []
        errs = check_outputs(checked, st, eng.read)
        assert max(errs.values()) <= 1e-4, errs
    finally:
        eng.close()
