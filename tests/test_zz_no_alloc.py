"""fk_attend_decode_noalloc (include/fkrocm_ops.h) on the GPU through the C
ABI: its caches and rows bit for bit fk_attend_decode's (and the oracle's),
on two calls in a row, the second smaller (the scratch then holds the first
call's partials, which the second overwrites), and a step too large for the
scratch refused."""

import numpy as np
import pytest

from attention_cases import CASES, case_id, inputs, oracle
from furykernel_amd import kernels as K
from furykernel_amd import runtime
from test_gpu_ops import bits, run_op

pytestmark = pytest.mark.gpu


def test_noalloc_matches_the_allocating_entry_on_two_calls(device):
    for case in (CASES[6], CASES[5]):  # the 1B shape (270 KB of partials), then a smaller one
        print(f"fk_attend_decode_noalloc {case_id(case)}", flush=True)
        x = inputs(case)
        kc_n, vc_n, out_n = run_op(device, x, entry="fk_attend_decode_noalloc")
        kc_a, vc_a, out_a = run_op(device, x, entry="fk_attend_decode")
        assert np.array_equal(kc_n, kc_a) and np.array_equal(vc_n, vc_a)
        assert np.array_equal(bits(out_n), bits(out_a)), int(np.sum(bits(out_n) != bits(out_a)))
        o = oracle(x)
        assert np.array_equal(bits(out_n), bits(o["out"]))


def test_noalloc_refuses_a_step_past_its_scratch(device):
    # 64 heads over 8, width 64, a ring of 65536 in splits of 128: 512 splits,
    # 64 * 512 * 66 * 4 = 8.65 MB of partials, past the 4 MiB scratch; refused
    # before anything is launched (the addresses are never read).
    p = K.StepAttendParams(64, 8, 64, 65536, 1, 512, 128, 0, 0, 1, 0.125, 0, 0, 0, 0)
    args = K.AttendArgs(256, 256, 256, 256, 256, 256, 256, 256, 256, p)
    with pytest.raises(runtime.FkError) as err:
        runtime.attend_decode(device, args, entry="fk_attend_decode_noalloc")
    assert err.value.status == -3 and "static scratch holds" in err.value.message
