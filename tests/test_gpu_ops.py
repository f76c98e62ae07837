"""The library's one-call decode attention (include/fkrocm_ops.h:
fk_attend_decode) on the GPU through the C ABI: caches and rows bit for bit
the oracle's (the planned step's kernels and order), on shapes in turn that
grow and shrink its workspace, and the calls refused for what the kernels do
not take."""

import ctypes

import numpy as np
import pytest

from attention_cases import CASES, case_id, inputs, oracle
from furykernel_amd import kernels as K
from furykernel_amd import runtime

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint16)


def run_op(device, x, entry="fk_attend_decode"):
    """The operation on the case's inputs: (caches, rows) as the GPU left them."""
    heads, kv, d = x["heads"], x["kv"], x["d"]
    b = {k: device.upload(x[v]) for k, v in (("q", "q"), ("knew", "knew"), ("vnew", "vnew"), ("kc", "kc"),
                                              ("vc", "vc"), ("rope", "table"))}
    b["position"] = device.upload(np.array([x["pos"]], np.uint32))
    b["slot"] = device.upload(np.array([0], np.uint32))
    out = device.upload(np.zeros(heads * d, np.float32))
    p = K.StepAttendParams(heads, kv, d, x["length"], 1, x["splits"], x["split"], x["rope"], x["rotated"],
                           x["length"], x["scale"], x["window"], x["bf16"], x["store"], x["rope"] if x["store"] else 0)
    args = K.AttendArgs(b["q"].ptr, b["knew"].ptr, b["vnew"].ptr, b["kc"].ptr, b["vc"].ptr, b["position"].ptr,
                        b["slot"].ptr, b["rope"].ptr, out.ptr, p)
    try:
        runtime.attend_decode(device, args, entry=entry)
        device.sync()
        return (b["kc"].read(np.uint16, x["kc"].size), b["vc"].read(np.uint16, x["vc"].size),
                out.read(np.float32, heads * d))
    finally:
        for buf in (*b.values(), out):
            buf.free()


def test_attend_decode_matches_the_oracle_in_turn(device):
    # the 1B shape, then smaller and larger workspaces in turn
    for case in (CASES[6], CASES[4], CASES[0], CASES[8], CASES[3]):
        print(f"fk_attend_decode {case_id(case)}", flush=True)
        x = inputs(case)
        kc, vc, out = run_op(device, x)
        o = oracle(x)
        assert np.array_equal(kc, o["kc"]) and np.array_equal(vc, o["vc"])
        assert np.array_equal(bits(out), bits(o["out"])), int(np.sum(bits(out) != bits(o["out"])))


def test_attend_decode_refuses_what_the_kernels_do_not_take(device):
    x = inputs(CASES[4])
    bad = K.AttendArgs(0, 0, 0, 0, 0, 0, 0, 0, 0,
                       K.StepAttendParams(4, 3, 8, 128, 1, 2, 64, 0, 0, 1, 0.5, 0, 0, 0, 0))
    with pytest.raises(runtime.FkError) as err:
        runtime.attend_decode(device, bad)
    assert err.value.status == -2
    assert x is not None
