"""The decode attention and its combine launched directly through the C ABI,
against the oracle's restatement bit for bit, over shapes the planned models
do not reach: groups of 1 to 8 query heads a kv head (two heads a lane at 8),
head widths 8 to 64, splits of 64 and 128 positions, f16 and bf16 caches, a
window, the new key and value rows stored first (the key RoPE'd or not), a
position just past a split's start, and the 1B shape with every split full
and short of full.
Compared: both caches after the store, the partials, the combined rows."""

import numpy as np
import pytest

from attention_cases import CASES, WIDE, case_id, inputs, oracle, oracle_wide, within_bounds
from furykernel_amd import kernels as K

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint16)


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_attention_and_combine_match_the_oracle(device, kernels, case):
    x = inputs(case)
    heads, kv, d, splits = x["heads"], x["kv"], x["d"], x["splits"]
    n_part = heads * splits * (d + 2)
    print(f"decode attention {case_id(case)}", flush=True)

    # The device: the attention (storing the new rows first, if asked), then the combine.
    b = {name: device.upload(x[key]) for name, key in (("q", "q"), ("knew", "knew"), ("vnew", "vnew"), ("kc", "kc"),
                                                        ("vc", "vc"), ("rope", "table"))}
    b["position"] = device.upload(np.array([x["pos"]], np.uint32))
    b["slot"] = device.upload(np.array([0], np.uint32))
    partials = device.upload(np.zeros(n_part, np.float32))
    out = device.upload(np.zeros(heads * d, np.float32))
    params = K.StepAttendParams(heads, kv, d, x["length"], 1, splits, x["split"], x["rope"], x["rotated"],
                                x["length"], x["scale"], x["window"], x["bf16"], x["store"],
                                x["rope"] if x["store"] else 0)
    kernels.launch("fk_step_attend", kv * splits, 512, {**{k: v.ptr for k, v in b.items()}, "partials": partials.ptr,
                                                       "reach": 0}, params)
    kernels.launch("fk_step_combine", heads, 64, {"partials": partials.ptr, "out": out.ptr},
                   K.StepCombineParams(heads, d, splits))
    device.sync()
    g = dict(kc=b["kc"].read(np.uint16, x["kc"].size), vc=b["vc"].read(np.uint16, x["vc"].size),
             partials=partials.read(np.float32, n_part), out=out.read(np.float32, heads * d))
    for buf in (*b.values(), partials, out):
        buf.free()

    # The oracle, the same inputs: caches, partials and rows bit for bit.
    o = oracle(x)
    assert np.array_equal(g["kc"], o["kc"]) and np.array_equal(g["vc"], o["vc"])
    assert np.array_equal(bits(g["partials"]), bits(o["partials"])), int(np.sum(bits(g["partials"]) !=
                                                                                 bits(o["partials"])))
    assert np.array_equal(bits(g["out"]), bits(o["out"])), int(np.sum(bits(g["out"]) != bits(o["out"])))
    assert np.all(np.isfinite(g["out"]))
    # And binary64 attention over the caches the GPU left: the first query
    # head's elements within their attendBounds bounds, every head within
    # 1e-4 (1e-5 given the same RoPE table).
    within_bounds(x, g, g["out"], [0])


@pytest.mark.parametrize("case,split", WIDE, ids=[f"{case_id(c)}_S{S}" for c, S in WIDE])
def test_wide_attention_matches_the_oracle(device, kernels, case, split):
    """fk_step_attend_wide: splits of `split` positions, 64 a wavefront, one
    threadgroup of split/64 wavefronts a (kv head, split); checked on the
    host by the launch table's checks first, then against the oracle's wide
    restatement bit for bit (caches, partials) and, after the combine
    launch, the rows bit for bit and within the binary64 bars."""
    from furykernel_amd import runtime
    from furykernel_amd.lower import wide_lds_floats

    x = inputs(case)
    heads, kv, d = x["heads"], x["kv"], x["d"]
    waves = split // 64
    splits = -(-x["length"] // split)
    n_part = heads * splits * (d + 2)
    threads, lds = 64 * waves, 4 * wide_lds_floats(waves)
    print(f"wide decode attention {case_id(case)} split {split}", flush=True)

    b = {name: device.upload(x[key]) for name, key in (("q", "q"), ("knew", "knew"), ("vnew", "vnew"), ("kc", "kc"),
                                                        ("vc", "vc"), ("rope", "table"))}
    b["position"] = device.upload(np.array([x["pos"]], np.uint32))
    b["slot"] = device.upload(np.array([0], np.uint32))
    partials = device.upload(np.zeros(n_part, np.float32))
    out = device.upload(np.zeros(heads * d, np.float32))
    bound = {**{k: v for k, v in b.items()}, "partials": partials}
    params = K.StepAttendParams(heads, kv, d, x["length"], 1, splits, split, x["rope"], x["rotated"],
                                x["length"], x["scale"], x["window"], x["bf16"], x["store"],
                                x["rope"] if x["store"] else 0)
    entry = "fk_step_attend_wide"
    spans = [(bound[n].ptr, bound[n].size) if n in bound else (0, 0) for n in K.ABIS[entry].buffers]
    runtime.launch_check(entry, kv * splits, threads, lds, spans, params)
    kernels.launch(entry, kv * splits, threads, {**{k: v.ptr for k, v in bound.items()}, "reach": 0}, params,
                   lds_bytes=lds)
    kernels.launch("fk_step_combine", heads, 64, {"partials": partials.ptr, "out": out.ptr},
                   K.StepCombineParams(heads, d, splits))
    device.sync()
    g = dict(kc=b["kc"].read(np.uint16, x["kc"].size), vc=b["vc"].read(np.uint16, x["vc"].size),
             partials=partials.read(np.float32, n_part), out=out.read(np.float32, heads * d))
    for buf in (*b.values(), partials, out):
        buf.free()

    o = oracle_wide(x, split)
    assert np.array_equal(g["kc"], o["kc"]) and np.array_equal(g["vc"], o["vc"])
    assert np.array_equal(bits(g["partials"]), bits(o["partials"])), int(np.sum(bits(g["partials"]) !=
                                                                                 bits(o["partials"])))
    assert np.array_equal(bits(g["out"]), bits(o["out"])), int(np.sum(bits(g["out"]) != bits(o["out"])))
    within_bounds(x, g, g["out"], [0])
