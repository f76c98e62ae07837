"""The decode attention and its combine launched directly through the C ABI,
against the oracle's restatement bit for bit, over shapes the planned models
do not reach: groups of 1 to 8 query heads a kv head (two heads a lane at 8),
head widths 8 to 64, splits of 64 and 128 positions, f16 and bf16 caches, a
window, the new key and value rows stored first (the key RoPE'd or not), a
position just past a split's start, and the 1B shape with every split full.
Compared: both caches after the store, the partials, the combined rows."""

import numpy as np
import pytest

from furykernel_amd import kernels as K
from furykernel_amd.lower import rope_table
from oracle import fkref

pytestmark = pytest.mark.gpu

THETA = 10000.0

# heads, kv_heads, head_dim, split, length, position, window, bf16, rope, store
CASES = [
    (32, 4, 64, 128, 1024, 1000, 0, 0, 1, 1),
    (16, 4, 64, 64, 512, 200, 0, 0, 0, 0),
    (8, 4, 32, 128, 512, 300, 0, 1, 1, 1),
    (8, 1, 64, 128, 256, 250, 48, 0, 1, 0),
    (4, 4, 8, 64, 128, 70, 0, 0, 0, 1),
    (6, 2, 16, 128, 256, 128, 0, 1, 1, 1),
    (32, 8, 64, 128, 4096, 4095, 0, 0, 1, 1),
]


def cache(rng, n, bf16):
    x = rng.standard_normal(n).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16) if bf16 else x.astype(np.float16).view(np.uint16)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint16)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "h{}_kv{}_d{}_s{}_p{}_w{}_bf{}_r{}_st{}".format(
    c[0], c[1], c[2], c[3], c[5], c[6], c[7], c[8], c[9]))
def test_attention_and_combine_match_the_oracle(device, kernels, case):
    heads, kv, d, split, length, pos, window, bf16, rope, store = case
    rng = np.random.default_rng(heads * 1000 + d * 10 + split + pos)
    splits = -(-length // split)
    rotated = d // 2
    scale = float(np.float32(1.0 / np.sqrt(d)))
    theta = float(np.float32(THETA))
    q = (rng.standard_normal(heads * d) * 0.5).astype(np.float32)
    knew = (rng.standard_normal(kv * d) * 0.5).astype(np.float32)
    vnew = rng.standard_normal(kv * d).astype(np.float32)
    kc = cache(rng, kv * length * d, bf16)
    vc = cache(rng, kv * length * d, bf16)
    table = rope_table(theta, d, rotated, length).astype(np.float32)
    n_part = heads * splits * (d + 2)

    # The device: the attention (storing the new rows first, if asked), then the combine.
    b = {name: device.upload(a) for name, a in (("q", q), ("knew", knew), ("vnew", vnew), ("kc", kc), ("vc", vc),
                                                 ("rope", table), ("position", np.array([pos], np.uint32)),
                                                 ("slot", np.array([0], np.uint32)))}
    partials = device.upload(np.zeros(n_part, np.float32))
    out = device.upload(np.zeros(heads * d, np.float32))
    params = K.StepAttendParams(heads, kv, d, length, 1, splits, split, rope, rotated, length, scale, window, bf16,
                                store, rope if store else 0)
    kernels.launch("fk_step_attend", kv * splits, 512, {**{k: v.ptr for k, v in b.items()}, "partials": partials.ptr},
                   params)
    kernels.launch("fk_step_combine", heads, 64, {"partials": partials.ptr, "out": out.ptr},
                   K.StepCombineParams(heads, d, splits))
    device.sync()
    g_kc, g_vc = b["kc"].read(np.uint16, kc.size), b["vc"].read(np.uint16, vc.size)
    g_part, g_out = partials.read(np.float32, n_part), out.read(np.float32, heads * d)

    # The oracle, the same inputs.
    L = fkref.lib()
    o_kc, o_vc = kc.copy(), vc.copy()
    o_part, o_out = np.zeros(n_part, np.float32), np.zeros(heads * d, np.float32)
    if store:
        assert L.fkref_step_store(knew.ctypes.data, vnew.ctypes.data, o_kc.ctypes.data, o_vc.ctypes.data, 2,
                                  rope, 0, kv, d, length, 1, rotated, theta, pos, 0, bf16) == 0
    assert L.fkref_step_attend(q.ctypes.data, o_kc.ctypes.data, o_vc.ctypes.data, o_part.ctypes.data, heads, kv, d,
                               length, 1, splits, split, rope, rotated, theta, scale, window, pos, 0, bf16) == 0
    assert L.fkref_step_combine(o_part.ctypes.data, o_out.ctypes.data, heads, d, splits) == 0

    assert np.array_equal(g_kc, o_kc) and np.array_equal(g_vc, o_vc)
    assert np.array_equal(bits(g_part), bits(o_part)), int(np.sum(bits(g_part) != bits(o_part)))
    assert np.array_equal(bits(g_out), bits(o_out)), int(np.sum(bits(g_out) != bits(o_out)))
    assert np.all(np.isfinite(g_out))
