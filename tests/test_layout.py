"""The tile layout on the host (furykernel_amd/layout.py): the vectorised
packer against the element formula (the one fk_layout.h states in C), the
round trip, and the gate/up pairing."""

import numpy as np
import pytest

from furykernel_amd.layout import LayoutError, pack, pair, tile_offset, unpack


def test_pack_places_every_element_where_the_formula_says():
    rng = np.random.default_rng(5)
    r, k = 512, 96
    x = rng.integers(0, 60000, (r, k)).astype(np.uint16)
    flat = pack(x)
    for row in range(r):
        for col in range(0, k, 7):
            assert flat[tile_offset(row, col, k)] == x[row, col]


def test_pack_is_a_permutation_and_unpack_inverts_it():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((256, 64)).astype(np.float16)
    flat = pack(x)
    assert sorted(flat.view(np.uint16).tolist()) == sorted(x.view(np.uint16).ravel().tolist())
    assert np.array_equal(unpack(flat, 256, 64), x)


def test_a_chunk_is_16_rows_of_one_step_and_units_are_swizzled():
    x = np.arange(256 * 32, dtype=np.uint32).reshape(256, 32)
    flat = pack(x).reshape(16, 64, 8)            # one slab, one step: 16 chunks of 64 units
    assert np.array_equal(flat[1, 0], x[16, 0:8])  # chunk 1 starts at row 16
    # rows 0-3 of a chunk are unswizzled; row 4 has swizzle 1: its place 0
    # holds logical unit 1, row 13 (swizzle 3) place 1 holds unit 2
    assert np.array_equal(flat[0, 8], x[2, 0:8])
    assert np.array_equal(flat[0, 16], x[4, 8:16])
    assert np.array_equal(flat[0, 4 * 13 + 1], x[13, 16:24])


def test_pair_alternates_128_row_blocks():
    g = np.full((256, 32), 1.0, np.float16)
    u = np.full((256, 32), 2.0, np.float16)
    p = pair(g, u)
    assert p.shape == (512, 32)
    assert np.all(p[:128] == 1) and np.all(p[128:256] == 2) and np.all(p[256:384] == 1) and np.all(p[384:] == 2)


def test_shapes_the_layout_does_not_take():
    with pytest.raises(LayoutError):
        pack(np.zeros((100, 32), np.float16))
    with pytest.raises(LayoutError):
        pack(np.zeros((256, 48), np.float16))
    with pytest.raises(LayoutError):
        pair(np.zeros((100, 32), np.float16), np.zeros((100, 32), np.float16))
