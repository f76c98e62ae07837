"""The tile layout of matrices that feed the matrix cores (the prefill GEMM's
operands), on the host: packing weights once, and reading packed values
back.

A matrix X [R, K] of f16 (R a multiple of 256, K of 32) is held as slabs of
256 rows; a slab, for each step of 32 columns, as 16 chunks of 1 KB (rows
16 c .. 16 c + 15 of the slab); a chunk as 64 units of 16 bytes, unit L
holding row L div 4 of the chunk and the 8 columns of logical unit
(L mod 4) ^ ((row div 4) mod 4) of the step.  It is the image the GEMM
stages in LDS (furykernel_amd/csrc/kernels/fk_layout.h says the same in C).

The SiLU·mul GEMM takes its gate and up weights paired: slab j of the pair is
gate rows 128 j .. 128 j + 127 then up rows 128 j .. 128 j + 127, so one
threadgroup's slab holds both halves of the elements it finishes.
"""

from __future__ import annotations

import numpy as np

SLAB = 256
STEP = 32


class LayoutError(ValueError):
    pass


def _swizzle_index() -> np.ndarray:
    rows = np.arange(16)
    return np.arange(4)[None, :] ^ ((rows // 4) % 4)[:, None]   # [row, place] -> logical unit


def pack(x: np.ndarray) -> np.ndarray:
    """X [R, K] -> its tile layout, as a flat array of X's dtype."""
    x = np.asarray(x)
    if x.ndim != 2 or x.shape[0] % SLAB or x.shape[1] % STEP:
        raise LayoutError(f"a matrix of {x.shape}: rows a multiple of {SLAB}, columns of {STEP}")
    r, k = x.shape
    t = x.reshape(r // SLAB, 16, 16, k // STEP, 4, 8).transpose(0, 3, 1, 2, 4, 5)
    rows = np.arange(16)
    return np.ascontiguousarray(t[:, :, :, rows[:, None], _swizzle_index(), :]).ravel()


def unpack(flat: np.ndarray, r: int, k: int) -> np.ndarray:
    """The tile layout of an [r, k] matrix -> the matrix."""
    flat = np.asarray(flat)
    if flat.size != r * k or r % SLAB or k % STEP:
        raise LayoutError(f"{flat.size} elements as a tiled [{r}, {k}]")
    t = flat.reshape(r // SLAB, k // STEP, 16, 16, 4, 8)
    out = np.empty((r // SLAB, k // STEP, 16, 16, 4, 8), flat.dtype)
    rows = np.arange(16)
    out[:, :, :, rows[:, None], _swizzle_index(), :] = t
    return np.ascontiguousarray(out.transpose(0, 2, 3, 1, 4, 5)).reshape(r, k)


def pair(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """The SiLU·mul GEMM's weights: gate [n, k] and up [n, k] (n a multiple
    of 128) as one [2 n, k] matrix of alternating 128-row blocks."""
    gate, up = np.asarray(gate), np.asarray(up)
    if gate.shape != up.shape or gate.ndim != 2 or gate.shape[0] % (SLAB // 2):
        raise LayoutError(f"gate {gate.shape} and up {up.shape}: one shape, rows a multiple of {SLAB // 2}")
    n, k = gate.shape
    h = SLAB // 2
    return np.concatenate([gate.reshape(n // h, h, k), up.reshape(n // h, h, k)], axis=1).reshape(2 * n, k)


def tile_offset(row: int, col: int, k: int) -> int:
    """Offset in elements of (row, col) in a tiled matrix of k columns."""
    slab, chunk, r = row // SLAB, (row // 16) % 16, row % 16
    step, unit, half = col // STEP, (col // 8) % 4, col % 8
    place = unit ^ ((r // 4) % 4)
    return ((slab * (k // STEP) + step) * 16 + chunk) * 512 + (4 * r + place) * 8 + half
