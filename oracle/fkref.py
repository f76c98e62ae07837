"""ctypes bindings of the oracle's C restatement (``oracle/fkref.c``).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "libfkref.so"

F32, F16, BF16, I8, U32 = 0, 1, 2, 3, 4
TYPE_OF = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.int8): I8}

_lib: ctypes.CDLL | None = None
_fp = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_i = ctypes.c_int


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY} is not built: run `make -C oracle` or __graft_entry__.build()")
        L = ctypes.CDLL(str(LIBRARY))
        sig = {
            "fkref_widen_bf16": (ctypes.c_float, [ctypes.c_uint16]),
            "fkref_narrow_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "fkref_widen_f16": (ctypes.c_float, [ctypes.c_uint16]),
            "fkref_narrow_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "fkref_narrow_f16_f64": (ctypes.c_uint16, [ctypes.c_double]),
            "fkref_min": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "fkref_max": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "fkref_rsqrt": (ctypes.c_float, [ctypes.c_float]),
            "fkref_exp": (ctypes.c_float, [ctypes.c_float]),
            "fkref_simd_sum": (ctypes.c_float, [_vp, _i]),
            "fkref_simd_max": (ctypes.c_float, [_vp, _i]),
            "fkref_tg_reduce_sum": (ctypes.c_float, [_vp, _i, _i]),
            "fkref_tg_reduce_max": (ctypes.c_float, [_vp, _i, _i]),
            "fkref_combine_splits": (ctypes.c_float, [_vp, _i]),
            "fkref_set_threads": (_i, [_i]),
            "fkref_gemv": (_i, [_vp, _i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i]),
            "fkref_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _i, ctypes.c_float, ctypes.c_float, _i, _i, _i]),
            "fkref_softmax": (_i, [_vp, _vp, _i, _i, _i, _i, _i]),
            "fkref_step_gemv": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, ctypes.c_uint32, _i, _i,
                                     ctypes.c_float, ctypes.c_float, ctypes.c_float, _i, _vp, _vp, ctypes.c_uint32,
                                     _vp, _i, _i, _i, _i]),
            "fkref_tanh": (ctypes.c_float, [ctypes.c_float]),
            "fkref_gelu_tanh": (ctypes.c_float, [ctypes.c_float]),
            "fkref_softcap": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "fkref_act_mul": (_i, [_vp, _vp, _vp, _i, _i]),
            "fkref_rope_elem": (ctypes.c_float, [_vp, _i, _i, _i, ctypes.c_uint32, ctypes.c_float]),
            "fkref_step_store": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float,
                                      ctypes.c_uint32, ctypes.c_uint32, _i]),
            "fkref_step_attend": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float,
                                       ctypes.c_float, _i, ctypes.c_uint32, ctypes.c_uint32, _i]),
            "fkref_step_combine": (_i, [_vp, _vp, _i, _i, _i]),
            "fkref_step_attend_reach": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i,
                                             ctypes.c_float, ctypes.c_float, _i, ctypes.c_uint32, ctypes.c_uint32,
                                             ctypes.c_uint32, _i]),
            "fkref_step_attend_paged": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _i, _i, _i, _i,
                                             ctypes.c_float, ctypes.c_float, _i, ctypes.c_uint32, ctypes.c_uint32,
                                             _i]),
            "fkref_step_store_paged": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _i, _i,
                                            ctypes.c_float, ctypes.c_uint32, _i]),
            "fkref_step_attend_wide": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float,
                                            ctypes.c_float, _i, ctypes.c_uint32, ctypes.c_uint32, _i]),
            "fkref_argmax": (ctypes.c_uint32, [_vp, _i]),
            "fkref_argmax_key": (ctypes.c_uint64, [ctypes.c_float, ctypes.c_uint32]),
            "fkref_argmax_keyed": (ctypes.c_uint64, [_vp, _i]),
            "fkref_silu_mul": (_i, [_vp, _vp, _vp, _i]),
            "fkref_route": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
            "fkref_combine_ranks": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
            "fkref_widen_f16_n": (None, [_vp, _vp, ctypes.c_size_t]),
            "fkref_widen_bf16_n": (None, [_vp, _vp, ctypes.c_size_t]),
            "fkref_narrow_f16_n": (None, [_vp, _vp, ctypes.c_size_t]),
            "fkref_narrow_bf16_n": (None, [_vp, _vp, ctypes.c_size_t]),
            "fkref_narrow_f16_f64_n": (None, [_vp, _vp, ctypes.c_size_t]),
            "fkref_fma_f32_n": (None, [_vp, _vp, _vp, _vp, ctypes.c_size_t]),
            "fkref_unary_f64_n": (None, [_i, _vp, _vp, ctypes.c_size_t]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# Numerics -------------------------------------------------------------------

def widen_bf16(b: int) -> float:
    return lib().fkref_widen_bf16(b)


def narrow_bf16(x: float) -> int:
    return lib().fkref_narrow_bf16(x)


def widen_f16(h: int) -> float:
    return lib().fkref_widen_f16(h)


def narrow_f16(x: float) -> int:
    return lib().fkref_narrow_f16(x)


def narrow_f16_f64(x: float) -> int:
    return lib().fkref_narrow_f16_f64(x)


def simd_sum(lanes, width: int | None = None) -> np.float32:
    a = _f32(lanes)
    return np.float32(lib().fkref_simd_sum(_ptr(a), len(a) if width is None else width))


def simd_max(lanes) -> np.float32:
    a = _f32(lanes)
    return np.float32(lib().fkref_simd_max(_ptr(a), len(a)))


def tg_reduce_sum(per_thread, width: int) -> np.float32:
    a = _f32(per_thread)
    return np.float32(lib().fkref_tg_reduce_sum(_ptr(a), len(a), width))


def tg_reduce_max(per_thread, width: int) -> np.float32:
    a = _f32(per_thread)
    return np.float32(lib().fkref_tg_reduce_max(_ptr(a), len(a), width))


def combine_splits(partials) -> np.float32:
    a = _f32(partials)
    return np.float32(lib().fkref_combine_splits(_ptr(a), len(a)))


# Kernels --------------------------------------------------------------------

def gemv(w: np.ndarray, x: np.ndarray, width: int, pack: int, split: int = 1,
         row_scale: np.ndarray | None = None) -> np.ndarray:
    """y = W x in the reference GEMV's order; W [n, k], x [m, k] (or [k])."""
    w = np.ascontiguousarray(w)
    x2 = np.ascontiguousarray(x)
    m = 1 if x2.ndim == 1 else x2.shape[0]
    n, k = w.shape
    y = np.empty((m, n), np.float32)
    s = None if row_scale is None else _f32(row_scale)
    st = lib().fkref_gemv(_ptr(w), TYPE_OF[w.dtype], _ptr(x2), TYPE_OF[x2.dtype], _ptr(y), _ptr(s), n, k, m, width,
                          pack, split)
    if st:
        raise ValueError(f"fkref_gemv refused the shape (status {st})")
    return y[0] if x2.ndim == 1 else y


def rmsnorm(x: np.ndarray, gamma: np.ndarray | None, eps: float, threads: int, width: int, pack: int = 4,
            seg: int | None = None, factor: float = 1.0) -> np.ndarray:
    x = _f32(x)
    rows, w = (1, x.shape[0]) if x.ndim == 1 else x.shape
    seg = w if seg is None else seg
    g = None if gamma is None else _f32(gamma)
    y = np.empty_like(x)
    st = lib().fkref_rmsnorm(_ptr(x), _ptr(g), _ptr(y), rows, w, seg, eps, factor, threads, width, pack)
    if st:
        raise ValueError(f"fkref_rmsnorm refused the shape (status {st})")
    return y


def softmax(x: np.ndarray, threads: int, width: int, pack: int = 4) -> np.ndarray:
    x = _f32(x)
    rows, n = (1, x.shape[0]) if x.ndim == 1 else x.shape
    y = np.empty_like(x)
    st = lib().fkref_softmax(_ptr(x), _ptr(y), rows, n, threads, width, pack)
    if st:
        raise ValueError(f"fkref_softmax refused the shape (status {st})")
    return y
