"""The launch table of the hand-written gfx950 kernels.

What a ``Lowered``'s ``loweredKernels`` carries for a runtime
(src/FuryKernel/Backend.hs:76-101): each kernel's entry, its buffers in
binding order, its parameter struct in C layout (src/FuryKernel/Abi.hs:
113-133) and its threads.  Kernargs are the buffers' device addresses in that
order, then the struct.

Every launcher checks the shapes it is given against what its kernel assumes
(packs dividing rows, buffers large enough for every access) before it
launches, and raises ``LaunchError`` otherwise: a kernel is never launched on
a shape it would read or write past.
"""

from __future__ import annotations

import ctypes
import re
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import runtime

PACKAGE = Path(__file__).resolve().parent
CODE_OBJECT = PACKAGE / "fk_kernels.hsaco"
ATTEND_OBJECT = PACKAGE / "fk_attend.hsaco"   # the prefill attention, built apart (fk_attend.h)
# Both code objects as read-only data of one shared library (build.py
# build_kernel_library): what the device runs is mapped into the process.
KERNEL_LIBRARY = PACKAGE / "libfkkernels.so"
WAVE = 64


class LaunchError(ValueError):
    """A launch whose shapes or buffers don't fit its kernel."""


class GemvParams(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint32), ("k", ctypes.c_uint32)]


class RmsNormParams(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_uint32),
        ("width", ctypes.c_uint32),
        ("seg", ctypes.c_uint32),
        ("eps", ctypes.c_float),
        ("factor", ctypes.c_float),
        ("has_gamma", ctypes.c_uint32),
    ]


class SoftmaxParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("n", ctypes.c_uint32)]


class FillParams(ctypes.Structure):
    _fields_ = [("count", ctypes.c_uint32), ("value", ctypes.c_uint32)]


class StreamReadParams(ctypes.Structure):
    _fields_ = [("words", ctypes.c_uint64)]


class NoopParams(ctypes.Structure):
    _fields_ = [("unused", ctypes.c_uint32)]


class StepGemvParams(ctypes.Structure):
    _fields_ = [
        ("n_anchors", ctypes.c_uint32),
        ("rows", ctypes.c_uint32 * 3),
        ("first_row", ctypes.c_uint32 * 4),
        ("k", ctypes.c_uint32),
        ("pro_mode", ctypes.c_uint32),
        ("seg", ctypes.c_uint32),
        ("eps", ctypes.c_float),
        ("factor", ctypes.c_float),
        ("gfactor", ctypes.c_float),
        ("has_gamma", ctypes.c_uint32),
        ("epi_mode", ctypes.c_uint32),
        ("store_tile", ctypes.c_uint32),
        ("table_rows", ctypes.c_uint32),
        ("blocks", ctypes.c_uint32),
        ("arg_slots", ctypes.c_uint32),
        ("act", ctypes.c_uint32),
        ("src2_off", ctypes.c_uint32),
        ("cap", ctypes.c_float),
        ("splits", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
    ]


class GemmParams(ctypes.Structure):
    _fields_ = [("m", ctypes.c_uint32), ("k", ctypes.c_uint32), ("n_anchors", ctypes.c_uint32),
                ("first_col", ctypes.c_uint32 * 4), ("ldc", ctypes.c_uint32 * 3), ("act", ctypes.c_uint32)]


class GemmQkvParams(ctypes.Structure):
    """fk_gemm_qkv_params: the GEMM's parameters, then the RoPE and caches'."""
    _fields_ = GemmParams._fields_ + [("kv_heads", ctypes.c_uint32), ("rope_rows", ctypes.c_uint32),
                                      ("length", ctypes.c_uint32), ("slots", ctypes.c_uint32),
                                      ("cache_bf16", ctypes.c_uint32), ("staged", ctypes.c_uint32)]


class PrefillGatherParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("width", ctypes.c_uint32), ("table_rows", ctypes.c_uint32),
                ("table_f16", ctypes.c_uint32), ("factor", ctypes.c_float)]


class PrefillNormParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("width", ctypes.c_uint32), ("eps", ctypes.c_float),
                ("factor", ctypes.c_float), ("has_gamma", ctypes.c_uint32)]


class PrefillRopeParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("rotated", ctypes.c_uint32), ("rope_rows", ctypes.c_uint32),
                ("length", ctypes.c_uint32), ("slots", ctypes.c_uint32), ("cache_bf16", ctypes.c_uint32),
                ("staged", ctypes.c_uint32)]


class PrefillAttendParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("length", ctypes.c_uint32), ("slots", ctypes.c_uint32), ("window", ctypes.c_uint32),
                ("cache_bf16", ctypes.c_uint32), ("scale", ctypes.c_float), ("staged", ctypes.c_uint32),
                ("run_rows", ctypes.c_uint32)]


class GemmQkvPagedParams(ctypes.Structure):
    """fk_gemm_qkv_paged_params: the QKV GEMM's, then the pools' paging."""
    _fields_ = GemmQkvParams._fields_ + [("block_size", ctypes.c_uint32), ("table_len", ctypes.c_uint32),
                                         ("blocks", ctypes.c_uint32)]


class PrefillRopePagedParams(ctypes.Structure):
    """fk_prefill_rope_paged_params: the RoPE store's, then the pools' paging."""
    _fields_ = PrefillRopeParams._fields_ + [("block_size", ctypes.c_uint32), ("table_len", ctypes.c_uint32),
                                             ("blocks", ctypes.c_uint32)]


class PrefillAttendPagedParams(ctypes.Structure):
    """fk_prefill_attend_paged_params: the attention's, then the pools' paging."""
    _fields_ = PrefillAttendParams._fields_ + [("block_size", ctypes.c_uint32), ("table_len", ctypes.c_uint32),
                                               ("blocks", ctypes.c_uint32)]


class PrefillLandParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("length", ctypes.c_uint32), ("slots", ctypes.c_uint32)]


class PrefillSoftcapParams(ctypes.Structure):
    _fields_ = [("count", ctypes.c_uint32), ("cap", ctypes.c_float)]


class ActMulParams(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint32), ("act", ctypes.c_uint32), ("b_off", ctypes.c_uint32), ("half", ctypes.c_uint32)]


class ElementwiseParams(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint32), ("op", ctypes.c_uint32), ("width", ctypes.c_uint32),
                ("width_b", ctypes.c_uint32), ("factor", ctypes.c_float)]


class GatherParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("width", ctypes.c_uint32), ("count", ctypes.c_uint32),
                ("table_rows", ctypes.c_uint32), ("factor", ctypes.c_float)]


# fk_step_elementwise's operations.
ELT_ADD, ELT_SCALE, ELT_STANDARDIZE, ELT_CONCAT = range(4)


class PrefillArgmaxParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("width", ctypes.c_uint32)]


class PrefillArgmaxKeysParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("parts", ctypes.c_uint32)]


class StepTokenParams(ctypes.Structure):
    _fields_ = [("slots", ctypes.c_uint32), ("context", ctypes.c_uint32), ("step", ctypes.c_uint32),
                ("advance", ctypes.c_uint32)]


class StepStoreParams(ctypes.Structure):
    _fields_ = [
        ("n_stores", ctypes.c_uint32),
        ("rope", ctypes.c_uint32 * 2),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("length", ctypes.c_uint32),
        ("slots", ctypes.c_uint32),
        ("rotated", ctypes.c_uint32),
        ("rope_rows", ctypes.c_uint32),
        ("cache_bf16", ctypes.c_uint32),
    ]


class StepAttendParams(ctypes.Structure):
    _fields_ = [
        ("heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("length", ctypes.c_uint32),
        ("slots", ctypes.c_uint32),
        ("splits", ctypes.c_uint32),
        ("split", ctypes.c_uint32),
        ("rope", ctypes.c_uint32),
        ("rotated", ctypes.c_uint32),
        ("rope_rows", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("window", ctypes.c_uint32),
        ("cache_bf16", ctypes.c_uint32),
        ("store", ctypes.c_uint32),
        ("krope", ctypes.c_uint32),
        ("has_reach", ctypes.c_uint32),
    ]


class Paging(ctypes.Structure):
    """``fk_paging``: a paged pool's blocks of block_size positions, a row's
    table of table_len blocks, the pool's `blocks`."""
    _fields_ = [("block_size", ctypes.c_uint32), ("table_len", ctypes.c_uint32), ("blocks", ctypes.c_uint32)]


class StepAttendPagedParams(ctypes.Structure):
    _fields_ = [("a", StepAttendParams), ("g", Paging)]


class StepStorePagedParams(ctypes.Structure):
    _fields_ = [("s", StepStoreParams), ("g", Paging)]


class AttendArgs(ctypes.Structure):
    """``fk_attend_args`` (include/fkrocm_ops.h): device addresses, then the
    attention's parameters."""
    _fields_ = [("q", ctypes.c_uint64), ("knew", ctypes.c_uint64), ("vnew", ctypes.c_uint64),
                ("kc", ctypes.c_uint64), ("vc", ctypes.c_uint64), ("position", ctypes.c_uint64),
                ("slot", ctypes.c_uint64), ("rope", ctypes.c_uint64), ("out", ctypes.c_uint64),
                ("p", StepAttendParams)]


class RouteParams(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint32), ("k", ctypes.c_uint32), ("has_scale", ctypes.c_uint32)]


class GemvRoutedParams(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint32), ("k", ctypes.c_uint32), ("ranks", ctypes.c_uint32),
                ("shared", ctypes.c_uint32), ("entries", ctypes.c_uint32), ("groups_per_rank", ctypes.c_uint32)]


class CombineRanksParams(ctypes.Structure):
    _fields_ = [("seg", ctypes.c_uint32), ("ranks", ctypes.c_uint32), ("residual", ctypes.c_uint32)]


class StepCombineParams(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32), ("splits", ctypes.c_uint32)]


class CountParams(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint32)]


class AdvanceParams(ctypes.Structure):
    _fields_ = [("context", ctypes.c_uint32), ("step", ctypes.c_uint32)]


class InitNormalParams(ctypes.Structure):
    _fields_ = [("count", ctypes.c_uint64), ("seed", ctypes.c_uint64), ("std", ctypes.c_float),
                ("dtype", ctypes.c_uint32)]


@dataclass(frozen=True)
class KernelAbi:
    """A kernel's binary interface: buffers in binding order, then the params struct."""

    entry: str
    buffers: tuple[str, ...]
    params: type
    threads: int = 0  # the threads a launch must have, when the kernel is compiled for one count

    def kernarg(self, bound: dict[str, int], params: ctypes.Structure) -> bytes:
        missing = [b for b in self.buffers if b not in bound]
        if missing:
            raise LaunchError(f"{self.entry}: buffers {missing} not bound")
        ptrs = struct.pack(f"<{len(self.buffers)}Q", *[int(bound[b]) for b in self.buffers])
        return ptrs + bytes(params)


def _gemv_abis() -> dict[str, KernelAbi]:
    out = {}
    for wt, xt in (("f32", "f32"), ("f16", "f32")):
        for r in (1, 2, 4):
            e = f"fk_gemv_{wt}_{xt}_r{r}"
            out[e] = KernelAbi(e, ("w", "x", "y"), GemvParams)
    for r in (1, 2, 4):
        e = f"fk_gemv_i8_f16_r{r}"
        out[e] = KernelAbi(e, ("w", "scale", "x", "y"), GemvParams)
    for wt in ("f32", "f16", "bf16"):
        e = f"fk_gemv_p4_{wt}"
        out[e] = KernelAbi(e, ("w", "x", "y"), GemvParams)
    return out


# The GEMV step kernels (fk_step_gemv.h): <shape>_p<prologue>_e<epilogue>, a
# shape being the weight type, the largest input width it takes and its rows a
# block; the SiLU·mul epilogue (3) on every shape but the widest inputs' (at
# one row a block, a wavefront's row meets its neighbour's in LDS).
STEP_GEMV_SHAPES = {"fk_step_gemv_f16_k2048_r1": True, "fk_step_gemv_f16_k2048_r2": True,
                    "fk_step_gemv_f16_k8192_r1": False, "fk_step_gemv_bf16_k2048_r1": True,
                    "fk_step_gemv_bf16_k2048_r2": True, "fk_step_gemv_bf16_k8192_r1": False,
                    "fk_step_gemv_f32_k256_r1": True,
                    "fk_step_gemv_f32_k256_r2": True, "fk_step_gemv_f32_k1024_r1": True,
                    "fk_step_gemv_f32_k1024_r2": True}
STEP_GEMV_ENTRIES = tuple(f"{shape}_p{pro}_e{epi}" for shape, pairs in STEP_GEMV_SHAPES.items() for pro in range(6)
                          for epi in ((0, 1, 2, 3, 4, 5) if pairs else (0, 1, 2, 4, 5)))
STEP_GEMV_BUFFERS = ("w0", "w1", "w2", "y0", "y1", "y2", "src", "src2", "gamma", "table", "token", "res", "res_table",
                     "res_token", "epi_out", "arg")

# Keys a block of the prefill attention stages (fk_attend.h): ring lengths are
# multiples of it.
ATTEND_KEYS = 64

# Row widths the one-pass RMSNorm-to-tiles holds in registers (fk_prefill.h).
NORM_PACK_HELD = (512, 1024, 2048, 4096)

ABIS: dict[str, KernelAbi] = {
    **_gemv_abis(),
    "fk_rmsnorm_f32": KernelAbi("fk_rmsnorm_f32", ("x", "gamma", "y"), RmsNormParams),
    "fk_softmax_f32": KernelAbi("fk_softmax_f32", ("x", "y"), SoftmaxParams),
    "fk_fill_u32": KernelAbi("fk_fill_u32", ("dst",), FillParams),
    **{e: KernelAbi(e, STEP_GEMV_BUFFERS, StepGemvParams, 512) for e in STEP_GEMV_ENTRIES},
    "fk_step_token": KernelAbi("fk_step_token", ("arg", "out", "token", "position"), StepTokenParams, 64),
    **{f"fk_gemm_f16_{mode}": KernelAbi(f"fk_gemm_f16_{mode}", ("a", "b0", "b1", "b2", "c0", "c1", "c2", "r0"),
                                        GemmParams, 256) for mode in ("store", "add", "silu_mul")},
    "fk_gemm_f16_store_keys": KernelAbi("fk_gemm_f16_store_keys", ("a", "b0", "b1", "b2", "c0", "c1", "c2", "r0",
                                                                   "keys"), GemmParams, 256),
    "fk_gemm_f16_qkv_rope": KernelAbi("fk_gemm_f16_qkv_rope", ("a", "b0", "b1", "b2", "c0", "c1", "c2", "r0",
                                                               "position", "slot", "rope"), GemmQkvParams, 256),
    "fk_gemm_f16_qkv_rope_paged": KernelAbi("fk_gemm_f16_qkv_rope_paged", ("a", "b0", "b1", "b2", "c0", "c1", "c2",
                                                                           "r0", "position", "table", "rope"),
                                            GemmQkvPagedParams, 256),
    "fk_prefill_gather": KernelAbi("fk_prefill_gather", ("table", "tokens", "x"), PrefillGatherParams, 256),
    "fk_prefill_norm_pack": KernelAbi("fk_prefill_norm_pack", ("x", "gamma", "y"), PrefillNormParams, 256),
    **{f"fk_prefill_norm_pack_w{w}": KernelAbi(f"fk_prefill_norm_pack_w{w}", ("x", "gamma", "y"), PrefillNormParams,
                                               256) for w in NORM_PACK_HELD},
    "fk_prefill_rope_store_paged": KernelAbi("fk_prefill_rope_store_paged", ("q", "k", "v", "position", "table",
                                                                             "rope", "qr", "kc", "vc"),
                                             PrefillRopePagedParams),
    "fk_prefill_rope_store": KernelAbi("fk_prefill_rope_store", ("q", "k", "v", "position", "slot", "rope", "qr",
                                                                 "kc", "vc"), PrefillRopeParams),
    **{f"{form}{g}": KernelAbi(f"{form}{g}", ("qr", "kc", "vc", "position", "slot", "out", "ks", "vs"),
                               PrefillAttendParams, 64 * g)
       for form in ("fk_prefill_attend_g", "fk_prefill_attend_f16_g") for g in (1, 2, 4)},
    **{f"{form}{g}": KernelAbi(f"{form}{g}", ("qr", "kc", "vc", "position", "table", "out"),
                               PrefillAttendPagedParams, 64 * g)
       for form in ("fk_prefill_attend_paged_g", "fk_prefill_attend_paged_f16_g") for g in (1, 2, 4)},
    "fk_prefill_land": KernelAbi("fk_prefill_land", ("ks", "vs", "position", "slot", "kc", "vc"),
                                 PrefillLandParams, 256),
    "fk_prefill_argmax": KernelAbi("fk_prefill_argmax", ("x", "out"), PrefillArgmaxParams, 256),
    "fk_prefill_argmax_keys": KernelAbi("fk_prefill_argmax_keys", ("keys", "out"), PrefillArgmaxKeysParams, 256),
    "fk_prefill_softcap": KernelAbi("fk_prefill_softcap", ("x", "y"), PrefillSoftcapParams, 256),
    "fk_step_store": KernelAbi("fk_step_store", ("x0", "x1", "c0", "c1", "position", "slot", "rope"),
                               StepStoreParams),
    "fk_step_store_paged": KernelAbi("fk_step_store_paged", ("x0", "x1", "p0", "p1", "position", "table", "rope"),
                                     StepStorePagedParams),
    "fk_step_attend": KernelAbi("fk_step_attend", ("q", "knew", "vnew", "kc", "vc", "position", "slot", "rope",
                                                   "partials", "reach"), StepAttendParams),
    "fk_step_attend_wide": KernelAbi("fk_step_attend_wide", ("q", "knew", "vnew", "kc", "vc", "position", "slot",
                                                             "rope", "partials", "reach"), StepAttendParams),
    "fk_step_attend_paged": KernelAbi("fk_step_attend_paged", ("q", "knew", "vnew", "kpool", "vpool", "position",
                                                               "table", "rope", "partials", "reach"),
                                      StepAttendPagedParams),
    "fk_step_combine": KernelAbi("fk_step_combine", ("partials", "out"), StepCombineParams, 64),
    "fk_step_argmax": KernelAbi("fk_step_argmax", ("x", "out"), CountParams),
    "fk_step_act_mul": KernelAbi("fk_step_act_mul", ("a", "b", "y"), ActMulParams),
    "fk_step_route": KernelAbi("fk_step_route", ("x", "scale", "ids", "ws"), RouteParams, 64),
    "fk_step_combine_ranks": KernelAbi("fk_step_combine_ranks", ("w", "x", "res", "y"), CombineRanksParams),
    **{e: KernelAbi(e, ("table", "ids", "x", "y"), GemvRoutedParams)
       for e in ("fk_gemv_routed_f16_r1", "fk_gemv_routed_f16_r2", "fk_gemv_routed_f32_r1",
                 "fk_gemv_routed_bf16_r1", "fk_gemv_routed_bf16_r2")},
    "fk_step_elementwise": KernelAbi("fk_step_elementwise", ("a", "b", "c", "y"), ElementwiseParams),
    **{f"fk_step_gather_{t}": KernelAbi(f"fk_step_gather_{t}", ("table", "tokens", "y"), GatherParams)
       for t in ("f32", "f16", "bf16")},
    "fk_step_advance": KernelAbi("fk_step_advance", ("next_token", "token", "position"), AdvanceParams),
    "fk_init_normal": KernelAbi("fk_init_normal", ("dst",), InitNormalParams),
    "fk_noop": KernelAbi("fk_noop", (), NoopParams),
    "fk_stream_read": KernelAbi("fk_stream_read", ("src", "out"), StreamReadParams),
}

# Elements a lane loads at once, by weight type: one 16-byte load of W.
GEMV_PACK = {"f32": 4, "f16": 8, "i8": 16}
ELEM_BYTES = {"f32": 4, "f16": 2, "i8": 1}


def _need(buf: runtime.Buffer, nbytes: int, what: str, entry: str) -> None:
    if buf.size < nbytes:
        raise LaunchError(f"{entry}: {what} holds {buf.size} bytes, the launch reads or writes {nbytes}")
    if buf.ptr % 16:
        raise LaunchError(f"{entry}: {what} is not 16-byte aligned")


ATTEND_PREFIX = "fk_prefill_attend"


class Kernels:
    """The code object loaded on a device, and a launcher per kernel family."""

    def __init__(self, device: runtime.Device, library: Path = KERNEL_LIBRARY):
        if not Path(library).exists():
            raise runtime.NativeMissing(f"{library} is not built; run __graft_entry__.build()")
        self.device = device
        self.library = ctypes.CDLL(str(library))
        images = []
        for sym in ("fk_kernels_co", "fk_attend_co"):
            start = ctypes.addressof(ctypes.c_char.in_dll(self.library, sym))
            end = ctypes.addressof(ctypes.c_char.in_dll(self.library, sym + "_end"))
            if end <= start:
                raise runtime.NativeMissing(f"{library}: {sym} is empty")
            images.append((start, end - start))
        self.module = device.load_module_image(*images[0])
        self.attend_module = device.load_module_image(*images[1])

    def fn(self, entry: str) -> runtime.Function:
        module = self.attend_module if entry.startswith(ATTEND_PREFIX) else self.module
        return module.function(entry)

    def launch(self, entry: str, groups: int, threads: int, bound: dict[str, int], params: ctypes.Structure,
               stream: runtime.Stream | None = None, lds_bytes: int = 0) -> None:
        abi = ABIS[entry]
        self.fn(entry).launch(groups, threads, abi.kernarg(bound, params), lds_bytes, stream)

    # y = W x: the GEMV family (test/Test/FuryKernel/Gemv.hs:131-191) at split 1.
    def gemv(self, w: runtime.Buffer, x: runtime.Buffer, y: runtime.Buffer, n: int, k: int, wtype: str = "f32",
             rows_per_wave: int = 1, threads: int = 256, scale: runtime.Buffer | None = None,
             stream: runtime.Stream | None = None) -> None:
        xtype = "f16" if wtype == "i8" else "f32"
        entry = f"fk_gemv_{wtype}_{xtype}_r{rows_per_wave}"
        if entry not in ABIS:
            raise LaunchError(f"no GEMV kernel {entry}")
        pack = GEMV_PACK[wtype]
        if n <= 0 or k <= 0 or k % pack:
            raise LaunchError(f"{entry}: k = {k} is not a positive multiple of the pack width {pack}")
        if threads % WAVE or not 0 < threads <= 256:
            raise LaunchError(f"{entry}: {threads} threads is not 1 to 4 wavefronts")
        _need(w, n * k * ELEM_BYTES[wtype], "W", entry)
        _need(x, k * ELEM_BYTES[xtype], "x", entry)
        _need(y, n * 4, "y", entry)
        bound = {"w": w.ptr, "x": x.ptr, "y": y.ptr}
        if wtype == "i8":
            if scale is None:
                raise LaunchError(f"{entry}: the int8 layer needs its per-row scales")
            _need(scale, n * 4, "scale", entry)
            bound["scale"] = scale.ptr
        rows_per_group = threads // WAVE * rows_per_wave
        groups = (n + rows_per_group - 1) // rows_per_group
        self.launch(entry, groups, threads, bound, GemvParams(n, k), stream)

    # C = A Bᵀ on the matrix cores (fk_gemm.h): the prefill GEMM.  256 × 256
    # tiles, K steps of 32 taken in pairs; LDS: a ring of 4 stages of A's and
    # B's 256 rows × 32 halves.
    GEMM_TILE, GEMM_K, GEMM_LDS = 256, 64, 4 * 2 * 256 * 32 * 2

    def gemm(self, a: runtime.Buffer, bs: list, cs: list, m: int, k: int, rows: list, mode: str = "store",
             r: runtime.Buffer | None = None, stream: runtime.Stream | None = None, act: int = 0,
             keys: runtime.Buffer | None = None) -> None:
        """A [m, k] f16 in the tile layout (furykernel_amd.layout) times the
        weights bs[j] ([rows[j], k] f16, tiled: the anchors) into cs[j]
        ([m, rows[j]] f32 rows; "add": plus r, [m, rows[0]] f32, which may be
        cs[0]).  "silu_mul": one weight, the pair of gate and up ([2 rows[0],
        k], layout.pair), into cs[0] [m, rows[0]] f16 tiled as silu(gate) up.
        "store_keys": one anchor stored as "store" does, and `keys` [m,
        rows[0] / 128] u64 the greedy token's keys (prefill_argmax_keys)."""
        entry = f"fk_gemm_f16_{mode}"
        if entry not in ABIS:
            raise LaunchError(f"no GEMM {entry}")
        if (mode == "store_keys") != (keys is not None) or (keys is not None and len(bs) != 1):
            raise LaunchError(f"{entry}: keys go with the store_keys mode and one anchor")
        t = self.GEMM_TILE
        if m <= 0 or m % t or k <= 0 or k % self.GEMM_K:
            raise LaunchError(f"{entry}: m = {m} must be a multiple of {t}, k = {k} of {self.GEMM_K}")
        silu = mode == "silu_mul"
        if not 1 <= len(bs) <= (1 if silu else 3) or len(bs) != len(rows) or len(cs) != len(bs):
            raise LaunchError(f"{entry}: {len(bs)} weights, {len(cs)} outputs, {len(rows)} row counts")
        unit = t // 2 if silu else t
        if any(n <= 0 or n % unit for n in rows):
            raise LaunchError(f"{entry}: anchors of {rows} rows, not multiples of {unit}")
        if mode == "add" and (len(bs) != 1 or r is None):
            raise LaunchError(f"{entry}: the residual epilogue takes one anchor and its residual")
        if mode != "add" and r is not None:
            raise LaunchError(f"{entry}: a residual without the residual epilogue")
        _need(a, m * k * 2, "A", entry)
        if silu:
            _need(bs[0], 2 * rows[0] * k * 2, "the gate/up pair", entry)
            _need(cs[0], m * rows[0] * 2, "C", entry)
            groups = (m // t) * (rows[0] // unit)
        else:
            for j, (b, n) in enumerate(zip(bs, rows)):
                _need(b, n * k * 2, f"B{j}", entry)
            for j, (c, n) in enumerate(zip(cs, rows)):
                _need(c, m * n * 4, f"C{j}", entry)
            groups = (m // t) * (sum(rows) // t)
        if r is not None:
            _need(r, m * rows[0] * 4, "R", entry)
        if keys is not None:
            _need(keys, m * (rows[0] // 128) * 8, "keys", entry)
        first = [0]
        for n in rows:
            first.append(first[-1] + n)
        first += [first[-1]] * (4 - len(first))
        ldc = (list(rows) + [0, 0, 0])[:3]
        bufs = {"a": a.ptr, "r0": r.ptr if r is not None else 0}
        if keys is not None:
            bufs["keys"] = keys.ptr
        for j in range(3):
            bufs[f"b{j}"] = bs[j].ptr if j < len(bs) else 0
            bufs[f"c{j}"] = cs[j].ptr if j < len(cs) else 0
        if act not in (ACT_SILU, ACT_GELU_TANH):
            raise LaunchError(f"{entry}: activation {act}")
        params = GemmParams(m, k, len(bs), (ctypes.c_uint32 * 4)(*first), (ctypes.c_uint32 * 3)(*ldc), act)
        self.launch(entry, groups, 256, bufs, params, stream, lds_bytes=self.GEMM_LDS)

    # The kernels around the prefill GEMM (fk_prefill.h).

    def prefill_norm_pack(self, x: runtime.Buffer, gamma: runtime.Buffer | None, y: runtime.Buffer, rows: int,
                          width: int, eps: float = 1e-5, factor: float = 1.0,
                          stream: runtime.Stream | None = None) -> None:
        """RMSNorm of f32 rows [rows, width] into f16 tiles (the GEMM's A)."""
        entry = f"fk_prefill_norm_pack_w{width}" if width in NORM_PACK_HELD else "fk_prefill_norm_pack"
        if rows <= 0 or rows % 256 or width <= 0 or width % 32:
            raise LaunchError(f"{entry}: [{rows}, {width}] does not tile (rows of 256, columns of 32)")
        _need(x, rows * width * 4, "x", entry)
        _need(y, rows * width * 2, "y", entry)
        if gamma is not None:
            _need(gamma, width * 4, "gamma", entry)
        self.launch(entry, rows // 4, 256, {"x": x.ptr, "gamma": gamma.ptr if gamma is not None else 0, "y": y.ptr},
                    PrefillNormParams(rows, width, eps, factor, int(gamma is not None)), stream)

    def prefill_argmax(self, x: runtime.Buffer, out: runtime.Buffer, rows: int, width: int,
                       stream: runtime.Stream | None = None) -> None:
        """The greedy token of each f32 row [rows, width] into out (u32)."""
        entry = "fk_prefill_argmax"
        if rows <= 0 or width <= 0:
            raise LaunchError(f"{entry}: [{rows}, {width}]")
        _need(x, rows * width * 4, "x", entry)
        _need(out, rows * 4, "out", entry)
        self.launch(entry, (rows + 3) // 4, 256, {"x": x.ptr, "out": out.ptr}, PrefillArgmaxParams(rows, width), stream)

    def prefill_argmax_keys(self, keys: runtime.Buffer, out: runtime.Buffer, rows: int, parts: int,
                            stream: runtime.Stream | None = None) -> None:
        """The greedy token of each row from its `parts` keys (u64, [rows,
        parts], as gemm's store_keys mode leaves them) into out (u32)."""
        entry = "fk_prefill_argmax_keys"
        if rows <= 0 or parts <= 0:
            raise LaunchError(f"{entry}: {rows} rows of {parts} keys")
        _need(keys, rows * parts * 8, "keys", entry)
        _need(out, rows * 4, "out", entry)
        self.launch(entry, (rows + 3) // 4, 256, {"keys": keys.ptr, "out": out.ptr},
                    PrefillArgmaxKeysParams(rows, parts), stream)

    def prefill_attend(self, qr: runtime.Buffer, kc: runtime.Buffer, vc: runtime.Buffer, position: runtime.Buffer,
                       slot: runtime.Buffer, out: runtime.Buffer, rows: int, heads: int, kv_heads: int,
                       length: int, slots: int, scale: float, window: int = 0, cache_bf16: bool = False,
                       positions=None, seqs=None, stream: runtime.Stream | None = None) -> None:
        """Causal attention of f16 rows q [rows, heads · 64] (RoPE'd) over the
        caches [slots][kv_heads][length][64] into f16 tiles [rows, heads · 64].
        Every block of 32 rows must be one sequence's consecutive positions:
        given the host copies (positions, seqs), that is checked here.  A bf16
        cache is converted to f16 as it is staged (the matrix operations take
        f16): an element beyond f16's range (|x| > 65504) becomes infinite and
        one below 2^-24 flushes to zero, so bf16 caches are for values inside
        f16's range, as the prefill's own stores of f16-range rows are."""
        g = heads // kv_heads if kv_heads and heads % kv_heads == 0 else 0
        entry = f"fk_prefill_attend_{'g' if cache_bf16 else 'f16_g'}{g}"
        if rows <= 0 or rows % 256 or kv_heads <= 0 or heads % kv_heads or heads // kv_heads not in (1, 2, 4):
            raise LaunchError(f"{entry}: {rows} rows, {heads} heads over {kv_heads}")
        if length <= 0 or length % ATTEND_KEYS:
            raise LaunchError(f"{entry}: a ring of {length}; keys go by blocks of {ATTEND_KEYS} that must not wrap")
        if positions is not None:
            from .prefill import check_rows
            check_rows(positions, seqs)
            if np.max(np.asarray(positions)) >= length:
                raise LaunchError(f"{entry}: positions past the ring's {length}")
        _need(qr, rows * heads * 64 * 2, "q", entry)
        for b, what in ((kc, "K cache"), (vc, "V cache")):
            _need(b, slots * kv_heads * length * 64 * 2, what, entry)
        _need(position, rows * 4, "position", entry)
        _need(slot, rows * 4, "slot", entry)
        _need(out, rows * heads * 64 * 2, "out", entry)
        bound = {"qr": qr.ptr, "kc": kc.ptr, "vc": vc.ptr, "position": position.ptr, "slot": slot.ptr, "out": out.ptr,
                 "ks": 0, "vs": 0}
        self.launch(entry, (rows // 32) * kv_heads, 64 * (heads // kv_heads), bound,
                    PrefillAttendParams(rows, heads, kv_heads, length, slots, window, int(cache_bf16), scale), stream)

    def rmsnorm(self, x: runtime.Buffer, gamma: runtime.Buffer | None, y: runtime.Buffer, rows: int, width: int,
                seg: int | None = None, eps: float = 1e-6, factor: float = 1.0, threads: int = 256,
                stream: runtime.Stream | None = None) -> None:
        entry = "fk_rmsnorm_f32"
        seg = width if seg is None else seg
        if rows <= 0 or seg <= 0 or width % seg or seg % 4:
            raise LaunchError(f"{entry}: segments of {seg} don't divide rows of {width} into packs of 4")
        if threads % WAVE or not 0 < threads <= 1024:
            raise LaunchError(f"{entry}: {threads} threads is not 1 to 16 wavefronts")
        _need(x, rows * width * 4, "x", entry)
        _need(y, rows * width * 4, "y", entry)
        if gamma is not None:
            _need(gamma, seg * 4, "gamma", entry)
        bound = {"x": x.ptr, "gamma": gamma.ptr if gamma is not None else 0, "y": y.ptr}
        params = RmsNormParams(rows, width, seg, eps, factor, 1 if gamma is not None else 0)
        self.launch(entry, rows * (width // seg), threads, bound, params, stream)

    def fill_u32(self, dst: runtime.Buffer, value: int = 0, count: int | None = None,
                 stream: runtime.Stream | None = None) -> None:
        """Sets 32-bit words of a buffer: what a graph clears memory with."""
        count = dst.size // 4 if count is None else count
        if count * 4 > dst.size:
            raise LaunchError(f"fk_fill_u32: {count} words past a buffer of {dst.size} bytes")
        groups = min(max((count + 255) // 256, 1), 4096)
        self.launch("fk_fill_u32", groups, 256, {"dst": dst.ptr}, FillParams(count, value & 0xFFFFFFFF), stream)

    def stream_read(self, src: runtime.Buffer, out: runtime.Buffer, groups: int, nbytes: int | None = None,
                    stream: runtime.Stream | None = None) -> None:
        """Reads `nbytes` of a buffer once (the attainable read bandwidth)."""
        nbytes = src.size if nbytes is None else nbytes
        if nbytes > src.size or nbytes % 16 or src.ptr % 16:
            raise LaunchError("fk_stream_read: a read past the buffer or not in 16-byte words")
        if out.size < groups * 4 * 4:
            raise LaunchError("fk_stream_read: the output holds a word per wavefront")
        self.launch("fk_stream_read", groups, 256, {"src": src.ptr, "out": out.ptr}, StreamReadParams(nbytes // 16),
                    stream)

    def softmax(self, x: runtime.Buffer, y: runtime.Buffer, rows: int, n: int, threads: int = 256,
                stream: runtime.Stream | None = None) -> None:
        entry = "fk_softmax_f32"
        if rows <= 0 or n <= 0 or n % 4:
            raise LaunchError(f"{entry}: rows of {n} are not packs of 4")
        if threads % WAVE or not 0 < threads <= 1024:
            raise LaunchError(f"{entry}: {threads} threads is not 1 to 16 wavefronts")
        _need(x, rows * n * 4, "x", entry)
        _need(y, rows * n * 4, "y", entry)
        self.launch(entry, rows, threads, {"x": x.ptr, "y": y.ptr}, SoftmaxParams(rows, n), stream)


# What each launch reads and writes: the buffers its kernel dereferences for
# its entry and parameters.  A buffer outside this set may be unbound (passed
# as address 0); one inside it never may.

_GEMV_SUFFIX = re.compile(r"^(fk_step_gemv_(f16|bf16|f32)_k(\d+)_r(\d+))_p(\d)_e(\d)$")
PRO_STORED, PRO_RMSNORM, PRO_GATHER, PRO_GATHER_RMSNORM, PRO_SILU_MUL, PRO_COMBINE = range(6)
COMBINE_SPLITS = 8  # the combine prologue's splits at most
EPI_NONE, EPI_ADD_STORED, EPI_ADD_GATHER, EPI_SILU_MUL, EPI_ARGMAX, EPI_SOFTCAP = range(6)
ACT_SILU, ACT_GELU_TANH = 0, 1


def gemv_entry(entry: str) -> tuple[str, str, int, int, int, int]:
    """(shape, weight type, widest k, rows a block, prologue, epilogue) of a
    GEMV step entry: the kernel is specialised on the modes its name carries,
    whatever its parameter struct says."""
    m = _GEMV_SUFFIX.match(entry)
    if m is None:
        raise LaunchError(f"{entry} is not a GEMV step entry")
    return m.group(1), m.group(2), int(m.group(3)), int(m.group(4)), int(m.group(5)), int(m.group(6))


def gemv_reads(pro: int, epi: int, n_anchors: int, store_tile: bool, arg_slots: int = 0) -> set[str]:
    """The buffers a GEMV step kernel of prologue `pro` and epilogue `epi`
    dereferences (fk_step_gemv.h): the gathers read the token unconditionally,
    the norms their gains, and so on."""
    need = {f"w{j}" for j in range(n_anchors)}
    if store_tile:
        need |= {f"y{j}" for j in range(n_anchors)}
    if pro in (PRO_GATHER, PRO_GATHER_RMSNORM):
        need |= {"table", "token"}
    else:
        need.add("src")
    if pro == PRO_SILU_MUL:
        need.add("src2")
    if pro in (PRO_RMSNORM, PRO_GATHER_RMSNORM):
        need.add("gamma")
    if epi == EPI_ADD_STORED:
        need |= {"res", "epi_out"}
    elif epi == EPI_ADD_GATHER:
        need |= {"res_table", "res_token", "epi_out"}
    elif epi == EPI_SILU_MUL:
        need.add("epi_out")
    elif epi == EPI_ARGMAX:
        need.add("arg")
    elif epi == EPI_SOFTCAP:
        need.add("epi_out")
        if arg_slots:
            need.add("arg")
    return need


def launch_reads(entry: str, params: dict) -> set[str]:
    """The buffers a launch of `entry` with `params` dereferences."""
    abi = ABIS[entry]
    if entry.startswith("fk_step_gemv"):
        _, _, _, _, pro, epi = gemv_entry(entry)
        return gemv_reads(pro, epi, params["n_anchors"], bool(params.get("store_tile", 0)), params.get("arg_slots", 0))
    if entry in ("fk_step_attend", "fk_step_attend_wide", "fk_step_attend_paged"):
        paged = entry == "fk_step_attend_paged"
        need = {"q", "position", "partials"} | ({"kpool", "vpool", "table"} if paged else {"kc", "vc", "slot"})
        if params.get("store"):
            need |= {"knew", "vnew"}
        if params.get("rope") or params.get("krope"):
            need.add("rope")
        if params.get("has_reach"):
            need.add("reach")
        return need
    if entry == "fk_step_route":
        return {"x", "ids", "ws"} | ({"scale"} if params.get("has_scale") else set())
    if entry == "fk_step_combine_ranks":
        return {"w", "x", "y"} | ({"res"} if params.get("residual") else set())
    if entry == "fk_step_act_mul":
        return {"a", "y"} | (set() if params.get("half") else {"b"})
    if entry == "fk_step_elementwise":
        op = params.get("op", ELT_ADD)
        return {"a", "y"} | ({"b", "c"} if op == ELT_STANDARDIZE else {"b"})
    if entry == "fk_step_store_paged":
        need = {"x0", "p0", "position", "table"}
        if params.get("n_stores", 1) > 1:
            need |= {"x1", "p1"}
        if any(params.get("rope", (0, 0))):
            need.add("rope")
        return need
    if entry == "fk_step_store":
        need = {"x0", "c0", "position", "slot"}
        if params.get("n_stores", 1) > 1:
            need |= {"x1", "c1"}
        if any(params.get("rope", (0, 0))):
            need.add("rope")
        return need
    if entry == "fk_step_token":
        return {"arg", "out"} | ({"token", "position"} if params.get("advance") else set())
    if entry.startswith("fk_gemm_f16_"):
        n = params.get("n_anchors", 1)
        need = {"a"} | {f"b{j}" for j in range(n)} | {f"c{j}" for j in range(n)}
        if entry == "fk_gemm_f16_add":
            need.add("r0")
        if entry == "fk_gemm_f16_qkv_rope":
            need |= {"position", "slot", "rope"}
        if entry == "fk_gemm_f16_qkv_rope_paged":
            need |= {"position", "table", "rope"}
        if entry == "fk_gemm_f16_store_keys":
            need.add("keys")
        return need
    if entry == "fk_rmsnorm_f32" or entry.startswith("fk_prefill_norm_pack"):
        return set(abi.buffers) - ({"gamma"} if not params.get("has_gamma") else set())
    if entry.startswith(("fk_prefill_attend_g", "fk_prefill_attend_f16_g")):
        return set(abi.buffers) - (set() if params.get("staged") else {"ks", "vs"})
    return set(abi.buffers)
