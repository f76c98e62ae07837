"""Running what the MI355X backend lowers: its source compiled by hipRTC
(``fk_rtc_compile``), the code object loaded, and each kernel launched from
its launch table (src/FuryKernel/Backend.hs:76-101): the dimensions held to
their ranges first, as the reference's generated runtimes hold them
(Emit/Rust.hs:94-104), the grid and the extents computed in u32 arithmetic
over them (Interp.hs:441-467), buffers checked against their declared
extents, a zero grid skipped, the kernarg the buffers' and tables' device
addresses in binding order and then the parameter struct in the ABI's layout
(Abi.hs:113-133)."""

from __future__ import annotations

import ctypes
import struct
from typing import Optional

import numpy as np

from .. import runtime
from ..program.graph import BF16, BOOL, F16, F32, I8, I32, SCALAR_SIZE, U8, U32
from . import ir as I
from .rocm import COMPILE_OPTIONS, Lowered, LoweredKernel


class LaunchError(ValueError):
    """A launch the kernel's contract refuses, refused before it runs."""


def compile_source(source: str, name: str = "unit.hip", options=COMPILE_OPTIONS) -> bytes:
    """A translation unit's code object for gfx950, by hipRTC (no device needed)."""
    lib = runtime.library()
    opts = (ctypes.c_char_p * len(options))(*[o.encode() for o in options])
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    log = ctypes.c_char_p()
    status = lib.fk_rtc_compile(source.encode(), name.encode(), opts, len(options), ctypes.byref(code),
                                ctypes.byref(size), ctypes.byref(log))
    text = log.value.decode(errors="replace") if log.value else ""
    if log.value:
        lib.fk_rtc_free(ctypes.cast(log, ctypes.c_void_p))
    if status != runtime.FK_OK:
        msg = (lib.fk_last_error(None) or b"").decode()
        raise runtime.FkError(status, msg + ("\n" + text if text else ""))
    try:
        return ctypes.string_at(code.value, size.value)
    finally:
        lib.fk_rtc_free(code)


def launch_size(params: dict, e) -> int:
    """A launch size over the dimensions, every step in u32 (Interp.hs:441-467)."""
    if isinstance(e, I.ELit) and e.lit.type == U32:
        return e.lit.bits
    if isinstance(e, I.EParam):
        return int(params[e.name])
    if isinstance(e, I.EBin):
        x, y = launch_size(params, e.a), launch_size(params, e.b)
        if e.op in ("div", "rem") and y == 0:
            raise LaunchError(f"a launch size divides by zero: {I.render_expr(e)}")
        v = {"add": x + y, "sub": x - y, "mul": x * y}.get(e.op)
        if v is None:
            v = x // y if e.op == "div" else x % y
        if not 0 <= v <= 0xFFFFFFFF:
            raise LaunchError(f"the launch size {I.render_expr(e)} is {v}, outside u32")
        return v
    raise LaunchError(f"not a launch size: {I.render_expr(e)}")


def dim_range_text(r: I.DimRange) -> str:
    return f"{r.min}..{r.max}" + (f" multiple of {r.multiple_of}" if r.multiple_of > 1 else "")


_PACK = {F32: "<f", I32: "<i", U32: "<I", I8: "<b", U8: "<B"}


def params_bytes(lk: LoweredKernel, params: dict) -> bytes:
    """The parameter struct in the ABI's C layout: f16 and bf16 given as their
    bits, bool as 0 or 1."""
    out = bytearray(lk.abi.params_size)
    for f in lk.abi.params:
        if f.name not in params:
            raise LaunchError(f"{lk.name}: no value for the parameter {f.name}")
        v = params[f.name]
        if f.type in (F16, BF16):
            b = struct.pack("<H", int(v) & 0xFFFF)
        elif f.type == BOOL:
            b = struct.pack("<B", 1 if v else 0)
        elif f.type == F32:
            b = struct.pack("<I", int(np.float32(v).view(np.uint32)))
        else:
            b = struct.pack(_PACK[f.type], int(v))
        out[f.offset:f.offset + len(b)] = b
    return bytes(out)


class Unit:
    """A lowered translation unit compiled and loaded on a device."""

    def __init__(self, device: runtime.Device, lowered: Lowered, name: str = "unit.hip"):
        self.device = device
        self.lowered = lowered
        self.code = compile_source(lowered.source, name)
        lib = runtime.library()
        buf = ctypes.create_string_buffer(self.code, len(self.code))
        h = ctypes.c_void_p()
        runtime._check(device.ctx, lib.fk_module_load(device.ctx, buf, len(self.code), ctypes.byref(h)))
        self.module = runtime.Module(device, h.value)
        self.kernels = {lk.name: lk for lk in lowered.kernels}

    def check(self, name: str, params: dict, buffers: dict, tables: Optional[dict] = None) -> int:
        """The launch's grid, after the checks the reference's runtimes make:
        every dimension in its range and on its multiple, every buffer (and
        table) at least its declared extent."""
        lk = self.kernels[name]
        for f in lk.abi.params:
            if f.dim is not None:
                v = int(params[f.name])
                r = f.dim
                if v < r.min or v > r.max or (r.multiple_of > 1 and v % r.multiple_of):
                    raise LaunchError(f"{name}: the dimension {f.name} is {v}, outside its range {dim_range_text(r)}.")
        for b in lk.abi.buffers:
            if b.name not in buffers:
                raise LaunchError(f"{name}: no buffer {b.name}")
            need = launch_size(params, b.extent) * SCALAR_SIZE[b.type]
            if buffers[b.name].size < need:
                raise LaunchError(f"{name}: {b.name} holds {buffers[b.name].size} bytes, its extent {need}")
        for t in lk.abi.tables:
            if not tables or t.name not in tables:
                raise LaunchError(f"{name}: no table {t.name}")
        return launch_size(params, lk.groups)

    def launch(self, name: str, params: dict, buffers: dict, tables: Optional[dict] = None,
               stream: Optional[runtime.Stream] = None) -> int:
        """Launches kernel ``name``: ``buffers`` maps each buffer's name to a
        device buffer, ``tables`` each table's name to a device buffer of its
        entries' device addresses (u64).  Returns the grid (0: skipped)."""
        lk = self.kernels[name]
        groups = self.check(name, params, buffers, tables)
        if groups == 0:
            return 0
        addrs = [buffers[b.name].ptr for b in lk.abi.buffers] + [tables[t.name].ptr for t in lk.abi.tables]
        kernarg = struct.pack(f"<{len(addrs)}Q", *addrs) + params_bytes(lk, params)
        self.module.function(lk.entry).launch(groups, lk.threads, kernarg, 0, stream)
        return groups
