"""The host side of the C ABI in ``include/fkrocm.h``, through ctypes.

This is the binding a ``FuryKernel.Rocm`` target makes with ``foreign import
ccall``, one declaration an entry point, in the host language this repository
can run.  It loads ``libfkrocm.so`` from the package and nothing else: if the
library is missing, or no GPU is present, every entry point raises.  There is
no fallback of any kind.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path
from typing import Iterator

import numpy as np

PACKAGE = Path(__file__).resolve().parent
LIBRARY = PACKAGE / "libfkrocm.so"

FK_OK = 0
STATUS_NAMES = {
    -1: "FK_ERR_HIP",
    -2: "FK_ERR_ARG",
    -3: "FK_ERR_RANGE",
    -4: "FK_ERR_NOT_FOUND",
    -5: "FK_ERR_STATE",
    -6: "FK_ERR_OOM",
    -7: "FK_ERR_COMPILE",
}

# Every entry point of include/fkrocm.h: (name, restype, argtypes).
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_int = ctypes.c_int
_PP = ctypes.POINTER(ctypes.c_void_p)


class DeviceInfo(ctypes.Structure):
    """``fk_device_info``: the reflected caps of ``instance Target Rocm``."""

    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", ctypes.c_int32),
        ("simd_width", ctypes.c_int32),
        ("max_threads", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("global_bytes", ctypes.c_int64),
        ("l2_bytes", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_bits", ctypes.c_int32),
    ]


class AbiBuffer(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("access", ctypes.c_char_p), ("type", ctypes.c_char_p),
                ("align", ctypes.c_uint32)]


class AbiParam(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_char_p), ("offset", ctypes.c_uint32)]


class KernelAbi(ctypes.Structure):
    """``fk_kernel_abi``: a kernel's buffers, its parameter fields, its hash."""

    _fields_ = [("entry", ctypes.c_char_p), ("threads", ctypes.c_uint32), ("n_buffers", ctypes.c_uint32),
                ("buffers", ctypes.POINTER(AbiBuffer)), ("n_params", ctypes.c_uint32),
                ("params", ctypes.POINTER(AbiParam)), ("params_size", ctypes.c_uint32),
                ("abi_hash", ctypes.c_uint64)]


class Binding(ctypes.Structure):
    """``fk_binding``: a buffer's device address and the bytes it holds there."""

    _fields_ = [("addr", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]


_ABI_P = ctypes.POINTER(KernelAbi)

ENTRY_POINTS: list[tuple[str, object, list]] = [
    ("fk_init", _int, [_int, _PP]),
    ("fk_fini", _int, [_vp]),
    ("fk_last_error", ctypes.c_char_p, [_vp]),
    ("fk_device_info_get", _int, [_vp, ctypes.POINTER(DeviceInfo)]),
    ("fk_module_load", _int, [_vp, _vp, _sz, _PP]),
    ("fk_module_load_file", _int, [_vp, ctypes.c_char_p, _PP]),
    ("fk_module_unload", _int, [_vp]),
    ("fk_function", _int, [_vp, ctypes.c_char_p, _PP]),
    ("fk_alloc", _int, [_vp, _sz, _sz, _PP]),
    ("fk_free", _int, [_vp]),
    ("fk_buf_ptr", ctypes.c_uint64, [_vp]),
    ("fk_buf_size", _sz, [_vp]),
    ("fk_arena_create", _int, [_vp, _sz, _PP]),
    ("fk_arena_destroy", _int, [_vp]),
    ("fk_arena_alloc", _int, [_vp, _sz, _sz, _PP]),
    ("fk_arena_usage", _int, [_vp, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    ("fk_arena_reset", _int, [_vp]),
    ("fk_host_alloc", _int, [_vp, _sz, _PP]),
    ("fk_host_free", _int, [_vp, _vp]),
    ("fk_copy_h2d_async", _int, [_vp, _vp, _sz, _vp, _sz, _vp]),
    ("fk_copy_d2h_async", _int, [_vp, _vp, _vp, _sz, _sz, _vp]),
    ("fk_copy_d2d_async", _int, [_vp, _vp, _sz, _vp, _sz, _sz, _vp]),
    ("fk_memset_async", _int, [_vp, _vp, _sz, _int, _sz, _vp]),
    ("fk_stream_create", _int, [_vp, _PP]),
    ("fk_stream_destroy", _int, [_vp]),
    ("fk_stream_sync", _int, [_vp, _vp]),
    ("fk_launch", _int, [_vp, _u32, _u32, _u32, _vp, _sz, _vp]),
    ("fk_event_create", _int, [_vp, _PP]),
    ("fk_event_destroy", _int, [_vp]),
    ("fk_event_record", _int, [_vp, _vp]),
    ("fk_event_sync", _int, [_vp]),
    ("fk_stream_wait_event", _int, [_vp, _vp]),
    ("fk_event_elapsed_ms", _int, [_vp, _vp, ctypes.POINTER(ctypes.c_float)]),
    ("fk_graph_begin", _int, [_vp, _vp]),
    ("fk_graph_end", _int, [_vp, _vp, _PP]),
    ("fk_graph_replay", _int, [_vp, _vp]),
    ("fk_graph_destroy", _int, [_vp]),
    ("fk_fnv1a64", ctypes.c_uint64, [_vp, _sz]),
    ("fk_abi_description", _sz, [_ABI_P, ctypes.c_char_p, _sz]),
    ("fk_abi_hash", ctypes.c_uint64, [_ABI_P]),
    ("fk_manifest_count", _int, []),
    ("fk_manifest_at", _ABI_P, [_int]),
    ("fk_manifest_find", _ABI_P, [ctypes.c_char_p]),
    ("fk_launch_check", _int, [ctypes.c_char_p, _u32, _u32, _u32, ctypes.POINTER(Binding), _u32, _vp, _sz,
                               ctypes.c_uint64, ctypes.c_char_p, _sz]),
    ("fk_table_create", _int, [_vp, _PP]),
    ("fk_table_destroy", _int, [_vp]),
    ("fk_table_add", _int, [_vp, _vp, _u32, _u32, _u32, ctypes.POINTER(Binding), _u32, _vp, _sz, ctypes.c_uint64,
                            ctypes.POINTER(_u32)]),
    ("fk_table_count", _int, [_vp, ctypes.POINTER(_u32)]),
    ("fk_table_enqueue", _int, [_vp, _u32, _u32, _vp]),
    ("fk_attend_decode", _int, [_vp, _vp, _vp]),
    ("fk_attend_decode_noalloc", _int, [_vp, _vp, _vp]),
    ("fk_rtc_compile", _int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), _int, _PP,
                              ctypes.POINTER(_sz), ctypes.POINTER(ctypes.c_char_p)]),
    ("fk_rtc_free", None, [_vp]),
]


class NativeMissing(RuntimeError):
    """The native library is not built: run ``__graft_entry__.build()``."""


class FkError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


_LIB: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """The loaded ``libfkrocm.so``, its entry points typed."""
    global _LIB
    if _LIB is None:
        if not LIBRARY.exists():
            raise NativeMissing(f"{LIBRARY} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(LIBRARY))
        for name, restype, argtypes in ENTRY_POINTS:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = lib
    return _LIB


def _check(ctx: int | None, status: int) -> None:
    if status != FK_OK:
        msg = library().fk_last_error(ctx)
        raise FkError(status, msg.decode() if msg else "")


class Buffer:
    """Device memory: a handle, its device address and its size."""

    def __init__(self, device: "Device", handle: int, owned: bool):
        self.device = device
        self.handle = handle
        self.owned = owned
        self.ptr = int(library().fk_buf_ptr(handle))
        self.size = int(library().fk_buf_size(handle))

    def write(self, array: np.ndarray, offset: int = 0, stream: "Stream | None" = None) -> None:
        a = np.ascontiguousarray(array)
        _check(self.device.ctx, library().fk_copy_h2d_async(
            self.device.ctx, self.handle, offset, a.ctypes.data, a.nbytes, _sh(stream)))
        # The copy reads pageable host memory: wait, so the array may go.
        self.device.sync(stream)

    def read(self, dtype, count: int | None = None, offset: int = 0, stream: "Stream | None" = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = (self.size - offset) // dtype.itemsize if count is None else count
        out = np.empty(n, dtype)
        _check(self.device.ctx, library().fk_copy_d2h_async(
            self.device.ctx, out.ctypes.data, self.handle, offset, out.nbytes, _sh(stream)))
        self.device.sync(stream)
        return out

    def copy_from(self, src: "Buffer", nbytes: int | None = None, dst_offset: int = 0, src_offset: int = 0,
                  stream: "Stream | None" = None) -> None:
        n = src.size - src_offset if nbytes is None else nbytes
        _check(self.device.ctx, library().fk_copy_d2d_async(
            self.device.ctx, self.handle, dst_offset, src.handle, src_offset, n, _sh(stream)))

    def fill_bytes(self, value: int = 0, stream: "Stream | None" = None) -> None:
        _check(self.device.ctx, library().fk_memset_async(self.device.ctx, self.handle, 0, value, self.size,
                                                          _sh(stream)))

    def free(self) -> None:
        if self.owned and self.handle:
            _check(self.device.ctx, library().fk_free(self.handle))
        self.handle = 0


class Arena:
    """One device allocation, carved into resident buffers (weights, caches, stored values)."""

    def __init__(self, device: "Device", nbytes: int):
        self.device = device
        h = ctypes.c_void_p()
        _check(device.ctx, library().fk_arena_create(device.ctx, nbytes, ctypes.byref(h)))
        self.handle = h.value

    def alloc(self, nbytes: int, align: int = 256) -> Buffer:
        h = ctypes.c_void_p()
        _check(self.device.ctx, library().fk_arena_alloc(self.handle, max(nbytes, 1), align, ctypes.byref(h)))
        return Buffer(self.device, h.value, owned=False)

    def usage(self) -> tuple[int, int]:
        used, cap = ctypes.c_size_t(), ctypes.c_size_t()
        _check(self.device.ctx, library().fk_arena_usage(self.handle, ctypes.byref(used), ctypes.byref(cap)))
        return used.value, cap.value

    def destroy(self) -> None:
        if self.handle:
            _check(self.device.ctx, library().fk_arena_destroy(self.handle))
            self.handle = None


class Stream:
    def __init__(self, device: "Device", handle: int | None):
        self.device = device
        self.handle = handle

    def wait(self, event: "Event") -> None:
        """Work queued on this stream from now on waits for the event."""
        _check(self.device.ctx, library().fk_stream_wait_event(self.handle, event.handle))


def _sh(stream: Stream | None):
    return None if stream is None else stream.handle


class Event:
    def __init__(self, device: "Device"):
        self.device = device
        h = ctypes.c_void_p()
        _check(device.ctx, library().fk_event_create(device.ctx, ctypes.byref(h)))
        self.handle = h.value

    def record(self, stream: Stream | None = None) -> None:
        _check(self.device.ctx, library().fk_event_record(self.handle, _sh(stream)))

    def synchronize(self) -> None:
        _check(self.device.ctx, library().fk_event_sync(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(self.device.ctx, library().fk_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)))
        return float(ms.value)


class Function:
    """A kernel entry of a loaded module."""

    def __init__(self, device: "Device", handle: int, entry: str):
        self.device = device
        self.handle = handle
        self.entry = entry

    def launch(self, groups: int, threads: int, kernarg: bytes, lds_bytes: int = 0,
               stream: Stream | None = None) -> None:
        _check(self.device.ctx, library().fk_launch(self.handle, groups, threads, lds_bytes, kernarg,
                                                    len(kernarg), _sh(stream)))


class Module:
    def __init__(self, device: "Device", handle: int):
        self.device = device
        self.handle = handle
        self._fns: dict[str, Function] = {}

    def function(self, entry: str) -> Function:
        if entry not in self._fns:
            h = ctypes.c_void_p()
            _check(self.device.ctx, library().fk_function(self.handle, entry.encode(), ctypes.byref(h)))
            self._fns[entry] = Function(self.device, h.value, entry)
        return self._fns[entry]


class Graph:
    def __init__(self, device: "Device", handle: int):
        self.device = device
        self.handle = handle

    def replay(self, stream: Stream | None = None) -> None:
        _check(self.device.ctx, library().fk_graph_replay(self.handle, _sh(stream)))

    def destroy(self) -> None:
        if self.handle:
            _check(self.device.ctx, library().fk_graph_destroy(self.handle))
            self.handle = None


def abi_of(entry: str) -> KernelAbi:
    """The manifest's ABI of a kernel (host only: no GPU)."""
    p = library().fk_manifest_find(entry.encode())
    if not p:
        raise KeyError(f"{entry}: no such kernel in the manifest")
    return p.contents


def manifest_entries() -> list[str]:
    lib = library()
    return [lib.fk_manifest_at(i).contents.entry.decode() for i in range(lib.fk_manifest_count())]


def abi_description(abi: KernelAbi) -> str:
    lib = library()
    n = lib.fk_abi_description(ctypes.byref(abi), None, 0)
    out = ctypes.create_string_buffer(n + 1)
    lib.fk_abi_description(ctypes.byref(abi), out, n + 1)
    return out.value.decode()


def bindings(spans: list[tuple[int, int]]):
    arr = (Binding * max(len(spans), 1))()
    for i, (addr, nbytes) in enumerate(spans):
        arr[i].addr, arr[i].bytes = int(addr), int(nbytes)
    return arr


def launch_check(entry: str, groups: int, threads: int, lds_bytes: int, spans: list[tuple[int, int]],
                 params: ctypes.Structure, abi_hash: int | None = None) -> None:
    """The native launch table's checks of one launch, on the host (raises
    ``FkError`` with the reason)."""
    lib = library()
    if abi_hash is None:
        abi_hash = abi_of(entry).abi_hash
    err = ctypes.create_string_buffer(512)
    st = lib.fk_launch_check(entry.encode(), groups, threads, lds_bytes, bindings(spans), len(spans),
                             ctypes.byref(params), ctypes.sizeof(params), abi_hash, err, 512)
    if st != FK_OK:
        raise FkError(st, err.value.decode())


class Table:
    """A native launch table: launches checked once (``fk_launch_check``),
    kept with their kernargs, queued in order by one call."""

    def __init__(self, device: "Device"):
        self.device = device
        h = ctypes.c_void_p()
        _check(device.ctx, library().fk_table_create(device.ctx, ctypes.byref(h)))
        self.handle = h.value

    def add(self, fn: "Function", groups: int, threads: int, lds_bytes: int, spans: list[tuple[int, int]],
            params: ctypes.Structure, abi_hash: int | None = None) -> int:
        if abi_hash is None:
            abi_hash = abi_of(fn.entry).abi_hash
        idx = ctypes.c_uint32()
        _check(self.device.ctx, library().fk_table_add(self.handle, fn.handle, groups, threads, lds_bytes,
                                                       bindings(spans), len(spans), ctypes.byref(params),
                                                       ctypes.sizeof(params), abi_hash, ctypes.byref(idx)))
        return idx.value

    def __len__(self) -> int:
        n = ctypes.c_uint32()
        _check(self.device.ctx, library().fk_table_count(self.handle, ctypes.byref(n)))
        return n.value

    def enqueue(self, first: int = 0, count: int | None = None, stream: "Stream | None" = None) -> None:
        count = len(self) - first if count is None else count
        _check(self.device.ctx, library().fk_table_enqueue(self.handle, first, count, _sh(stream)))

    def destroy(self) -> None:
        if self.handle:
            _check(self.device.ctx, library().fk_table_destroy(self.handle))
            self.handle = None


def attend_decode(device: "Device", args: ctypes.Structure, stream: "Stream | None" = None,
                  entry: str = "fk_attend_decode") -> None:
    """One decode attention step through the library's operation
    (include/fkrocm_ops.h); `args` is a ``kernels.AttendArgs``."""
    _check(device.ctx, getattr(library(), entry)(device.ctx, ctypes.byref(args), _sh(stream)))


class Device:
    """One GPU: a context of the C ABI, its stream, and what it allocates."""

    def __init__(self, index: int = 0):
        lib = library()
        h = ctypes.c_void_p()
        status = lib.fk_init(index, ctypes.byref(h))
        if status != FK_OK:
            raise FkError(status, (lib.fk_last_error(None) or b"").decode())
        self.ctx = h.value
        self.stream = Stream(self, None)
        self._info: DeviceInfo | None = None

    @property
    def info(self) -> DeviceInfo:
        if self._info is None:
            info = DeviceInfo()
            _check(self.ctx, library().fk_device_info_get(self.ctx, ctypes.byref(info)))
            self._info = info
        return self._info

    def alloc(self, nbytes: int, align: int = 256) -> Buffer:
        h = ctypes.c_void_p()
        _check(self.ctx, library().fk_alloc(self.ctx, max(nbytes, 1), align, ctypes.byref(h)))
        return Buffer(self, h.value, owned=True)

    def upload(self, array: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(array)
        b = self.alloc(a.nbytes)
        b.write(a)
        return b

    def arena(self, nbytes: int) -> Arena:
        return Arena(self, nbytes)

    def new_stream(self) -> Stream:
        h = ctypes.c_void_p()
        _check(self.ctx, library().fk_stream_create(self.ctx, ctypes.byref(h)))
        return Stream(self, h.value)

    def load_module(self, path: str | os.PathLike) -> Module:
        h = ctypes.c_void_p()
        _check(self.ctx, library().fk_module_load_file(self.ctx, str(path).encode(), ctypes.byref(h)))
        return Module(self, h.value)

    def load_module_image(self, address: int, nbytes: int) -> Module:
        """A code object held in host memory at `address` (`nbytes` long)."""
        h = ctypes.c_void_p()
        _check(self.ctx, library().fk_module_load(self.ctx, ctypes.c_void_p(address), nbytes, ctypes.byref(h)))
        return Module(self, h.value)

    def event(self) -> Event:
        return Event(self)

    def sync(self, stream: Stream | None = None) -> None:
        _check(self.ctx, library().fk_stream_sync(self.ctx, _sh(stream)))

    @contextlib.contextmanager
    def capture(self, stream: Stream | None = None) -> Iterator[list]:
        """Captures the launches queued on the stream into a graph: ``with
        dev.capture() as out: ...`` leaves the ``Graph`` in ``out[0]``."""
        out: list = []
        _check(self.ctx, library().fk_graph_begin(self.ctx, _sh(stream)))
        try:
            yield out
        finally:
            h = ctypes.c_void_p()
            _check(self.ctx, library().fk_graph_end(self.ctx, _sh(stream), ctypes.byref(h)))
            out.append(Graph(self, h.value))

    def close(self) -> None:
        if self.ctx:
            _check(None, library().fk_fini(self.ctx))
            self.ctx = None
