"""The C ABI library loads and exports every entry point include/fkrocm.h
declares, the code object holds every kernel of the launch table, and the
kernarg layout is the C layout (src/FuryKernel/Abi.hs:113-133).  No GPU."""

import ctypes
import re
import struct
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_entry_points() -> list[str]:
    """Every function declared in include/*.h."""
    text = "".join(p.read_text() for p in sorted((ROOT / "include").glob("*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from furykernel_amd import runtime

    lib = runtime.library()
    names = declared_entry_points()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []
    # ...and the binding types every one of them.
    typed = {name for name, _, _ in runtime.ENTRY_POINTS}
    assert set(names) == typed


def test_code_object_holds_every_kernel_entry():
    from furykernel_amd import kernels

    blob = kernels.CODE_OBJECT.read_bytes()
    attend = kernels.ATTEND_OBJECT.read_bytes()
    for entry in kernels.ABIS:
        where = attend if entry.startswith(kernels.ATTEND_PREFIX) else blob
        assert entry.encode() + b"\0" in where, entry


def test_the_kernel_library_holds_the_code_objects_the_package_loads():
    """libfkkernels.so (what Kernels loads on a device) carries both code
    objects byte for byte, between its start and end symbols."""
    import ctypes

    from furykernel_amd import kernels

    lib = ctypes.CDLL(str(kernels.KERNEL_LIBRARY))
    for sym, path in (("fk_kernels_co", kernels.CODE_OBJECT), ("fk_attend_co", kernels.ATTEND_OBJECT)):
        start = ctypes.addressof(ctypes.c_char.in_dll(lib, sym))
        end = ctypes.addressof(ctypes.c_char.in_dll(lib, sym + "_end"))
        assert ctypes.string_at(start, end - start) == path.read_bytes(), sym


def test_kernarg_is_pointers_then_c_layout_params():
    from furykernel_amd import kernels

    abi = kernels.ABIS["fk_rmsnorm_f32"]
    raw = abi.kernarg({"x": 0x1000, "gamma": 0x2000, "y": 0x3000},
                      kernels.RmsNormParams(64, 4096, 4096, 1e-6, 1.0, 1))
    assert len(raw) == 3 * 8 + 24
    assert struct.unpack_from("<3Q", raw) == (0x1000, 0x2000, 0x3000)
    rows, width, seg, eps, factor, has_gamma = struct.unpack_from("<3Iffi", raw, 24)
    assert (rows, width, seg, has_gamma) == (64, 4096, 4096, 1)
    assert eps == pytest.approx(1e-6) and factor == 1.0


def test_errors_are_statuses_and_messages_without_a_gpu_or_device():
    """fk_init on a device that doesn't exist fails with a status and a message,
    as the reference's errors are values (src/FuryKernel/Interp.hs:148-186)."""
    from furykernel_amd import runtime

    lib = runtime.library()
    h = ctypes.c_void_p()
    status = lib.fk_init(4096, ctypes.byref(h))
    assert status != 0
    assert lib.fk_last_error(None)
    assert lib.fk_fini(None) == -2
    assert lib.fk_launch(None, 1, 64, 0, None, 0, None) == -2
