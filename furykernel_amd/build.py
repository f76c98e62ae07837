"""Builds the native parts of the target in-tree.

* ``libfkrocm.so`` — the C ABI of ``include/fkrocm.h`` over HIP (host code).
* ``fk_kernels.hsaco`` — the hand-written gfx950 kernels, one code object,
  which ``fk_module_load_file`` loads.

Kernels are compiled Strict, as ``CompileOptions`` asks of a target
(src/FuryKernel/Backend.hs:52-73): ``-ffp-contract=off`` and no fast-math, so
nothing contracts a multiply and an add, nothing reassociates.  Packed FP32
instructions are disabled (``-packed-fp32-ops``).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
ROOT = PACKAGE.parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

RUNTIME_SO = PACKAGE / "libfkrocm.so"
KERNELS_CO = PACKAGE / "fk_kernels.hsaco"
ATTEND_CO = PACKAGE / "fk_attend.hsaco"
KERNELS_SO = PACKAGE / "libfkkernels.so"   # the two code objects, as data of a shared library

KERNEL_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


def build_runtime() -> Path:
    """The C ABI's library: the runtime and manifest (host code) and the
    operations (fk_ops.hip, whose kernels are built with the kernels' flags)."""
    tmp = RUNTIME_SO.with_suffix(".so.tmp")
    objs = []
    for src in (CSRC / "fk_runtime.cpp", CSRC / "fk_manifest.cpp"):
        obj = PACKAGE / f".{src.stem}.o"
        _run([HIPCC, "-c", "-fPIC", "-O2", "-std=c++17", "-Wno-unused-value", "-Wno-unused-result",
              f"-I{ROOT / 'include'}", str(src), "-o", str(obj)])
        objs.append(obj)
    obj = PACKAGE / ".fk_ops.o"
    _run([HIPCC, "-c", "-fPIC", *KERNEL_FLAGS, f"-I{ROOT / 'include'}", str(CSRC / "fk_ops.hip"), "-o", str(obj)])
    objs.append(obj)
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp), "-lhiprtc"])
    for o in objs:
        o.unlink()
    os.replace(tmp, RUNTIME_SO)
    return RUNTIME_SO


def build_kernels() -> Path:
    src = CSRC / "kernels" / "fk_kernels.hip"
    tmp = KERNELS_CO.with_suffix(".hsaco.tmp")
    _run([HIPCC, "--genco", *KERNEL_FLAGS, str(src), "-o", str(tmp)])
    os.replace(tmp, KERNELS_CO)
    return KERNELS_CO


def build_attend() -> Path:
    """The prefill attention's code object: the same flags, and the matrix
    operations in their VGPR form (fk_attend.h says why)."""
    src = CSRC / "kernels" / "fk_attend.hip"
    tmp = ATTEND_CO.with_suffix(".hsaco.tmp")
    _run([HIPCC, "--genco", *KERNEL_FLAGS, "-mllvm", "-amdgpu-mfma-vgpr-form=1", str(src), "-o", str(tmp)])
    os.replace(tmp, ATTEND_CO)
    return ATTEND_CO


def build_kernel_library() -> Path:
    """The hand-written kernels' code objects as read-only data of one
    shared library (symbols fk_kernels_co .. fk_kernels_co_end and
    fk_attend_co .. fk_attend_co_end), which the package loads and hands to
    fk_module_load: the process maps the library that holds the device code
    it runs."""
    import tempfile
    with tempfile.TemporaryDirectory() as tmpdir:
        asm = Path(tmpdir) / "fk_kernels_blob.S"
        lines = ['.section .rodata']
        for sym, co in (("fk_kernels_co", KERNELS_CO), ("fk_attend_co", ATTEND_CO)):
            lines += [f".global {sym}", f".global {sym}_end", ".balign 4096", f"{sym}:",
                      f'.incbin "{co}"', f"{sym}_end:"]
        lines.append('.section .note.GNU-stack,"",@progbits')
        asm.write_text("\n".join(lines) + "\n")
        tmp = KERNELS_SO.with_suffix(".so.tmp")
        _run(["gcc", "-shared", "-fPIC", str(asm), "-o", str(tmp)])
        os.replace(tmp, KERNELS_SO)
    return KERNELS_SO


def build_all() -> list[Path]:
    return [build_runtime(), build_kernels(), build_attend(), build_kernel_library()]


if __name__ == "__main__":
    for p in build_all():
        print(p)
