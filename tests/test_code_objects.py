"""The built code objects' kernel resources, from their own metadata.

A kernel that indexes its accumulators with a value the compiler cannot fold
(an epilogue loop it declined to unroll) gets them in private memory: still
correct, many times slower, and invisible to every numeric test.  These
checks read the AMDGPU metadata note (msgpack) of the code objects this
build compiled and bound each matrix-core kernel's private segment and
spills, and check that every kernel the launchers name is there.
"""

import struct

import msgpack
import pytest

from furykernel_amd.build import ATTEND_CO, KERNELS_CO
from furykernel_amd.kernels import ABIS, ATTEND_PREFIX

NT_AMDGPU_METADATA = 32


def device_elf(data: bytes) -> bytes:
    """The gfx950 ELF of a code object: as built, or out of the clang offload
    bundle hipcc writes (magic, entry count, then offset, size, triple of
    each entry)."""
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    if not data.startswith(magic):
        return data
    n, = struct.unpack_from("<Q", data, len(magic))
    at = len(magic) + 8
    for _ in range(n):
        off, size, tlen = struct.unpack_from("<QQQ", data, at)
        triple = data[at + 24:at + 24 + tlen].decode()
        at += 24 + tlen
        if "gfx950" in triple:
            return data[off:off + size]
    raise AssertionError("no gfx950 entry in the bundle")


def kernel_metadata(path) -> dict:
    """Kernel name -> its metadata map, from the ELF's NT_AMDGPU_METADATA note."""
    data = device_elf(path.read_bytes())
    assert data[:4] == b"\x7fELF" and data[4] == 2 and data[5] == 1, "a 64-bit little-endian ELF"
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    out = {}
    for i in range(shnum):
        sh = shoff + i * shentsize
        sh_type, = struct.unpack_from("<I", data, sh + 4)
        if sh_type != 7:  # SHT_NOTE
            continue
        off, size = struct.unpack_from("<QQ", data, sh + 0x18)
        at = off
        while at + 12 <= off + size:
            namesz, descsz, ntype = struct.unpack_from("<III", data, at)
            name = data[at + 12:at + 12 + namesz].rstrip(b"\0")
            desc_at = at + 12 + (namesz + 3) // 4 * 4
            if name == b"AMDGPU" and ntype == NT_AMDGPU_METADATA:
                meta = msgpack.unpackb(data[desc_at:desc_at + descsz], raw=False)
                for k in meta["amdhsa.kernels"]:
                    out[k[".name"]] = k
            at = desc_at + (descsz + 3) // 4 * 4
    return out


@pytest.fixture(scope="module")
def metadata():
    if not KERNELS_CO.exists() or not ATTEND_CO.exists():
        pytest.skip("code objects not built (run __graft_entry__.build())")
    return {**kernel_metadata(KERNELS_CO), **kernel_metadata(ATTEND_CO)}


def test_every_launcher_entry_is_in_a_code_object(metadata):
    missing = [e for e in ABIS if e not in metadata]
    assert not missing, missing
    for e in ABIS:
        assert metadata[e][".kernarg_segment_size"] >= 8 * len(ABIS[e].buffers)


def test_matrix_core_kernels_keep_their_accumulators_in_registers(metadata):
    mm = [e for e in ABIS if e.startswith("fk_gemm_") or e.startswith(ATTEND_PREFIX)]
    assert len(mm) == 18
    for e in mm:
        k = metadata[e]
        assert k[".private_segment_fixed_size"] <= 64, (e, k[".private_segment_fixed_size"])
        assert k[".vgpr_spill_count"] <= 8, (e, k[".vgpr_spill_count"])
        if e.startswith("fk_gemm_"):
            # 8 × 8 blocks of 16 × 16 binary32: the 256 AGPRs
            assert k[".agpr_count"] == 256, (e, k[".agpr_count"])
