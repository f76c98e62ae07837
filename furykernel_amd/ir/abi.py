"""A kernel's ABI (src/FuryKernel/Abi.hs:53-159): its buffers and tables in
binding order, its parameter struct's C layout, and the FNV-1a hash of the
ABI's canonical text, which names, types, alignments, access and offsets
change and extents and contracts do not."""

from __future__ import annotations

from dataclasses import dataclass

from ..program.graph import SCALAR_SIZE
from .ir import READ, Kernel, fnv1a64


@dataclass(frozen=True)
class Field:
    name: str
    type: str
    offset: int
    dim: object  # the parameter's DimRange, or None for a scalar


@dataclass(frozen=True)
class Abi:
    buffers: tuple
    tables: tuple
    params: tuple
    params_size: int
    hash: int


def abi_of(k: Kernel) -> Abi:
    """Abi.hs:113-133: each field at the next multiple of its size, the
    struct rounded up to its largest field's size (0 with no fields)."""
    fields, off = [], 0
    for p in k.params:
        size = SCALAR_SIZE[p.type]
        at = (off + size - 1) // size * size
        fields.append(Field(p.name, p.type, at, p.dim))
        off = at + size
    align = max([1] + [SCALAR_SIZE[p.type] for p in k.params])
    size = (off + align - 1) // align * align
    a = Abi(tuple(k.buffers), tuple(k.tables), tuple(fields), size, 0)
    return Abi(a.buffers, a.tables, a.params, a.params_size, fnv1a64(abi_description(a).encode()))


def abi_description(a: Abi) -> str:
    """The text the ABI hash is over (Abi.hs:136-159)."""
    lines = ["abi 1"]
    lines += [f"buffer {b.name} {b.access} {b.type} align {b.align}" for b in a.buffers]
    lines += [f"table {t.name}" + ("" if t.access == READ else " " + t.access) + f" {t.type} align {t.align}"
              for t in a.tables]
    lines += [f"param {f.name} {f.type} at {f.offset}" for f in a.params]
    lines.append(f"params size {a.params_size}")
    return "\n".join(lines) + "\n"
