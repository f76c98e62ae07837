"""Manifests: what each kernel of the code objects is, as the JSON the
reference's tools read (src/FuryKernel/Manifest.hs:28-92), rendered the way
its JSON writer renders (src/FuryKernel/Json.hs:38-76: keys in the order
given, two-space indentation).

The ABI (buffers, parameter fields, sizes, the ABI hash) comes from the
native library's manifest (``fk_manifest_*``), so the JSON, the launch
table's hash assertions and the kernels' own structs all read one
definition.  What stands for the reference's IR hash — these kernels are
hand-written HIP, not lowered IR — is 64-bit FNV-1a over the source text of
the translation unit that holds the kernel (its ``.hip`` file and every
header of the kernels directory, in name order).  Extents are the byte
formulas the launch table checks, where it checks them.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Union

from . import runtime

KERNELS_DIR = Path(__file__).resolve().parent / "csrc" / "kernels"
FORMAT = "furykernel-manifest"
TARGET = "MI355X"

Json = Union[None, bool, int, str, list, "JObject"]


class JObject(list):
    """A JSON object as an ordered list of (key, value) pairs."""


def _string(s: str) -> str:
    out = []
    for c in s:
        if c == '"':
            out.append('\\"')
        elif c == "\\":
            out.append("\\\\")
        elif c == "\n":
            out.append("\\n")
        elif c == "\r":
            out.append("\\r")
        elif c == "\t":
            out.append("\\t")
        elif ord(c) < 0x20:
            out.append("\\u%04x" % ord(c))
        else:
            out.append(c)
    return '"' + "".join(out) + '"'


def render_json(j: Json) -> str:
    """Json.hs's renderJson: the value, then a newline."""

    def go(depth: int, v) -> str:
        pad = "  " * (depth + 1)
        if v is None:
            return "null"
        if isinstance(v, bool):
            return "true" if v else "false"
        if isinstance(v, int):
            return str(v)
        if isinstance(v, str):
            return _string(v)
        if isinstance(v, JObject):
            if not v:
                return "{}"
            return "{\n" + ",\n".join(pad + _string(k) + ": " + go(depth + 1, x) for k, x in v) + "\n" + \
                "  " * depth + "}"
        if isinstance(v, list):
            if not v:
                return "[]"
            return "[\n" + ",\n".join(pad + go(depth + 1, x) for x in v) + "\n" + "  " * depth + "]"
        raise TypeError(f"no JSON for {type(v).__name__}")

    return go(0, j) + "\n"


def hex64(w: int) -> str:
    return "0x%016x" % w


def kernel_manifest(name: str, abi_hash: int, ir_hash: int, threads: int, groups: str, buffers: list,
                    params: list, params_size: int, tg_memory: int, target: str = TARGET) -> JObject:
    """Manifest.hs's kernelManifest: buffers as (name, access, type, align,
    extent), params as (name, type, offset, dim or None)."""
    def buffer(b):
        return JObject([("name", b[0]), ("access", b[1]), ("type", b[2]), ("align", b[3]), ("extent", b[4])])

    def field(f):
        out = JObject([("name", f[0]), ("type", f[1]), ("offset", f[2])])
        if len(f) > 3 and f[3] is not None:
            lo, hi, mult = f[3]
            out.append(("dim", JObject([("min", lo), ("max", hi), ("multiple_of", mult)])))
        return out

    return JObject([("format", FORMAT), ("version", 1), ("target", target), ("name", name),
                    ("abi_hash", hex64(abi_hash)), ("ir_hash", hex64(ir_hash)), ("threads", threads),
                    ("groups", groups), ("buffers", [buffer(b) for b in buffers]),
                    ("params", [field(f) for f in params]), ("params_size", params_size),
                    ("threadgroup_memory", tg_memory)])


# The bytes the launch table checks each buffer for (fk_launch_check), by
# kernel family; other buffers are only checked to be bound.
_GEMV_EXTENTS = {"w0": "rows_0 * k * elem", "w1": "rows_1 * k * elem", "w2": "rows_2 * k * elem",
                 "y0": "rows_0 * 4", "y1": "rows_1 * 4", "y2": "rows_2 * 4", "src": "k * 4", "src2": "k * 4",
                 "gamma": "k * 4", "table": "table_rows * k * elem", "token": "4", "res": "max rows * 4",
                 "res_table": "table_rows * max rows * elem", "res_token": "4", "epi_out": "max rows * 4",
                 "arg": "arg_slots * 8"}
_EXTENTS = {
    "fk_step_attend": {"q": "heads * head_dim * 4", "knew": "kv_heads * head_dim * 4",
                       "vnew": "kv_heads * head_dim * 4", "kc": "slots * kv_heads * length * head_dim * 2",
                       "vc": "slots * kv_heads * length * head_dim * 2", "position": "4", "slot": "4",
                       "rope": "rope_rows * rotated * 8", "partials": "heads * splits * (head_dim + 2) * 4"},
    "fk_step_combine": {"partials": "heads * splits * (head_dim + 2) * 4", "out": "heads * head_dim * 4"},
    "fk_step_token": {"arg": "slots * 8", "out": "4", "token": "4", "position": "4"},
    "fk_step_store": {"position": "4", "slot": "4"},
}


def _extent(entry: str, buffer: str) -> str:
    if entry.startswith("fk_step_gemv"):
        return _GEMV_EXTENTS.get(buffer, "bound")
    return _EXTENTS.get(entry, {}).get(buffer, "bound")


def source_hash(unit: str) -> int:
    """FNV-1a 64 over a translation unit's source: its .hip file, then every
    header of the kernels directory in name order."""
    lib = runtime.library()
    text = (KERNELS_DIR / unit).read_bytes() + b"".join(p.read_bytes() for p in sorted(KERNELS_DIR.glob("*.h")))
    return lib.fk_fnv1a64(text, len(text))


# The header that defines each tuned family's entries.
_DEFINED_IN = (("fk_step_gemv_", "fk_step_gemv.h"), ("fk_gemv_", "fk_gemv.h"))


def _include_closure(header: str) -> list:
    """The header and the kernels-directory headers it includes, transitively,
    in name order (the parameter structs' header excepted: an entry's
    parameter layout is its ABI hash)."""
    seen, todo = set(), [header]
    while todo:
        h = todo.pop()
        if h in seen:
            continue
        seen.add(h)
        for line in (KERNELS_DIR / h).read_text().splitlines():
            t = line.strip()
            if t.startswith('#include "') and "/" not in t:
                todo.append(t.split('"')[1])
    return sorted(seen)


def entry_source_hash(entry: str) -> int:
    """FNV-1a 64 over what an entry's code is made of: the text of the header
    that defines it and of the kernels headers that header includes, then the
    entry's ABI hash (its bindings and parameter layout).  A change to another
    kernel's header leaves it as it is.  Entries of no tuned family take their
    whole translation unit's source hash."""
    lib = runtime.library()
    for prefix, header in _DEFINED_IN:
        if entry.startswith(prefix):
            text = b"".join((KERNELS_DIR / h).read_bytes() for h in _include_closure(header))
            text += f" {runtime.abi_of(entry).abi_hash:016x}".encode()
            return lib.fk_fnv1a64(text, len(text))
    return source_hash("fk_attend.hip" if entry.startswith("fk_prefill_attend") else "fk_kernels.hip")


def manifest_of(entry: str, tg_memory: int = 0) -> JObject:
    """The manifest of one kernel of the code objects."""
    abi = runtime.abi_of(entry)
    unit = "fk_attend.hip" if entry.startswith("fk_prefill_attend") else "fk_kernels.hip"
    buffers = [(abi.buffers[i].name.decode(), abi.buffers[i].access.decode(), abi.buffers[i].type.decode(),
                abi.buffers[i].align, _extent(entry, abi.buffers[i].name.decode())) for i in range(abi.n_buffers)]
    params = [(abi.params[i].name.decode(), abi.params[i].type.decode(), abi.params[i].offset)
              for i in range(abi.n_params)]
    return kernel_manifest(entry, abi.abi_hash, source_hash(unit), abi.threads, "set by the lowering", buffers,
                           params, abi.params_size, tg_memory)


def write_all(path: Path) -> Path:
    """Every kernel's manifest, one JSON array, next to the code objects."""
    text = render_json([manifest_of(e) for e in runtime.manifest_entries()])
    json.loads(text)  # well-formed
    path.write_text(text)
    return path
