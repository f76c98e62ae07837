"""Selections: which variant of a family each shape class runs on a target,
as tuning chose and a repository commits (src/FuryKernel/Selection.hs).

The format, version 1 (the reference's, field for field)::

    {
      "format": "furykernel-selection",
      "version": 1,
      "family": "step_gemv_f16",
      "target": "MI355X",
      "profile": {
        "cores": 256
      },
      "classes": {
        "n16384_k2048_m1": {
          "variant": "r2_g3",
          "ir_hash": "0x5b1e46d0c3a9f2e7"
        }
      }
    }

The profile is the GPU's as tuning measured it (its CUs).  Each class's key
is its shape key, its pick the axis key of its variant and the hash of the
variant's launch when it was picked (``variant.launch_hash``); classes are
written in key order, each once.  A selection is valid for a space and a
profile when the space passes ``check_space``, the selection was made for
that profile, names the space's family and target, picks a variant for every
class of the space and for no other, every pick survives pruning but for
duplicates and is the launch it was picked as, and the classes that differ
only in batch dimensions agree on every axis that decides a reduction's
order.
"""

from __future__ import annotations

import json
import re
from dataclasses import dataclass, field

from .manifest import JObject, hex64, render_json
from .variant import (IllegalOutcome, Indivisible, Kept, Profile, SameAs, Space, TooFewGroups, axis_key,
                      check_space, consider, parse_axis_key, shape_key, variant_name)

FORMAT = "furykernel-selection"
TARGET = "MI355X"


@dataclass(frozen=True)
class Pick:
    axes: str
    ir_hash: int


@dataclass
class Selection:
    family: str
    target: str
    profile: Profile
    classes: dict = field(default_factory=dict)  # shape key -> Pick


def render(sel: Selection) -> str:
    return render_json(JObject([
        ("format", FORMAT), ("version", 1), ("family", sel.family), ("target", sel.target),
        ("profile", JObject([("cores", sel.profile.cores)])),
        ("classes", JObject([(c, JObject([("variant", p.axes), ("ir_hash", hex64(p.ir_hash))]))
                             for c, p in sorted(sel.classes.items())]))]))


class SelectionError(ValueError):
    def __init__(self, problems: list):
        super().__init__("\n".join(problems))
        self.problems = list(problems)


_HASH = re.compile(r"^0x[0-9a-f]{16}$")


class _Obj(list):
    """A JSON object as its (key, value) pairs, in order."""


def parse(text: str) -> Selection:
    """A selection from its JSON: the format only, not what it selects
    (raises ``SelectionError``)."""
    try:
        j = json.loads(text, object_pairs_hook=_Obj)
    except json.JSONDecodeError as e:
        raise SelectionError([str(e)])
    if not isinstance(j, _Obj):
        raise SelectionError(["A selection is a JSON object."])
    fields = dict(j)

    def get(name, ok):
        if name not in fields:
            raise SelectionError([f"The field {name} is missing."])
        v = ok(fields[name])
        if v is None:
            raise SelectionError([f"The field {name} has the wrong type."])
        return v

    def string(v):
        return v if isinstance(v, str) else None

    def integer(v):
        return v if isinstance(v, int) and not isinstance(v, bool) else None

    fmt = get("format", string)
    if fmt != FORMAT:
        raise SelectionError([f"The format is {fmt}, not {FORMAT}."])
    version = get("version", integer)
    if version != 1:
        raise SelectionError([f"Version {version} of the format; this reads version 1."])
    unknown = [k for k, _ in j if k not in ("format", "version", "family", "target", "profile", "classes")]
    if unknown:
        raise SelectionError([f"An unknown field: {k}." for k in unknown])
    family = get("family", string)
    target = get("target", string)

    def profile(v):
        if isinstance(v, _Obj) and len(v) == 1 and v[0][0] == "cores" and integer(v[0][1]) is not None \
                and v[0][1] >= 0:
            return Profile(v[0][1])
        return None

    def pick(v):
        if isinstance(v, _Obj) and [k for k, _ in v] == ["variant", "ir_hash"]:
            a, h = v[0][1], v[1][1]
            if isinstance(a, str) and isinstance(h, str) and _HASH.match(h):
                return Pick(a, int(h, 16))
        return None

    def classes(v):
        if not isinstance(v, _Obj):
            return None
        out = {}
        for c, x in v:
            p = pick(x)
            if p is None:
                return None
            out[c] = p
        return out

    return Selection(family, target, get("profile", profile), get("classes", classes))


def validate(profile: Profile, space: Space, sel: Selection, target: str = TARGET) -> list:
    """The selected variant of every class, in the space's class order (raises
    ``SelectionError`` with everything that is wrong)."""
    problems = list(check_space(space))
    if sel.profile != profile:
        problems.append(f"The selection was made for a GPU of {sel.profile.cores} cores, not {profile.cores}.")
    if sel.family != space.family:
        problems.append(f"The selection is for the family {sel.family}, not {space.family}.")
    if sel.target != target:
        problems.append(f"The selection is for the target {sel.target}, not {target}.")
    keys = [shape_key(s) for s in space.shapes]
    problems += [f"No variant for the class {k}." for k in keys if k not in sel.classes]
    problems += [f"The class {c} is not one of the family's." for c in sel.classes if c not in keys]
    picked = []
    for s in space.shapes:
        p = sel.classes.get(shape_key(s))
        if p is None:
            continue
        try:
            point = parse_axis_key(space.axes, p.axes, f"The class {shape_key(s)}'s axis key")
        except ValueError as e:
            problems.append(str(e))
            continue
        name = variant_name(space, s, point)
        o = consider(profile, space, s, point)
        if isinstance(o, Kept):
            if o.variant.ir_hash != p.ir_hash:
                problems.append(f"{name} was picked as the kernel of IR hash {hex64(p.ir_hash)}, and is now "
                                f"{hex64(o.variant.ir_hash)}.")
            else:
                picked.append(o.variant)
        elif isinstance(o, IllegalOutcome):
            problems.append(f"{name} is illegal: {' '.join(o.findings)}")
        elif isinstance(o, Indivisible):
            problems.append(f"{name} does not divide its class: {' '.join(o.reasons)}")
        elif isinstance(o, TooFewGroups):
            problems.append(f"{name} launches {o.groups} threadgroups, fewer than twice the {profile.cores} cores.")
        elif isinstance(o, SameAs):
            problems.append(f"{name} is the same kernel as {axis_key(o.point)}.")
    order = [a.prefix for a in space.axes if a.order]

    def unbatched(shape):
        return tuple((d, v) for d, v in shape if d not in space.batch)

    for i, a in enumerate(picked):
        for b in picked[i + 1:]:
            pa = tuple((k, v) for k, v in a.point if k in order)
            pb = tuple((k, v) for k, v in b.point if k in order)
            if unbatched(a.shape) == unbatched(b.shape) and pa != pb:
                problems.append(f"The classes {shape_key(a.shape)} and {shape_key(b.shape)} differ only in batch "
                                f"size, and order reductions differently: {axis_key(pa)} against {axis_key(pb)}.")
    if problems:
        raise SelectionError(problems)
    return picked
