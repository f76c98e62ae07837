"""Variant spaces for gfx950: one kernel family, many ways to launch it
(src/FuryKernel/Variant.hs).

A family declares its axes (choices that change how its kernels run but not
what they compute: rows a wavefront, threads, threadgroups a CU) and its
shape classes (the problem sizes it is launched at).  For each class,
``enumerate`` visits every point of the axes and prunes, in the reference's
order:

1. legality: the family builds the launch, and the launch table's checks
   (``fk_launch_check``) accept it;
2. divisibility: the family's rule (a class's dimensions by a pack width, by
   the rows of a threadgroup);
3. parallelism: at least twice as many threadgroups as the GPU has CUs;
4. duplicates: points whose launches are another kept point's (the same
   entry, threads, threadgroups, LDS and parameters).

The reference's fifth rule, its hazard check over lowered IR, has no
counterpart: these kernels are hand-written HIP, and the launch check is the
gate.  What remains are the class's variants, named
``family_class_x_axiskey`` (``gemv_f32_n4096_k4096_m1_x_r2_t256``), and
``family_class`` for a family without axes.  A committed selection picks one
per class (``selection.py``).

Some axes decide the order of a reduction: the variants of classes that
differ only in a batch dimension must agree on those.  The families here
have none (each output row's sum runs in the same order whatever the rows a
wavefront, threads or threadgroups), and say so.
"""

from __future__ import annotations

import ctypes
import itertools
import re
from dataclasses import dataclass, field
from typing import Callable, Optional, Union

from . import runtime


@dataclass(frozen=True)
class Axis:
    """One choice of a family's, and the values tuning tries (Variant.hs:86-95)."""

    name: str
    prefix: str
    values: tuple
    order: bool = False  # whether the axis decides the order of a reduction


Point = tuple  # ((prefix, value), ...) in the axes' order
Shape = tuple  # ((dimension, value), ...)


def point_value(prefix: str, point: Point) -> Optional[int]:
    return dict(point).get(prefix)


def points(axes: list) -> list:
    """Every point, the first axis varying slowest."""
    return [tuple(zip([a.prefix for a in axes], vs)) for vs in itertools.product(*[a.values for a in axes])]


def axis_key(point: Point) -> str:
    """``r2_t128``."""
    return "_".join(f"{p}{v}" for p, v in point)


def parse_axis_key(axes: list, key: str, what: str = "The axis key") -> Point:
    """A point from its axis key: every axis, in order, with one of its values,
    written as ``axis_key`` writes it; raises ``ValueError`` with the reason."""
    parts = key.split("_") if key else []
    if len(parts) != len(axes):
        raise ValueError(f"{what} {key} has {len(parts)} parts for {len(axes)} axes.")
    out = []
    for a, part in zip(axes, parts):
        digits = part[len(a.prefix):] if part.startswith(a.prefix) else None
        if not digits or not digits.isdigit():
            raise ValueError(f"{what} {key} has {part} where {a.name} ({a.prefix}) belongs.")
        v = int(digits)
        if str(v) != digits:
            raise ValueError(f"{what} {key} writes {a.name} {v} as {digits}.")
        if v not in a.values:
            raise ValueError(f"{what} {key} gives {a.name} {digits}, which is not one of its values.")
        out.append((a.prefix, v))
    return tuple(out)


def shape_key(shape: Shape) -> str:
    """``n4096_k2048_m1``."""
    return "_".join(f"{d}{v}" for d, v in shape)


def shape_dim(d: str, shape: Shape) -> Optional[int]:
    return dict(shape).get(d)


@dataclass(frozen=True)
class Profile:
    """What tuning measured of a GPU that pruning uses: its CUs."""

    cores: int


@dataclass(frozen=True)
class Launch:
    """A variant's kernel for its class: the entry and how it is launched.
    ``params`` are the parameter struct's bytes."""

    entry: str
    groups: int
    threads: int
    lds_bytes: int
    params: bytes
    spans: tuple  # the bytes each buffer must hold, in the entry's order (0: unbound)

    def same_kernel(self) -> tuple:
        return (self.entry, self.groups, self.threads, self.lds_bytes, self.params)


class Illegal(Exception):
    """A point the family cannot build, with the findings."""

    def __init__(self, findings: list):
        super().__init__("; ".join(findings))
        self.findings = list(findings)


@dataclass
class Space:
    family: str
    axes: list
    shapes: list
    batch: list = field(default_factory=list)
    divides: Callable[[Shape, Point], list] = lambda s, p: []
    kernel: Callable[[str, Shape, Point], Launch] = None


@dataclass
class Variant:
    shape: Shape
    point: Point
    launch: Launch
    groups: int

    @property
    def ir_hash(self) -> int:
        return launch_hash(self.launch)


# What enumeration made of a point.
@dataclass
class Kept:
    variant: Variant


@dataclass
class IllegalOutcome:
    findings: list


@dataclass
class Indivisible:
    reasons: list


@dataclass
class TooFewGroups:
    groups: int


@dataclass
class SameAs:
    point: Point


Outcome = Union[Kept, IllegalOutcome, Indivisible, TooFewGroups, SameAs]


def variant_name(space: Space, shape: Shape, point: Point) -> str:
    """``family_class_x_axiskey``: ``family_class`` for a family without axes,
    ``family_x_axiskey`` for a class without dimensions."""
    cls = "_" + shape_key(shape) if shape_key(shape) else ""
    key = "_x_" + axis_key(point) if axis_key(point) else ""
    return space.family + cls + key


def split_join(valid: Callable[[str], bool], name: str) -> Optional[tuple]:
    """A name joined with ``_x_``, split back at the first ``_x_`` whose right
    side ``valid`` takes."""
    for i in range(len(name) - 2):
        if name[i:i + 3] == "_x_" and valid(name[i + 3:]):
            return name[:i], name[i + 3:]
    return None


def variant_of_name(space: Space, name: str) -> Optional[tuple]:
    """``variant_name``'s inverse: the class and point a name names."""
    if not space.axes:
        point = ()
    else:
        def valid(k):
            try:
                parse_axis_key(space.axes, k)
                return True
            except ValueError:
                return False
        sp = split_join(valid, name)
        if sp is None:
            return None
        point = parse_axis_key(space.axes, sp[1])
    for s in space.shapes:
        if variant_name(space, s, point) == name:
            return s, point
    return None


_LETTERS = re.compile(r"^[a-z]+$")


def _repeated(kvs):
    seen: dict = {}
    for k, v in kvs:
        seen.setdefault(k, []).append(v)
    return [(k, vs) for k, vs in sorted(seen.items()) if len(vs) > 1]


def check_space(space: Space) -> list:
    """What would make the space's names ambiguous or its classes misread."""
    out = []
    if "_x_" in space.family:
        out.append(f"The family {space.family} holds _x_, which joins a variant's name to its axis key.")
    out += [f"The axis {a.name}'s prefix \"{a.prefix}\" is not lowercase letters." for a in space.axes
            if not _LETTERS.match(a.prefix)]
    out += [f"The axes {' and '.join(names)} share the prefix {p}." for p, names in
            _repeated([(a.prefix, a.name) for a in space.axes])]
    out += [f"The axis {a.name} has no values." for a in space.axes if not a.values]
    for s in space.shapes:
        out += [f"The class {shape_key(s)}'s dimension \"{d}\" is not lowercase letters." for d, _ in s
                if not _LETTERS.match(d)]
        out += [f"The class {shape_key(s)} gives {d} {len(vs)} times." for d, vs in _repeated(list(s))]
    out += [f"The class {k} is given {len(vs)} times." for k, vs in
            _repeated([(shape_key(s), ()) for s in space.shapes])]
    out += [f"The batch dimension {b} is not a dimension of the class {shape_key(s)}." for b in space.batch
            for s in space.shapes if shape_dim(b, s) is None]
    return out


def launch_findings(launch: Launch) -> list:
    """The launch table's checks of a variant's launch, on the host, over
    distinct aligned fake addresses of the sizes the launch needs."""
    spans, at = [], 1 << 40
    for nbytes in launch.spans:
        if nbytes:
            spans.append((at, nbytes))
            at += (nbytes + 4095) // 4096 * 4096
        else:
            spans.append((0, 0))
    params = (ctypes.c_uint8 * len(launch.params)).from_buffer_copy(launch.params)
    try:
        runtime.launch_check(launch.entry, launch.groups, launch.threads, launch.lds_bytes, spans, params)
    except runtime.FkError as e:
        return [str(e)]
    return []


def _pruned(profile: Profile, space: Space, shape: Shape, point: Point):
    try:
        launch = space.kernel(variant_name(space, shape, point), shape, point)
    except Illegal as e:
        return IllegalOutcome(e.findings)
    findings = launch_findings(launch)
    if findings:
        return IllegalOutcome(findings)
    reasons = space.divides(shape, point)
    if reasons:
        return Indivisible(reasons)
    if launch.groups < 2 * profile.cores:
        return TooFewGroups(launch.groups)
    return launch


def consider(profile: Profile, space: Space, shape: Shape, point: Point) -> Outcome:
    """A point for a class, pruned by everything but duplicates."""
    r = _pruned(profile, space, shape, point)
    return Kept(Variant(shape, point, r, r.groups)) if isinstance(r, Launch) else r


def enumerate_class(profile: Profile, space: Space, shape: Shape) -> list:
    """Every point of a class and what pruning made of it; a point whose launch
    is a kept point's is that point's duplicate."""
    seen: dict = {}
    out = []
    for p in points(space.axes):
        r = _pruned(profile, space, shape, p)
        if not isinstance(r, Launch):
            out.append((p, r))
        elif r.same_kernel() in seen:
            out.append((p, SameAs(seen[r.same_kernel()])))
        else:
            seen[r.same_kernel()] = p
            out.append((p, Kept(Variant(shape, p, r, r.groups))))
    return out


def variants(profile: Profile, space: Space, shape: Shape) -> list:
    """The kept variants of a class, in enumeration order."""
    return [o.variant for _, o in enumerate_class(profile, space, shape) if isinstance(o, Kept)]


def launch_hash(launch: Launch) -> int:
    """What stands for the reference's IR hash of a variant's kernel: 64-bit
    FNV-1a over the source hash of the entry's own code (its defining header
    and what that includes, and its ABI hash) and the launch (entry,
    threadgroups, threads, LDS, parameter bytes), so that a pick is stale when
    its kernel's source or its launch changes, and only then."""
    from .manifest import entry_source_hash
    text = (f"{entry_source_hash(launch.entry):016x} {launch.entry} {launch.groups} {launch.threads} "
            f"{launch.lds_bytes} {launch.params.hex()}").encode()
    return runtime.library().fk_fnv1a64(text, len(text))
