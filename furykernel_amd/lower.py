"""A plan's steps as launches of the hand-written gfx950 kernels.

Each step of a plan (src/FuryKernel/Program/Plan.hs) is one launch.  A step's
shape — its anchors, the chains it recomputes, its epilogues, effects and
stores — picks the kernel and fills its parameters; buffers are named
logically (``value:``, ``weight:``, ``cache:``, ``ints:``, ``partials:``) and
the engine binds them to device memory.  A step of a shape no kernel here
takes is refused with ``LoweringError``: it is never run some other way.

This is pure host logic, the lowering a ``Backend Rocm`` does for the planned
step's kernels (src/FuryKernel/Backend.hs:29-101).
"""

from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass, field
from typing import Callable, Optional

import numpy as np

from .program.check import CheckedProgram
from .program.graph import (
    BF16, CACHE_BF16, F16, F32, GELU_TANH, SILU, U32, Add, ArgMax, Attend, CombineRanks, Concat, Gather, GatedGelu,
    GeluMul, Input, KvStore, Linear, LinearRouted, Paged, Ring, RmsNorm, Rope, ROPE_HALVES, Route, ScaleBy, SCache,
    SInput, Softcap, SRowInts, Standardize, STable, SWeight, op_values as _inputs_of)
from .program.plan import ANCHOR, COMBINE, EFFECT, EPILOGUE, LAND, RECOMPUTE, STAGE, Plan, Step, Stored, Work

THREADS = 256
ATTN_SPLIT = 128      # positions a split of the narrow attention covers (64 or 128)
ATTN_THREADS = 512
WIDE_RUN, WIDE_MAX_WAVES = 64, 8    # the wide attention: positions a wavefront, wavefronts a threadgroup
COMBINE_SPLITS = 8                  # splits the GEMV step's combine prologue takes


def wide_lds_floats(waves: int) -> int:
    """The wide attention's LDS (fk_attention.h: wide_lds_floats)."""
    return 512 + 64 + 8 + waves * (32 * 68 + 8 * 64 + 8 * 64 + 16 + 8)


MAX_K = 8192

# GEMV step prologue and epilogue modes (fk_step_gemv.h).
PRO_STORED, PRO_RMSNORM, PRO_GATHER, PRO_GATHER_RMSNORM, PRO_SILU_MUL, PRO_COMBINE = 0, 1, 2, 3, 4, 5
EPI_NONE, EPI_ADD_STORED, EPI_ADD_GATHER, EPI_SILU_MUL, EPI_ARGMAX, EPI_SOFTCAP = 0, 1, 2, 3, 4, 5
# Activations of an act·mul (the SiLU form this target adds, GELU-tanh the reference's).
ACT = {SILU: 0, GELU_TANH: 1}
# fk_step_elementwise's operations.
ELT_ADD, ELT_SCALE, ELT_STANDARDIZE, ELT_CONCAT = range(4)


class LoweringError(ValueError):
    """A step no kernel of this target takes."""


@dataclass(frozen=True)
class BufferSpec:
    name: str
    dtype: str   # "f32", "f16", "bf16", "u32", "u16", "u64"
    count: int   # elements

    @property
    def nbytes(self) -> int:
        return self.count * {"f32": 4, "u32": 4, "f16": 2, "bf16": 2, "u16": 2, "u64": 8}[self.dtype]


@dataclass
class Launch:
    step: str
    entry: str
    groups: int
    threads: int
    bind: dict      # binding name -> logical buffer name (None: unbound)
    params: dict    # parameter struct field -> value
    meta: dict = field(default_factory=dict)  # what the kernel's table buffers were made from
    lds_bytes: int = 0


@dataclass
class Lowered:
    program: object
    plan: Plan
    rows: int
    buffers: dict = field(default_factory=dict)  # name -> BufferSpec
    launches: list = field(default_factory=list)
    constants: dict = field(default_factory=dict)  # name -> what fills it: ("rope", theta, d, rotated, rows)
    layouts: dict = field(default_factory=dict)    # weight buffer -> (layout, source names) when not as given

    def buffer(self, name: str, dtype: str, count: int) -> str:
        spec = BufferSpec(name, dtype, count)
        old = self.buffers.get(name)
        if old is not None and old != spec:
            raise LoweringError(f"buffer {name} wanted as {spec} and {old}")
        self.buffers[name] = spec
        return name


def lower_plan(checked: CheckedProgram, plan: Plan, rows: int = 1, compute_units: int = 256,
               fuse: bool = True, wide: bool = False, choose: Optional[Callable] = None) -> Lowered:
    """The launches of every step of the plan, in order, for steps of `rows`
    rows (one, a decode step's), on a device of `compute_units` CUs.  With
    `fuse`, light steps fold into the launch before them: a KV store into the
    attention right after it, a stored act·mul into the GEMV step of its two
    anchors, the greedy token into the GEMV step of its logits, and the
    attention's combine into the GEMV step that reads its output.  With
    `wide`, attention over heads of 16, 32 or 64 runs in wide splits (at most
    8 a head, 64 positions a wavefront); else in splits of 128 positions.  The
    narrow splits are the default: at 4096 positions the wide kernel's 64
    threadgroups leave three CUs in four idle and are bound by each CU's LDS
    bandwidth (14-16 us a launch against 5.5 us for the narrow kernel and its
    combine's 3 us).  `choose`, given a GEMV step launch, may return the
    (rows a block, threadgroups a CU) a tuned selection picks for it (see
    ``tuning.committed_chooser``); a pick the launch cannot take is passed
    over.  None of these changes what any launch computes."""
    if rows != 1:
        raise LoweringError(f"steps of {rows} rows: the decode kernels take one row a step")
    out = Lowered(checked.program, plan, rows)
    low = _StepLowering(out, compute_units, wide, choose)
    for step in plan.steps:
        made = low.step(step)
        out.launches.extend(made if isinstance(made, list) else [made])
    if fuse:
        _fuse_attention(out)
        _fuse_light(out, compute_units, choose)
        _fuse_combine(out, compute_units, choose)
    return out


def _fuse_combine(out: Lowered, compute_units: int, choose: Optional[Callable] = None) -> None:
    """A combine launch whose output only the GEMV step right after it reads,
    as its stored input row, becomes that step's combine prologue: each of its
    threadgroups combines the partials (at most 8 splits a head) as the
    combine kernel does, then runs the GEMV on the row.  One launch fewer, and
    the row never leaves the registers: its buffer is dropped."""
    fused: list = []
    launches = out.launches
    for i, launch in enumerate(launches):
        prev = fused[-1] if fused else None
        if (prev is not None and prev.entry == "fk_step_combine" and launch.entry.startswith("fk_step_gemv")
                and launch.params["pro_mode"] == PRO_STORED and launch.bind["src"] == prev.bind["out"]
                and prev.params["splits"] <= COMBINE_SPLITS and prev.params["head_dim"] % 4 == 0
                and launch.params["k"] == prev.params["heads"] * prev.params["head_dim"]
                and not any(prev.bind["out"] in L.bind.values() for L in launches[i + 1:])
                and prev.bind["out"] not in _program_outputs(out)):
            launch.params.update(pro_mode=PRO_COMBINE, splits=prev.params["splits"],
                                 head_dim=prev.params["head_dim"])
            launch.bind["src"] = prev.bind["partials"]
            launch.step = f"{prev.step}+{launch.step}"
            _shape_gemv(launch, compute_units, choose=choose)
            del out.buffers[prev.bind["out"]]  # the combined row lives in registers only
            fused[-1] = launch
            continue
        fused.append(launch)
    out.launches = fused


def _program_outputs(out: Lowered) -> set:
    p = out.program
    return {f"value:{p.value(o.value).name}" for o in p.outputs}


def _fuse_attention(out: Lowered) -> None:
    """Folds a KV store step into the attention step right after it that
    reads those caches at the same position and sequence: one launch, whose
    threadgroup holding the position stores each kv head's new rows and
    takes them as that position's key and value, with the same arithmetic.
    (The combine stays a launch of its own: folding it in needs every split
    of a kv head to see the others' partials, a device-wide release and
    acquire that costs more on this GPU than the launch it saves.)"""
    fused: list = []
    for launch in out.launches:
        prev = fused[-1] if fused else None
        merged = None
        if prev is not None and launch.entry in ("fk_step_attend", "fk_step_attend_wide", "fk_step_attend_paged") \
                and prev.entry in ("fk_step_store", "fk_step_store_paged"):
            merged = _store_into_attend(prev, launch)
        if merged is not None:
            fused[-1] = merged
        else:
            fused.append(launch)
    out.launches = fused


def _store_into_attend(st: Launch, at: Launch) -> Optional[Launch]:
    sp, ap, sb, ab = st.params, at.params, st.bind, at.bind
    paged = at.entry == "fk_step_attend_paged"
    if paged != (st.entry == "fk_step_store_paged"):
        return None
    seq, c0, c1, kc, vc = ("table", "p0", "p1", "kpool", "vpool") if paged else ("slot", "c0", "c1", "kc", "vc")
    if sp["n_stores"] != 2 or ap["store"] or sb["position"] != ab["position"] or sb[seq] != ab[seq]:
        return None
    shape = ("kv_heads", "head_dim", "cache_bf16") + (("block_size", "table_len", "blocks") if paged
                                                      else ("length", "slots"))
    if any(sp[f] != ap[f] for f in shape):
        return None
    if (sb[c0], sb[c1]) == (ab[kc], ab[vc]):
        kj, vj = 0, 1
    elif (sb[c1], sb[c0]) == (ab[kc], ab[vc]):
        kj, vj = 1, 0
    else:
        return None
    krope = sp["rope"][kj]
    if sp["rope"][vj]:
        return None
    params, bind, meta = dict(ap), dict(ab), dict(at.meta)
    if krope:
        if ap["rope"]:
            if sb["rope"] != ab["rope"]:
                return None  # the key's RoPE and the query's differ: keep the store apart
        else:
            params.update(rotated=sp["rotated"], rope_rows=sp["rope_rows"])
            bind["rope"] = sb["rope"]
    meta["store_theta"] = st.meta["theta"]
    params.update(store=1, krope=krope)
    bind.update(knew=sb[f"x{kj}"], vnew=sb[f"x{vj}"])
    return Launch(f"{st.step}+{at.step}", at.entry, at.groups, at.threads, bind, params, meta, at.lds_bytes)


def _fuse_light(out: Lowered, compute_units: int, choose: Optional[Callable] = None) -> None:
    """A light step of one stored act·mul (SiLU or GELU-tanh) of the two
    anchors of the GEMV step right before it becomes that step's epilogue: its
    wavefronts hold row j of both anchors and store act(gate_j) * up_j — the
    light kernel's arithmetic.  A light step of the greedy token of the row the
    GEMV step before it stores (its tile, or the softcap its epilogue stores)
    becomes part of that step's epilogue (each row's argmax key into a 64-bit
    maximum) and a one-thread launch that turns the key into the token."""
    fused: list = []
    for launch in out.launches:
        prev = fused[-1] if fused else None
        if prev is not None and prev.entry.startswith("fk_step_gemv"):
            pp, pb = prev.params, prev.bind
            epi = pp["epi_mode"]
            if (epi == EPI_NONE and launch.entry == "fk_step_act_mul" and launch.params["b_off"] == 0
                    and pp["n_anchors"] == 2 and pp["rows"][0] == pp["rows"][1]
                    and pb["y0"] == launch.bind["a"] and pb["y1"] == launch.bind["b"]):
                pp["epi_mode"] = EPI_SILU_MUL
                pp["act"] = launch.params["act"]
                pb["epi_out"] = launch.bind["y"]
                prev.step = f"{prev.step}+{launch.step}"
                _shape_gemv(prev, compute_units, choose=choose)
                continue
            keyed = (epi == EPI_NONE and pp["n_anchors"] == 1 and pp["store_tile"] and pb["y0"] == launch.bind.get("x")) \
                or (epi == EPI_SOFTCAP and pb["epi_out"] == launch.bind.get("x"))
            if launch.entry == "fk_step_argmax" and keyed:
                if epi == EPI_NONE:
                    pp["epi_mode"] = EPI_ARGMAX
                prev.step = f"{prev.step}+{launch.step}"
                _shape_gemv(prev, compute_units, choose=choose)
                arg = out.buffer(f"argmax:{launch.bind['out'].split(':', 1)[1]}", "u64", prev.groups)
                pb["arg"] = arg
                pp["arg_slots"] = prev.groups
                fused.append(Launch(launch.step, "fk_step_token", 1, 64,
                                    {"arg": arg, "out": launch.bind["out"], "token": None, "position": None},
                                    {"slots": prev.groups, "context": 1, "step": 0, "advance": 0}))
                continue
        fused.append(launch)
    out.launches = fused


GEMV_THREADS = 512


def _shape_gemv(launch: Launch, compute_units: int, rows: Optional[int] = None, per_cu: int = 2,
                choose: Optional[Callable] = None) -> None:
    """The GEMV step variant for the launch's weights, input width, rows and
    epilogue — rows a block, packs a lane — and its grid: blocks of rows, and
    threadgroups of 8 wavefronts up to `per_cu` a CU, each wavefront taking
    blocks in turn.  `rows` (1 or 2) asks for that many rows a block where the
    input width has both; by default 2 for a pair epilogue or more than 4096
    rows.  `choose` (see ``lower_plan``) may pick both."""
    if choose is not None and rows is None:
        pick = choose(launch)
        if pick is not None:
            saved = (launch.entry, launch.groups, launch.threads, launch.lds_bytes, dict(launch.params))
            try:
                _shape_gemv(launch, compute_units, rows=pick[0], per_cu=pick[1])
                if launch.entry.split("_r")[1].split("_")[0] == str(pick[0]):
                    return
            except LoweringError:
                pass
            launch.entry, launch.groups, launch.threads, launch.lds_bytes = saved[:4]
            launch.params.clear()
            launch.params.update(saved[4])
    p = launch.params
    k, wt = p["k"], launch.meta["wtype"]
    total = p["first_row"][p["n_anchors"]]
    pairs = p["epi_mode"] == EPI_SILU_MUL
    if wt in (F16, BF16):
        if k <= 2048:
            r = rows if rows in (1, 2) else (2 if pairs or total > 4096 else 1)
            entry, kmax = f"fk_step_gemv_{wt}_k2048_r{r}", 2048
        elif k <= MAX_K:
            r, entry, kmax = 1, f"fk_step_gemv_{wt}_k8192_r1", 8192
        else:
            raise LoweringError(f"{launch.step}: an input row of {k}; the {wt} GEMV steps take up to {MAX_K}")
    elif wt == F32:
        r = rows if rows in (1, 2) else (2 if pairs else 1)
        if k <= 256:
            entry, kmax = f"fk_step_gemv_f32_k256_r{r}", 256
        elif k <= 1024:
            entry, kmax = f"fk_step_gemv_f32_k1024_r{r}", 1024
        else:
            raise LoweringError(f"{launch.step}: an input row of {k}; the f32 GEMV steps take up to 1024")
    else:
        raise LoweringError(f"{launch.step}: weights of {wt}")
    entry = f"{entry}_p{p['pro_mode']}_e{p['epi_mode']}"
    if p["epi_mode"] == EPI_SILU_MUL:
        if r == 1 and k > 2048 and wt in (F16, BF16):
            raise LoweringError(f"{launch.step}: no SiLU·mul epilogue at an input row of {k}")
        # r 2: row j of both anchors a block; r 1: row j of the first anchor,
        # then of the second, in blocks 2j and 2j + 1.
        blocks = 2 * p["rows"][0] if r == 1 else -(-p["rows"][0] // (r // 2))
    else:
        blocks = -(-total // r)
    p["blocks"] = blocks
    launch.entry = entry
    launch.threads = GEMV_THREADS
    waves = GEMV_THREADS // 64
    launch.groups = max(1, min(-(-blocks // waves), per_cu * compute_units))
    # The input row transposed in LDS, padded to the variant's widest row, and
    # the norm's gains beside it.
    norm = p["pro_mode"] in (PRO_RMSNORM, PRO_GATHER_RMSNORM)
    launch.lds_bytes = kmax * 4 * (2 if norm else 1)


def rope_table(theta: float, d: int, rotated: int, rows: int) -> np.ndarray:
    """RoPE's cosines and sines by position: row p holds (cos, sin) of pair i's
    angle, the binary32 product p * theta^(-2i/d), the frequency and the
    cosine and sine each binary64's rounded once to binary32 (the contract of
    src/FuryKernel/Program/Eval.hs:819-829 with tables)."""
    t32 = float(np.float32(theta))
    freqs = np.array([math.pow(t32, -(2.0 * i) / d) for i in range(rotated)], np.float32)
    angles = (np.arange(rows, dtype=np.float32)[:, None] * freqs[None, :]).astype(np.float32).ravel().tolist()
    out = np.empty((rows * rotated, 2), np.float32)
    out[:, 0] = [math.cos(a) for a in angles]
    out[:, 1] = [math.sin(a) for a in angles]
    return out.reshape(rows, rotated, 2)


class _StepLowering:
    def __init__(self, out: Lowered, compute_units: int = 256, wide: bool = True,
                 choose: Optional[Callable] = None):
        self.out = out
        self.compute_units = compute_units
        self.wide = wide
        self.choose = choose
        self.materialized: set = set()  # values a launch of an earlier part of the step made
        self.p = out.program
        self.producer = {v: n for n in self.p.nodes for v in n.outputs}

    # Buffers -------------------------------------------------------------------

    def value(self, v: int) -> str:
        val = self.p.value(v)
        prod = self.producer.get(v)
        if prod is not None and isinstance(prod.op, Input):
            src = self.p.source(prod.op.source)
            if isinstance(src.kind, SInput) and src.kind.type not in (F32,):
                raise LoweringError(f"input {src.name} of {src.kind.type}: the kernels read f32 rows")
        dtype = "u32" if val.type == U32 else "f32"
        return self.out.buffer(f"value:{val.name}", dtype, val.shape.width * self.out.rows)

    def weight(self, s: int) -> tuple[str, str]:
        src = self.p.source(s)
        if not isinstance(src.kind, SWeight):
            raise LoweringError(f"{src.name} is not a weight")
        t = src.kind.type
        if t not in (F16, BF16, F32):
            raise LoweringError(f"weight {src.name} of {t}: the GEMV steps take f16, bf16 and f32 weights")
        return self.out.buffer(f"weight:{src.name}", t, int(np.prod(src.kind.dims))), t

    def gains(self, s: int) -> str:
        """An RMSNorm's gains as the f32 row the kernels read: an f32 weight as
        it is, a bf16 or f16 one widened (exactly) into a buffer of its own."""
        name, t = self.weight(s)
        if t == F32:
            return name
        src = self.p.source(s)
        wide = self.out.buffer(f"widen:{src.name}", "f32", int(np.prod(src.kind.dims)))
        self.out.layouts[wide] = ("widen", (src.name,))
        return wide

    def ints(self, s: int) -> str:
        src = self.p.source(s)
        if not isinstance(src.kind, SRowInts):
            raise LoweringError(f"{src.name} is not a row of integers")
        return self.out.buffer(f"ints:{src.name}", "u32", src.kind.count * self.out.rows)

    def cache(self, s: int) -> tuple[str, object, bool]:
        """A ring's buffer; for a paged pool, the address table of its blocks
        (u64, one a block), whose buffer ``cache:<name>`` holds the blocks in
        order and whose addresses the engine writes (the constant
        ("addresses", pool, block bytes))."""
        src = self.p.source(s)
        if not isinstance(src.kind, SCache):
            raise LoweringError(f"{src.name} is not a cache")
        lay = src.kind.layout
        bf16 = src.kind.elem == CACHE_BF16
        elem = "bf16" if bf16 else "f16"
        if isinstance(lay, Paged):
            block = lay.block_size * lay.kv_heads * lay.head_dim
            pool = self.out.buffer(f"cache:{src.name}", elem, lay.blocks * block)
            addr = self.out.buffer(f"addr:{src.name}", "u64", lay.blocks)
            self.out.constants[addr] = ("addresses", pool, block * 2)
            return addr, lay, bf16
        count = lay.slots * lay.kv_heads * lay.length * lay.head_dim
        return self.out.buffer(f"cache:{src.name}", elem, count), lay, bf16

    def paging(self, lay, table: int) -> dict:
        """A paged pool's paging fields, the row's table of the source `table`."""
        src = self.p.source(table)
        return {"block_size": lay.block_size, "table_len": src.kind.count, "blocks": lay.blocks}

    def rope(self, spec, d: int, rows: int) -> str:
        name = f"rope:{spec.theta!r}:{d}:{spec.rotated}:{rows}"
        self.out.buffer(name, "f32", rows * spec.rotated * 2)
        self.out.constants[name] = ("rope", float(spec.theta), d, spec.rotated, rows)
        return name

    def stored_before(self, step: Step, v: int) -> bool:
        if v in self.materialized:
            return True
        prod = self.producer.get(v)
        if prod is not None and isinstance(prod.op, Input):
            return True
        return any(st.value == v and st.form[0] == "elements" for st in step.reads)

    # Steps -----------------------------------------------------------------------

    def step(self, step: Step):
        """The step's launches: one fused kernel where the step's work fits
        one (its recomputes in the kernel's prologue), else the fewest of its
        recomputes, in plan order, made first by launches of their own
        (``light_launch``) and read as stored by the rest."""
        kinds = {w.kind for w in step.work}
        if STAGE in kinds or LAND in kinds:
            raise LoweringError(f"{step.name}: staged stores are not lowered yet")
        try:
            return self.fused_step(step)
        except LoweringError as first:
            last = first
            recs = [w for w in step.work if w.kind == RECOMPUTE]
            for k in range(1, len(recs) + 1):
                saved = (set(self.materialized), dict(self.out.buffers), dict(self.out.constants),
                         dict(self.out.layouts))
                try:
                    made = []
                    for w in recs[:k]:
                        L = self.light_launch(step, self.p.node(w.node))
                        made.append(L)
                        self.materialized |= set(L.meta["values"])
                    done = {v for L in made for v in L.meta["values"]}
                    rest = dataclasses.replace(step, work=[w for w in step.work if w not in recs[:k]],
                                               stores=[st for st in step.stores if st.value not in done])
                    if not rest.work:
                        return made
                    more = self.fused_step(rest)
                    return made + (more if isinstance(more, list) else [more])
                except LoweringError as e:
                    last = e
                    self.materialized, bufs, consts, lays = saved
                    for d, old in ((self.out.buffers, bufs), (self.out.constants, consts), (self.out.layouts, lays)):
                        d.clear()
                        d.update(old)
            raise last if recs else first

    def fused_step(self, step: Step):
        kinds = {w.kind for w in step.work}
        anchors = [self.p.node(w.node) for w in step.work if w.kind == ANCHOR]
        groups = self.anchor_groups(anchors)
        if len(groups) > 1:
            out = []
            for g in groups:
                made = self.fused_step(self.sub_step(step, g))
                out += made if isinstance(made, list) else [made]
            return out
        if anchors and any(isinstance(a.op, LinearRouted) for a in anchors):
            return self.routed_step(step, anchors)
        # An RMSNorm the step recomputes and stores: made once by its own
        # launch, then read as stored by the rest of the step.
        pre = []
        for w in step.work:
            node = self.p.node(w.node)
            if w.kind == RECOMPUTE and isinstance(node.op, RmsNorm) and \
                    any(st.value == node.outputs[0] for st in step.stores) and self.stored_before(step, node.op.x):
                pre.append(self.norm_launch(step, node))
        if pre:
            made = {L.bind["y"] for L in pre}
            kept = [w for w in step.work if not (w.kind == RECOMPUTE and
                                                 self.value(self.p.node(w.node).outputs[0]) in made)]
            step = dataclasses.replace(step, work=kept,
                                       stores=[st for st in step.stores if self.value(st.value) not in made])
            for L in pre:
                self.materialized.add(L.meta["value"])
            rest = self.step(step)
            return pre + (rest if isinstance(rest, list) else [rest])
        if anchors and all(isinstance(a.op, Linear) for a in anchors):
            return self.gemv_step(step, anchors)
        if len(anchors) == 1 and isinstance(anchors[0].op, Attend):
            return self.attend_step(step, anchors[0])
        if anchors:
            raise LoweringError(f"{step.name}: anchors of mixed or unknown kinds")
        if EFFECT in kinds:
            return self.store_step(step)
        if COMBINE in kinds:
            return self.combine_step(step)
        return self.light_step(step)

    def anchor_groups(self, anchors: list) -> list:
        """Anchors one kernel cannot take together, apart: linear layers by
        their input row, routed ones each alone."""
        groups: dict = {}
        for a in anchors:
            key = ("routed", a.id) if isinstance(a.op, LinearRouted) else \
                ("linear", a.op.x) if isinstance(a.op, Linear) else ("other", a.id)
            groups.setdefault(key, []).append(a)
        return list(groups.values())

    def sub_step(self, step: Step, anchors: list) -> Step:
        """The part of a step that makes these anchors: the recomputes their
        inputs come from, the epilogues on their tiles, the stores of what
        they and those make."""
        recs = {self.p.node(w.node).outputs[0]: w for w in step.work if w.kind == RECOMPUTE}
        ids = {a.id for a in anchors}
        need, todo = set(), [v for a in anchors for v in _inputs_of(a.op)]
        while todo:
            v = todo.pop()
            if v in recs and v not in need:
                need.add(v)
                todo += _inputs_of(self.p.node(recs[v].node).op)
        tiles = {v for a in anchors for v in a.outputs}
        work = []
        for w in step.work:
            node = self.p.node(w.node)
            if (w.kind == ANCHOR and w.node in ids) or (w.kind == RECOMPUTE and node.outputs[0] in need) or \
                    (w.kind == EPILOGUE and tiles & set(_inputs_of(node.op))):
                work.append(w)
        made = {v for w in work for v in self.p.node(w.node).outputs}
        return dataclasses.replace(step, work=work, stores=[st for st in step.stores if st.value in made])

    def light_launch(self, step: Step, node) -> Launch:
        """One recomputed value made by a launch of its own, from stored (or
        already made) values, into its value buffer: the step's fused kernel
        then reads it as stored.  ``meta["values"]`` names what it makes."""
        op = node.op
        out = node.outputs[0]
        name = f"{step.name}:{self.p.value(out).name}"
        for v in _inputs_of(op):
            if not self.stored_before(step, v):
                raise LoweringError(f"{step.name}: {self.p.value(out).name} of a value neither stored nor made")
        width = self.p.value(out).shape.width
        grid = max(1, -(-width // THREADS))

        def elementwise(eop, a, b=None, c=None, w=None, wb=0, factor=1.0):
            params = {"n": width, "op": eop, "width": w or width, "width_b": wb, "factor": float(np.float32(factor))}
            bind = {"a": a, "b": b or a, "c": c or a, "y": self.value(out)}
            return Launch(name, "fk_step_elementwise", grid, THREADS, bind, params, {"values": [out]})

        if isinstance(op, Add):
            return elementwise(ELT_ADD, self.value(op.a), self.value(op.b))
        if isinstance(op, ScaleBy):
            return elementwise(ELT_SCALE, self.value(op.x), self.gains(op.weight))
        if isinstance(op, Standardize):
            seg = self.p.value(op.x).shape.width
            bias, scale = self.gains(op.bias), self.gains(op.scale)
            if int(np.prod(self.p.source(op.bias).kind.dims)) < seg or \
                    int(np.prod(self.p.source(op.scale).kind.dims)) < seg:
                raise LoweringError(f"{step.name}: a standardize of rows of {seg} by a narrower bias or scale")
            return elementwise(ELT_STANDARDIZE, self.value(op.x), bias, scale, w=seg, factor=op.factor)
        if isinstance(op, Concat):
            wa, wb = self.p.value(op.a).shape.width, self.p.value(op.b).shape.width
            return elementwise(ELT_CONCAT, self.value(op.a), self.value(op.b), w=wa, wb=wb)
        if isinstance(op, Gather):
            tname, ttype = self.weight(op.table)
            tsrc = self.p.source(op.tokens)
            rows_ = self.p.source(op.table).kind.dims[0]
            params = {"rows": 1, "width": width, "count": tsrc.kind.count, "table_rows": rows_,
                      "factor": float(np.float32(op.factor))}
            return Launch(name, f"fk_step_gather_{ttype}", grid, THREADS,
                          {"table": tname, "tokens": self.ints(op.tokens), "y": self.value(out)}, params,
                          {"values": [out]})
        if isinstance(op, RmsNorm):
            L = self.norm_launch(step, node)
            L.meta["values"] = [out]
            return L
        if isinstance(op, Route):
            return self.route_launch(step, node)
        if isinstance(op, (GeluMul, GatedGelu, Softcap, ArgMax, CombineRanks)):
            shape = self.p.value(op.x if not isinstance(op, GeluMul) else op.a).shape
            if isinstance(op, GatedGelu) and shape.segment != shape.width:
                L = self.gated_launch(step, node)
                return L
            one = dataclasses.replace(step, work=[Work(RECOMPUTE, node.id)], stores=[Stored(out, ("elements", F32))])
            L = self.light_step(one)
            L.step = name
            L.meta = dict(L.meta or {}, values=[out])
            return L
        raise LoweringError(f"{step.name}: no launch of its own makes {type(op).__name__}")

    def recomputes(self, step: Step) -> dict:
        return {self.p.node(w.node).outputs[0]: self.p.node(w.node) for w in step.work if w.kind == RECOMPUTE}

    def gemv_step(self, step: Step, anchors: list) -> Launch:
        if len(anchors) > 3:
            raise LoweringError(f"{step.name}: {len(anchors)} anchors; a GEMV step takes up to 3")
        xs = {a.op.x for a in anchors}
        if len(xs) != 1:
            raise LoweringError(f"{step.name}: anchors of different inputs")
        x = xs.pop()
        rec = self.recomputes(step)
        k = self.p.value(x).shape.width
        if k % 8 and k % 4 == 0:
            return self.small_gemv_step(step, anchors, x)
        used: set = set()
        bind: dict = {k: None for k in ("w0", "w1", "w2", "y0", "y1", "y2", "src", "src2", "gamma", "table", "token",
                                        "res", "res_table", "res_token", "epi_out", "arg")}
        params: dict = {"eps": 0.0, "factor": 1.0, "gfactor": 1.0, "has_gamma": 0, "table_rows": 1, "arg_slots": 0,
                        "act": 0, "src2_off": 0, "cap": 0.0}
        wtypes = set()
        k = self.p.value(x).shape.width
        if k > MAX_K or k % 8:
            raise LoweringError(f"{step.name}: an input row of {k}, not a multiple of 8 up to {MAX_K}")

        gathers: list = []

        def gather_of(v: int):
            n = rec.get(v)
            if n is None or not isinstance(n.op, Gather):
                return None
            tsrc = self.p.source(n.op.tokens)
            if not isinstance(tsrc.kind, SRowInts) or tsrc.kind.count != 1:
                raise LoweringError(f"{step.name}: a gather of several rows is not lowered yet")
            used.add(v)
            tname, ttype = self.weight(n.op.table)
            rows_, factor = self.p.source(n.op.table).kind.dims[0], float(np.float32(n.op.factor))
            # One launch's gathers share table_rows and gfactor (the prologue's
            # and the epilogue's): a second gather must be of the same table.
            if gathers and gathers[0] != (tname, rows_, factor):
                raise LoweringError(f"{step.name}: gathers of two tables or factors in one launch")
            gathers.append((tname, rows_, factor))
            params["table_rows"], params["gfactor"] = rows_, factor
            return tname, self.ints(n.op.tokens), ttype

        # Prologue: how the anchors' input row is made.
        if x not in rec:
            if not self.stored_before(step, x):
                raise LoweringError(f"{step.name}: the anchors' input is neither stored nor recomputed")
            pro = PRO_STORED
            bind["src"] = self.value(x)
        else:
            node = rec[x]
            used.add(x)
            op = node.op
            if isinstance(op, RmsNorm):
                params["eps"] = float(np.float32(op.eps))
                params["factor"] = float(np.float32(op.factor))
                params["seg"] = self.p.value(op.x).shape.segment
                if op.gamma is not None:
                    params["has_gamma"] = 1
                    bind["gamma"] = self.gains(op.gamma)
                else:
                    # The kernel loads gains whatever the norm: a row of ones
                    # it never multiplies by.
                    width = self.p.value(op.x).shape.width
                    bind["gamma"] = self.out.buffer(f"ones:{width}", "f32", width)
                    self.out.constants[bind["gamma"]] = ("ones",)
                g = gather_of(op.x)
                if g is not None:
                    pro = PRO_GATHER_RMSNORM
                    bind["table"], bind["token"], gtype = g
                    wtypes.add(gtype)
                elif self.stored_before(step, op.x):
                    pro = PRO_RMSNORM
                    bind["src"] = self.value(op.x)
                else:
                    raise LoweringError(f"{step.name}: an RMSNorm of a value neither stored nor gathered")
            elif isinstance(op, Gather):
                pro = PRO_GATHER
                bind["table"], bind["token"], gtype = gather_of(x)
                wtypes.add(gtype)
            elif isinstance(op, GeluMul) and op.form in ACT:
                if not (self.stored_before(step, op.a) and self.stored_before(step, op.b)):
                    raise LoweringError(f"{step.name}: an act·mul of values not stored")
                pro = PRO_SILU_MUL
                params["act"] = ACT[op.form]
                bind["src"], bind["src2"] = self.value(op.a), self.value(op.b)
            elif isinstance(op, GatedGelu) and op.form in ACT:
                # act(first half) * second half of one stored row, whose one
                # segment is the whole row (Eval.hs:356-362).
                shape = self.p.value(op.x).shape
                if shape.segment != shape.width or not self.stored_before(step, op.x):
                    raise LoweringError(f"{step.name}: a gated activation in segments of {shape.segment} of a row "
                                        f"of {shape.width}, or of a value not stored")
                pro = PRO_SILU_MUL
                params["act"], params["src2_off"] = ACT[op.form], shape.width // 2
                bind["src"] = bind["src2"] = self.value(op.x)
            else:
                raise LoweringError(f"{step.name}: no prologue computes {type(op).__name__}")
        params["pro_mode"] = pro
        params.setdefault("seg", k)
        if params["seg"] != k or k % 4:
            raise LoweringError(f"{step.name}: RMSNorm in segments of {params['seg']} of a row of {k}; the GEMV "
                                f"prologue norms the whole row")

        # Anchors: their rows one after another.
        rows, first, g = [], [0], 0
        anchor_outs = {}
        for j, a in enumerate(anchors):
            wname, wt = self.weight(a.op.weight)
            wtypes.add(wt)
            bind[f"w{j}"] = wname
            n = self.p.value(a.outputs[0]).shape.width
            rows.append(n)
            g += n
            first.append(g)
            anchor_outs[a.outputs[0]] = j
        if len(wtypes) != 1:
            raise LoweringError(f"{step.name}: weights of several types {wtypes}")
        wt = wtypes.pop()

        # Epilogues: one residual add, or one softcap, on a single anchor's tile.
        epis = [self.p.node(w.node) for w in step.work if w.kind == EPILOGUE]
        epi, epi_value = EPI_NONE, None
        if epis and len(epis) == 1 and len(anchors) == 1 and isinstance(epis[0].op, Softcap):
            if epis[0].op.x != anchors[0].outputs[0]:
                raise LoweringError(f"{step.name}: a softcap off its anchor's tile")
            cap = float(np.float32(epis[0].op.cap))
            if not 0 < cap < math.inf:
                raise LoweringError(f"{step.name}: a softcap of {epis[0].op.cap}")
            epi, epi_value = EPI_SOFTCAP, epis[0].outputs[0]
            params["cap"] = cap
        elif epis:
            if len(epis) != 1 or len(anchors) != 1 or not isinstance(epis[0].op, Add):
                raise LoweringError(f"{step.name}: epilogues other than one residual add or one softcap on one anchor")
            op = epis[0].op
            tile = anchors[0].outputs[0]
            if tile not in (op.a, op.b):
                raise LoweringError(f"{step.name}: an epilogue off its anchor's tile")
            other = op.b if op.a == tile else op.a
            g2 = gather_of(other)
            if g2 is not None:
                epi = EPI_ADD_GATHER
                bind["res_table"], bind["res_token"], rtype = g2
                # The kernel reads the residual's table as the weights' type.
                if rtype != wt:
                    raise LoweringError(f"{step.name}: a residual gathered from a table of {rtype} under weights of "
                                        f"{wt}; the kernel reads both as one type")
            elif self.stored_before(step, other):
                epi = EPI_ADD_STORED
                bind["res"] = self.value(other)
            else:
                raise LoweringError(f"{step.name}: a residual neither stored nor gathered")
            epi_value = epis[0].outputs[0]
        params["epi_mode"] = epi
        leftover = set(rec) - used
        if leftover:
            raise LoweringError(f"{step.name}: recomputes {[self.p.value(v).name for v in leftover]} no kernel takes")

        # Stores: the anchors' tiles, or the epilogue's value.
        store_tile = 0
        for st in step.stores:
            if st.form[0] != "elements":
                raise LoweringError(f"{step.name}: stores of {st.form}")
            if st.value in anchor_outs:
                store_tile = 1
                bind[f"y{anchor_outs[st.value]}"] = self.value(st.value)
            elif st.value == epi_value:
                bind["epi_out"] = self.value(st.value)
            else:
                raise LoweringError(f"{step.name}: stores {self.p.value(st.value).name}, which no kernel output holds")
        if store_tile and len([st for st in step.stores if st.value in anchor_outs]) != len(anchors):
            raise LoweringError(f"{step.name}: some anchors' tiles stored and some not")
        if epi != EPI_NONE and bind["epi_out"] is None:
            raise LoweringError(f"{step.name}: an epilogue whose value isn't stored")
        params.update(n_anchors=len(anchors), rows=rows + [0] * (3 - len(rows)),
                      first_row=first + [g] * (4 - len(first)), k=k, store_tile=store_tile)
        launch = Launch(step.name, "", 0, GEMV_THREADS, bind, params, {"wtype": wt})
        _shape_gemv(launch, self.compute_units, choose=self.choose)
        return launch

    def small_gemv_step(self, step: Step, anchors: list, x: int) -> list:
        """Linear anchors over a row of a multiple of 4 elements but not of a
        16-byte pack: a launch each (fk_gemv_p4_*, a wavefront a row, packs of
        4), from the stored row, their tiles stored."""
        if any(w.kind not in (ANCHOR,) for w in step.work) or not self.stored_before(step, x):
            raise LoweringError(f"{step.name}: a linear layer over a row of {self.p.value(x).shape.width} with "
                                f"other work, or of a row not stored")
        outs = {a.outputs[0] for a in anchors}
        if {st.value for st in step.stores} != outs:
            raise LoweringError(f"{step.name}: a linear layer over a short row whose tiles are not all stored")
        k = self.p.value(x).shape.width
        launches = []
        for a in anchors:
            wname, wt = self.weight(a.op.weight)
            n = self.p.value(a.outputs[0]).shape.width
            launches.append(Launch(step.name, f"fk_gemv_p4_{wt}", -(-n // 4), THREADS,
                                   {"w": wname, "x": self.value(x), "y": self.value(a.outputs[0])},
                                   {"n": n, "k": k}))
        return launches

    def rope_of(self, step: Step, node, rec: dict) -> Optional[int]:
        if not isinstance(node.op, Rope):
            return None
        spec = node.op.spec
        if spec.axes != 1 or spec.pairs != ROPE_HALVES:
            raise LoweringError(f"{step.name}: RoPE of {spec.axes} axes is not lowered yet")
        return node.op.x

    def store_step(self, step: Step) -> Launch:
        rec = self.recomputes(step)
        effects = [self.p.node(w.node) for w in step.work if w.kind == EFFECT]
        if not 1 <= len(effects) <= 2 or not all(isinstance(e.op, KvStore) for e in effects):
            raise LoweringError(f"{step.name}: effects other than one or two KV stores")
        paged = isinstance(self.p.source(effects[0].op.at.cache).kind.layout, Paged)
        c, seq = ("p", "table") if paged else ("c", "slot")
        bind = {"x0": None, "x1": None, f"{c}0": None, f"{c}1": None, "position": None, seq: None, "rope": None}
        params: dict = {"n_stores": len(effects), "rope": [0, 0], "rotated": 0, "rope_rows": 1}
        meta: dict = {"theta": 1.0}
        layouts, used = set(), set()
        for j, e in enumerate(effects):
            at = e.op.at
            cname, lay, bf16 = self.cache(at.cache)
            if isinstance(lay, Paged) != paged:
                raise LoweringError(f"{step.name}: stores into a ring and a paged pool")
            layouts.add((lay.kv_heads, lay.head_dim, bf16) + ((lay.block_size, lay.blocks) if paged
                                                              else (lay.length, lay.slots)))
            bind[f"{c}{j}"] = cname
            pos, slot = self.ints(at.positions), self.ints(at.sequences)
            if bind["position"] not in (None, pos) or bind[seq] not in (None, slot):
                raise LoweringError(f"{step.name}: stores at different positions or sequences")
            bind["position"], bind[seq] = pos, slot
            if paged:
                params.update(self.paging(lay, at.sequences))
            v = e.op.x
            if v in rec:
                inner = self.rope_of(step, rec[v], rec)
                if inner is None or not self.stored_before(step, inner):
                    raise LoweringError(f"{step.name}: a stored value recomputed by other than RoPE of a stored row")
                used.add(v)
                spec = rec[v].op.spec
                if params["rope"] != [0, 0] and (params["rotated"], meta["theta"]) != (
                        spec.rotated, float(np.float32(spec.theta))):
                    raise LoweringError(f"{step.name}: two RoPEs of different specs")
                params["rope"][j] = 1
                params["rotated"] = spec.rotated
                meta["theta"] = float(np.float32(spec.theta))
                rope_rows = self.p.source(at.positions).kind.bound
                params["rope_rows"] = rope_rows
                bind["rope"] = self.rope(spec, self.p.value(inner).shape.segment, rope_rows)
                bind[f"x{j}"] = self.value(inner)
            elif self.stored_before(step, v):
                bind[f"x{j}"] = self.value(v)
            else:
                raise LoweringError(f"{step.name}: a store of a value neither stored nor recomputed")
        if len(layouts) != 1:
            raise LoweringError(f"{step.name}: stores into caches of different layouts")
        if set(rec) - used:
            raise LoweringError(f"{step.name}: recomputes no store kernel takes")
        if step.stores:
            raise LoweringError(f"{step.name}: a store step that also stores values")
        kv, d, bf16, a, b = layouts.pop()
        params.update(kv_heads=kv, head_dim=d, cache_bf16=int(bf16), length=0 if paged else a,
                      slots=0 if paged else b)
        if bind["rope"] is None:
            bind["rope"] = bind["position"]  # bound but never read
        return Launch(step.name, "fk_step_store_paged" if paged else "fk_step_store", 1, THREADS, bind, params, meta)

    def attend_step(self, step: Step, anchor) -> Launch:
        op = anchor.op
        spec = op.spec
        rec = self.recomputes(step)
        if spec.head_dim > 64 or spec.heads // spec.kv_heads > 8:
            raise LoweringError(f"{step.name}: heads of {spec.head_dim} or groups of {spec.heads // spec.kv_heads}")
        kname, lay, bf16 = self.cache(op.to.keys)
        vname, vlay, _ = self.cache(op.to.values)
        if spec.head_dim % 8:
            raise LoweringError(f"{step.name}: heads of {spec.head_dim}, not a multiple of 8")
        paged = isinstance(lay, Paged)
        if paged != isinstance(vlay, Paged):
            raise LoweringError(f"{step.name}: keys and values of a ring and a paged pool")
        span = lay.block_size * self.p.source(op.to.sequences).kind.count if paged else lay.length
        params = {"heads": spec.heads, "kv_heads": spec.kv_heads, "head_dim": spec.head_dim, "length": span,
                  "slots": 0 if paged else lay.slots, "split": ATTN_SPLIT, "rope": 0, "rotated": 0,
                  "rope_rows": 1, "scale": float(np.float32(spec.scale)), "window": spec.window or 0,
                  "cache_bf16": int(bf16), "store": 0, "krope": 0, "has_reach": int(spec.reach is not None)}
        if paged:
            params.update(self.paging(lay, op.to.sequences))
        meta = {"theta": 1.0}
        rope_buf = None
        q = op.q
        if q in rec:
            inner = self.rope_of(step, rec[q], rec)
            if inner is None or not self.stored_before(step, inner):
                raise LoweringError(f"{step.name}: queries recomputed by other than RoPE of a stored row")
            rspec = rec[q].op.spec
            rope_rows = self.p.source(op.to.positions).kind.bound
            params.update(rope=1, rotated=rspec.rotated, rope_rows=rope_rows)
            meta["theta"] = float(np.float32(rspec.theta))
            rope_buf = self.rope(rspec, spec.head_dim, rope_rows)
            qbuf = self.value(inner)
            if set(rec) - {q}:
                raise LoweringError(f"{step.name}: recomputes the attention kernel doesn't take")
        elif self.stored_before(step, q):
            qbuf = self.value(q)
        else:
            raise LoweringError(f"{step.name}: queries neither stored nor recomputed")
        if ATTN_SPLIT not in (64, 128):
            raise LoweringError(f"{step.name}: attention splits of {ATTN_SPLIT} positions; the kernel takes 64 or 128")
        # The positions a row may read: below the bound of its positions, or
        # of its reach; a ring without a window holds no more than its length.
        bound = self.p.source(op.to.positions).kind.bound
        if spec.reach is not None:
            bound = max(bound, self.p.source(spec.reach.source).kind.bound)
        positions = min(bound, span if spec.window is None else bound)
        entry, threads, lds = ("fk_step_attend_paged" if paged else "fk_step_attend"), ATTN_THREADS, 0
        split = ATTN_SPLIT
        if self.wide and not paged and spec.reach is None and spec.head_dim in (16, 32, 64):
            # Wide splits: 64 positions a wavefront, up to 8 wavefronts, so
            # that a head has at most 8 splits (the combine prologue's) up to
            # 4096 positions.
            waves = min(WIDE_MAX_WAVES, max(1, -(-positions // (WIDE_RUN * COMBINE_SPLITS))))
            split, entry, threads = WIDE_RUN * waves, "fk_step_attend_wide", 64 * waves
            lds = 4 * wide_lds_floats(waves)
        splits = -(-positions // split)
        if splits > 4096:
            raise LoweringError(f"{step.name}: {splits} splits")
        params["splits"], params["split"] = splits, split
        out = anchor.outputs[0]
        pname = self.out.buffer(f"partials:{self.p.value(out).name}", "f32",
                                spec.heads * splits * (spec.head_dim + 2))
        pos_buf = self.ints(op.to.positions)
        bind = {"q": qbuf, "knew": None, "vnew": None, "position": pos_buf, "rope": rope_buf or pos_buf,
                "partials": pname, "reach": None if spec.reach is None else self.ints(spec.reach.source)}
        if paged:
            bind.update(kpool=kname, vpool=vname, table=self.ints(op.to.sequences))
        else:
            bind.update(kc=kname, vc=vname, slot=self.ints(op.to.sequences))
        return Launch(step.name, entry, spec.kv_heads * splits, threads, bind, params, meta, lds)

    def combine_step(self, step: Step) -> Launch:
        combines = [self.p.node(w.node) for w in step.work if w.kind == COMBINE]
        others = [w for w in step.work if w.kind != COMBINE]
        if len(combines) != 1 or others:
            raise LoweringError(f"{step.name}: a combine step with other work")
        node = combines[0]
        spec = node.op.spec
        out = node.outputs[0]
        if [st.value for st in step.stores] != [out]:
            raise LoweringError(f"{step.name}: a combine that doesn't store its output alone")
        pname = f"partials:{self.p.value(out).name}"
        if pname not in self.out.buffers:
            raise LoweringError(f"{step.name}: combines partials no step stored")
        splits = self.out.buffers[pname].count // (spec.heads * (spec.head_dim + 2))
        if splits > 256:
            raise LoweringError(f"{step.name}: {splits} splits; the combine takes up to 256")
        params = {"heads": spec.heads, "head_dim": spec.head_dim, "splits": splits}
        return Launch(step.name, "fk_step_combine", spec.heads, 64,
                      {"partials": pname, "out": self.value(out)}, params)

    def norm_launch(self, step: Step, node) -> Launch:
        """An RMSNorm of one stored row as its own launch (fk_rmsnorm_f32, one
        row in segments, tgReduceSum's order over 256 threads)."""
        op = node.op
        shape = self.p.value(op.x).shape
        seg = shape.segment or shape.width
        if seg % 4 or shape.width % seg:
            raise LoweringError(f"{step.name}: an RMSNorm in segments of {seg} of a row of {shape.width}")
        gamma = None if op.gamma is None else self.gains(op.gamma)
        out = self.value(node.outputs[0])
        x = self.value(op.x)
        return Launch(f"{step.name}:{self.p.value(node.outputs[0]).name}", "fk_rmsnorm_f32", shape.width // seg, 256,
                      {"x": x, "gamma": gamma, "y": out},
                      {"rows": 1, "width": shape.width, "seg": seg, "eps": float(np.float32(op.eps)),
                       "factor": float(np.float32(op.factor)), "has_gamma": int(gamma is not None)},
                      {"value": node.outputs[0]})

    def table(self, s: int) -> tuple[str, STable]:
        """A table of weights: its entries in order in ``table:<name>``, their
        addresses in ``tableaddr:<name>`` (u64, the engine writes them)."""
        src = self.p.source(s)
        if not isinstance(src.kind, STable):
            raise LoweringError(f"{src.name} is not a table")
        t = src.kind.type
        if t not in (F16, BF16, F32):
            raise LoweringError(f"table {src.name} of {t}: the routed GEMV takes f16, bf16 and f32 entries")
        size = int(np.prod(src.kind.dims))
        pool = self.out.buffer(f"table:{src.name}", t, src.kind.entries * size)
        addr = self.out.buffer(f"tableaddr:{src.name}", "u64", src.kind.entries)
        self.out.constants[addr] = ("addresses", pool, size * (4 if t == F32 else 2))
        return addr, src.kind

    def routed_step(self, step: Step, anchors: list) -> list:
        """A step anchoring LinearRouted (Eval.hs:291-321): its route (if it
        recomputes it) by fk_step_route into the stored ids and weights, a
        gated activation of its input (if it recomputes one) by fk_step_act_mul
        into a row of its own, then the routed GEMV."""
        if len(anchors) != 1:
            raise LoweringError(f"{step.name}: {len(anchors)} routed anchors; the routed GEMV takes one")
        anchor = anchors[0]
        op = anchor.op
        launches = []
        for w in step.work:
            node = self.p.node(w.node)
            if w.kind == ANCHOR:
                continue
            if w.kind != RECOMPUTE:
                raise LoweringError(f"{step.name}: {w.kind} work beside a routed anchor")
            if isinstance(node.op, Route):
                launches.append(self.route_launch(step, node))
            elif isinstance(node.op, GatedGelu) and node.outputs[0] == op.x:
                launches.append(self.gated_launch(step, node))
            else:
                raise LoweringError(f"{step.name}: no routed step recomputes {type(node.op).__name__}")
        for L in launches:
            self.materialized |= set(L.meta["values"])
        if not self.stored_before(step, op.ids) or not self.stored_before(step, op.x):
            raise LoweringError(f"{step.name}: the routed GEMV's ids and input neither stored nor made")
        addr, tk = self.table(op.table)
        n, k = tk.dims
        ranks = self.p.value(op.ids).shape.width
        width = self.p.value(op.x).shape.width
        if width not in (k, ranks * k):
            raise LoweringError(f"{step.name}: an input of {width} for {ranks} ranks of {k}")
        out = anchor.outputs[0]
        if [st.value for st in step.stores if st.value not in self.materialized] != [out]:
            raise LoweringError(f"{step.name}: a routed step storing other than its anchor's rows")
        r = 2 if tk.type in (F16, BF16) and n >= 2048 else 1
        entry = f"fk_gemv_routed_{tk.type}_r{r}"
        per_group = 4 * r  # 256 threads
        gpr = -(-n // per_group)
        params = {"n": n, "k": k, "ranks": ranks, "shared": int(width == k), "entries": tk.entries,
                  "groups_per_rank": gpr}
        bind = {"table": addr, "ids": self.value(op.ids), "x": self.value(op.x), "y": self.value(out)}
        launches.append(Launch(step.name, entry, ranks * gpr, 256, bind, params))
        return launches

    def route_launch(self, step: Step, node) -> Launch:
        op = node.op
        ids, ws = node.outputs
        n = self.p.value(op.x).shape.width
        if not self.stored_before(step, op.x):
            raise LoweringError(f"{step.name}: a route of logits not stored")
        scale = None if op.spec.expert_scale is None else self.gains(op.spec.expert_scale)
        x = self.value(op.x)
        return Launch(f"{step.name}:route", "fk_step_route", 1, 64,
                      {"x": x, "scale": scale or x, "ids": self.value(ids), "ws": self.value(ws)},
                      {"n": n, "k": op.spec.k, "has_scale": int(scale is not None)}, {"values": [ids, ws]})

    def gated_launch(self, step: Step, node) -> Launch:
        op = node.op
        if op.form not in ACT or not self.stored_before(step, op.x):
            raise LoweringError(f"{step.name}: a gated activation of a row not stored")
        shape = self.p.value(op.x).shape
        half = shape.segment // 2
        n = shape.width // 2
        x = self.value(op.x)
        return Launch(f"{step.name}:{self.p.value(node.outputs[0]).name}", "fk_step_act_mul", -(-n // THREADS),
                      THREADS, {"a": x, "b": x, "y": self.value(node.outputs[0])},
                      {"n": n, "act": ACT[op.form], "b_off": 0, "half": half}, {"values": [node.outputs[0]]})

    def light_step(self, step: Step) -> Launch:
        rec = [self.p.node(w.node) for w in step.work if w.kind == RECOMPUTE]
        comb = [r for r in rec if isinstance(r.op, CombineRanks)]
        if comb and len(rec) <= 2:
            return self.combine_ranks_step(step, rec, comb[0])
        rec = [self.p.node(w.node) for w in step.work if w.kind == RECOMPUTE]
        if len(rec) != 1 or len(step.stores) != 1 or step.stores[0].value != rec[0].outputs[0]:
            raise LoweringError(f"{step.name}: a light step other than one stored recompute")
        node = rec[0]
        op = node.op
        if isinstance(op, ArgMax) and self.stored_before(step, op.x):
            n = self.p.value(op.x).shape.width
            return Launch(step.name, "fk_step_argmax", 1, 1024,
                          {"x": self.value(op.x), "out": self.value(node.outputs[0])}, {"n": n})
        if isinstance(op, GeluMul) and op.form in ACT and self.stored_before(step, op.a) and \
                self.stored_before(step, op.b):
            n = self.p.value(op.a).shape.width
            return Launch(step.name, "fk_step_act_mul", -(-n // THREADS), THREADS,
                          {"a": self.value(op.a), "b": self.value(op.b), "y": self.value(node.outputs[0])},
                          {"n": n, "act": ACT[op.form], "b_off": 0})
        if isinstance(op, GatedGelu) and op.form in ACT and self.stored_before(step, op.x):
            shape = self.p.value(op.x).shape
            if shape.segment != shape.width:
                raise LoweringError(f"{step.name}: a gated activation in segments of {shape.segment} of a row of "
                                    f"{shape.width}")
            n = shape.width // 2
            x = self.value(op.x)
            return Launch(step.name, "fk_step_act_mul", -(-n // THREADS), THREADS,
                          {"a": x, "b": x, "y": self.value(node.outputs[0])},
                          {"n": n, "act": ACT[op.form], "b_off": n})
        if isinstance(op, Softcap) and self.stored_before(step, op.x):
            n = self.p.value(op.x).shape.width
            cap = float(np.float32(op.cap))
            if not 0 < cap < math.inf:
                raise LoweringError(f"{step.name}: a softcap of {op.cap}")
            return Launch(step.name, "fk_prefill_softcap", max(1, -(-n // 256)), 256,
                          {"x": self.value(op.x), "y": self.value(node.outputs[0])}, {"count": n, "cap": cap})
        raise LoweringError(f"{step.name}: no light kernel recomputes {type(op).__name__}")

    def combine_ranks_step(self, step: Step, rec: list, comb) -> Launch:
        """CombineRanks of stored weights and rows, and the residual add of it
        (if the step recomputes one), into the stored value."""
        op = comb.op
        if not self.stored_before(step, op.weights) or not self.stored_before(step, op.x):
            raise LoweringError(f"{step.name}: a combine of ranks not stored")
        res, out = None, comb.outputs[0]
        adds = [r for r in rec if r is not comb]
        if adds:
            a = adds[0].op
            if not isinstance(a, Add) or comb.outputs[0] not in (a.a, a.b):
                raise LoweringError(f"{step.name}: a combine of ranks with {type(a).__name__}")
            other = a.b if a.a == comb.outputs[0] else a.a
            if not self.stored_before(step, other):
                raise LoweringError(f"{step.name}: a residual not stored")
            res, out = self.value(other), adds[0].outputs[0]
        if [st.value for st in step.stores] != [out]:
            raise LoweringError(f"{step.name}: a combine of ranks storing other than its value")
        seg = self.p.value(op.x).shape.segment
        ranks = self.p.value(op.weights).shape.width
        x = self.value(op.x)
        return Launch(step.name, "fk_step_combine_ranks", -(-seg // THREADS), THREADS,
                      {"w": self.value(op.weights), "x": x, "res": res or x, "y": self.value(out)},
                      {"seg": seg, "ranks": ranks, "residual": int(res is not None)})
