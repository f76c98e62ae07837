"""A plan's steps, for a step of many rows (the prefill of one or more
sequences), as launches of the prefill kernels: the tile-layout GEMM
(fk_gemm.h) for the Linear anchors and the kernels of fk_prefill.h around it.

The decode lowering (lower.py) turns each step into one launch that works on
one row; here a step of M rows is a few launches, and values live in one of
two layouts: f32 rows (``value:`` buffers: the residual stream, q/k/v, the
logits) or f16 in the tile layout (``tiled:`` buffers: what feeds the matrix
cores).  Each value is made in the layout its readers take:

- a Linear step's input is its RMSNorm (recomputed in the plan) packed to
  f16 tiles by ``fk_prefill_norm_pack``, or a value already tiled;
- two anchors whose only reader is one SiLU·mul (gate, up) run as one paired
  GEMM whose epilogue writes the product tiled — the down projection's input;
- a residual add epilogue is the GEMM's add mode, into f32 rows;
- KV stores are held until the attention of the same caches, which runs as
  ``fk_prefill_rope_store`` (q RoPE'd to f16 rows, k RoPE'd and v into the
  caches) then ``fk_prefill_attend`` (tiled output: the o projection's input);
  when the three came from one GEMM and every pair of the heads turns, the
  GEMM's epilogue does the RoPE and the stores (``fk_gemm_f16_qkv_rope``) and
  q, k, v are never f32 rows in HBM;
- the greedy token is ``fk_prefill_argmax`` over each row's logits, or,
  when the head's GEMM stored them, keys that GEMM leaves (128 columns a
  key) reduced by ``fk_prefill_argmax_keys``.

Staged KV stores (the ring has no room for a step's rows: Plan.hs:41-50)
store each row's k and v heads, as the cache holds them, into staging rows
(``staged:`` buffers, [rows][kv_heads][64]) instead of the ring; the
attention reads a sequence's positions from its run's first row on from
there and the rest from the ring; and the step that lands them copies them
into the ring (``fk_prefill_land``).  A staged step's rows come in runs of
``run_rows`` rows, each one sequence's consecutive positions.

Steps of other shapes (a gathered Linear input, segments narrower than the
row) are refused with ``LoweringError``.  Pure host logic:
the lowering a ``Backend Rocm`` does for a step of many rows
(src/FuryKernel/Backend.hs:29-101, src/FuryKernel/Program/Plan.hs:270-300 for
the sequence rows of a step).
"""

from __future__ import annotations

from collections import defaultdict
from typing import Optional

import numpy as np

from .kernels import ATTEND_KEYS, NORM_PACK_HELD
from .layout import SLAB, pack, pair
from .lower import ACT, Launch, Lowered, LoweringError, rope_table
from .program.check import CheckedProgram
from .program.graph import (
    CACHE_BF16, F16, F32, GELU_TANH, SILU, U32, Add, ArgMax, Attend, Gather, GeluMul, Input, KvStore, Linear, Paged, Ring,
    RmsNorm, Softcap,
    Rope, ROPE_HALVES, SCache, SInput, SRowInts, SWeight, op_values)
from .program.plan import ANCHOR, COMBINE, EFFECT, EPILOGUE, LAND, RECOMPUTE, STAGE, Plan, Step

GEMM_K = 64                        # the GEMM's K granule
GEMM_LDS = 4 * 2 * 256 * 32 * 2    # its LDS ring
QBLOCK = 32                        # rows an attention threadgroup takes
HEAD_DIM = 64                      # the attention kernel's head dimension


def lower_prefill(checked: CheckedProgram, plan: Plan, rows: int, run_rows: Optional[int] = None,
                  scratch_slot: bool = False) -> Lowered:
    """The launches of every step of the plan for a step of `rows` rows (a
    multiple of 256: the sequences' rows one after another, each sequence's
    run a multiple of 32 rows; `run_rows` rows each where the plan stages
    KV stores, the plan's sequence rows).  With `scratch_slot`, each ring
    holds one slot more (and each paged pool one block more) past the
    program's: rows that only fill a step out to its tiles store there, so
    that a step's real rows may be any number (``PrefillSession``,
    ``DecodeRows``)."""
    if rows <= 0 or rows % SLAB:
        raise LoweringError(f"a step of {rows} rows; the prefill kernels take multiples of {SLAB}")
    run_rows = rows if run_rows is None else run_rows
    if run_rows <= 0 or run_rows % QBLOCK or rows % run_rows:
        raise LoweringError(f"runs of {run_rows} rows in a step of {rows}: multiples of {QBLOCK} that divide it")
    out = Lowered(checked.program, plan, rows)
    _Prefill(out, run_rows, scratch_slot).run()
    _fuse_qkv_rope(out)
    _fuse_argmax(out)
    return out


def _fuse_argmax(out: Lowered) -> None:
    """Folds each ``fk_prefill_argmax`` over rows that a one-anchor
    ``fk_gemm_f16_store`` made (the head's logits, no softcap between) into
    that GEMM: ``fk_gemm_f16_store_keys`` stores the same rows and leaves
    each row's greedy-token keys, 128 columns a key, and
    ``fk_prefill_argmax_keys`` takes their maximum, the same token as the
    argmax over the rows.  No launch between the two may touch the rows."""
    launches = out.launches
    for i, am in enumerate(launches):
        if am.entry != "fk_prefill_argmax":
            continue
        x = am.bind["x"]
        j = next((j for j in range(i - 1, -1, -1) if x in launches[j].bind.values()), None)
        if j is None:
            continue
        gm = launches[j]
        p = gm.params
        if gm.entry != "fk_gemm_f16_store" or gm.bind["c0"] != x or p["n_anchors"] != 1 or \
                p["first_col"][0] != 0 or p["ldc"][0] != p["first_col"][1] or p["ldc"][0] != am.params["width"]:
            continue
        rows, parts = am.params["rows"], p["ldc"][0] // 128
        keys = out.buffer(f"keys:{x}", "u64", rows * parts)
        launches[j] = Launch(gm.step, "fk_gemm_f16_store_keys", gm.groups, gm.threads, dict(gm.bind, keys=keys),
                             dict(p), {}, gm.lds_bytes)
        launches[i] = Launch(am.step, "fk_prefill_argmax_keys", am.groups, am.threads,
                             {"keys": keys, "out": am.bind["out"]}, {"rows": rows, "parts": parts}, {},
                             am.lds_bytes)


def _fuse_qkv_rope(out: Lowered) -> None:
    """Folds each ``fk_prefill_rope_store`` into the GEMM that made its q, k
    and v (its three anchors, in that order) when the RoPE turns every pair
    of the heads of 64: the GEMM's epilogue then RoPEs q into the attention's
    f16 rows and k into the K cache and stores v, with the same arithmetic,
    and the f32 rows of q, k, v go.  Nothing between the GEMM and the RoPE
    launch may touch what either writes or reads."""
    launches = out.launches
    i = 0
    while i < len(launches):
        rs = launches[i]
        if rs.entry not in ("fk_prefill_rope_store", "fk_prefill_rope_store_paged") or \
                rs.params["rotated"] != HEAD_DIM // 2 or rs.params["head_dim"] != HEAD_DIM:
            i += 1
            continue
        qkv = (rs.bind["q"], rs.bind["k"], rs.bind["v"])
        j = next((j for j in range(i - 1, -1, -1) if set(qkv) & set(launches[j].bind.values())), None)
        gm = launches[j] if j is not None else None
        if gm is None or gm.entry != "fk_gemm_f16_store" or gm.params["n_anchors"] != 3 or \
                (gm.bind["c0"], gm.bind["c1"], gm.bind["c2"]) != qkv:
            i += 1
            continue
        touched = set(qkv) | {rs.bind[b] for b in ("qr", "kc", "vc")}
        between = any(touched & set(launches[t].bind.values()) for t in range(j + 1, i))
        elsewhere = any(set(qkv) & set(l.bind.values()) for t, l in enumerate(launches) if t not in (i, j))
        if between or elsewhere or any(f"value:{out.program.value(o.value).name}" in qkv
                                       for o in out.program.outputs):
            i += 1
            continue
        p = rs.params
        paging = {f: p[f] for f in ("block_size", "table_len", "blocks")} if rs.entry.endswith("_paged") else None
        bind = dict(gm.bind, c0=rs.bind["qr"], c1=rs.bind["kc"], c2=rs.bind["vc"], position=rs.bind["position"],
                    rope=rs.bind["rope"], **({"table": rs.bind["table"]} if paging else {"slot": rs.bind["slot"]}))
        params = dict(gm.params, kv_heads=p["kv_heads"], rope_rows=p["rope_rows"], length=p["length"],
                      slots=p["slots"], cache_bf16=p["cache_bf16"], staged=p["staged"], **(paging or {}))
        launches[j] = Launch(gm.step, "fk_gemm_f16_qkv_rope_paged" if paging else "fk_gemm_f16_qkv_rope",
                             gm.groups, gm.threads, bind, params, {}, gm.lds_bytes)
        del launches[i]
        for name in qkv:
            del out.buffers[name]


class _Prefill:
    def __init__(self, out: Lowered, run_rows: int, scratch: bool = False):
        self.out = out
        self.run_rows = run_rows
        self.scratch = int(scratch)  # a ring's slots (a pool's blocks) one past the program's
        self.staged: set = set()   # KvStore nodes the plan stages
        self.landing: dict = {}    # KvStore node id -> (staging buffer, ring buffer)
        self.p = out.program
        self.rows = out.rows
        self.producer = {v: n for n in self.p.nodes for v in n.outputs}
        self.readers = defaultdict(list)
        for n in self.p.nodes:
            for v in op_values(n.op):
                self.readers[v].append(n)
        self.rows_of: dict = {}    # value -> its f32 rows buffer
        self.tiled_of: dict = {}   # value -> its f16 tile-layout buffer
        self.pending: list = []    # KvStore nodes waiting for their attention
        for n in self.p.nodes:
            if isinstance(n.op, Input):
                src = self.p.source(n.op.source)
                if not isinstance(src.kind, SInput) or src.kind.type != F32:
                    raise LoweringError(f"input {src.name}: the prefill kernels read f32 rows")
                self.rows_of[n.outputs[0]] = self.value_rows(n.outputs[0])

    def run(self) -> None:
        for step in self.out.plan.steps:
            self.step(step)
        if self.pending:
            raise LoweringError(f"KV stores {[n.name for n in self.pending]} with no attention after them")
        if self.landing:
            raise LoweringError(f"staged KV stores {sorted(self.landing)} never landed")
        for o in self.p.outputs:
            if o.value not in self.rows_of:
                raise LoweringError(f"output {o.name} is never made as rows")

    # Buffers -------------------------------------------------------------------

    def width(self, v: int) -> int:
        return self.p.value(v).shape.width

    def value_rows(self, v: int) -> str:
        val = self.p.value(v)
        return self.out.buffer(f"value:{val.name}", "u32" if val.type == U32 else "f32", val.shape.width * self.rows)

    def value_tiled(self, v: int) -> str:
        val = self.p.value(v)
        if val.shape.width % 32:
            raise LoweringError(f"{val.name}: rows of {val.shape.width} do not tile (multiples of 32)")
        return self.out.buffer(f"tiled:{val.name}", "f16", val.shape.width * self.rows)

    def weight_source(self, s: int) -> tuple:
        src = self.p.source(s)
        if not isinstance(src.kind, SWeight):
            raise LoweringError(f"{src.name} is not a weight")
        return src, src.kind.type, tuple(src.kind.dims)

    def weight_plain(self, s: int) -> tuple[str, str]:
        src, t, dims = self.weight_source(s)
        name = self.out.buffer(f"weight:{src.name}", t, int(np.prod(dims)))
        self.out.layouts[name] = ("plain", (src.name,))
        return name, t

    def weight_tiled(self, s: int, unit: int = SLAB) -> tuple[str, int, int]:
        src, t, dims = self.weight_source(s)
        if t != F16 or len(dims) != 2 or dims[0] % unit or dims[1] % GEMM_K:
            raise LoweringError(f"weight {src.name} {t}{list(dims)}: the GEMM takes f16 [n, k], n a multiple of "
                                f"{unit}, k of {GEMM_K}")
        name = self.out.buffer(f"tiled:{src.name}", "f16", dims[0] * dims[1])
        self.out.layouts[name] = ("tiled", (src.name,))
        return name, dims[0], dims[1]

    def ints(self, s: int) -> str:
        src = self.p.source(s)
        if not isinstance(src.kind, SRowInts) or src.kind.count != 1:
            raise LoweringError(f"{src.name}: the prefill kernels take one integer a row")
        return self.out.buffer(f"ints:{src.name}", "u32", self.rows)

    def tables(self, s: int) -> tuple[str, int]:
        """The rows' block tables, [rows][table length] u32."""
        src = self.p.source(s)
        if not isinstance(src.kind, SRowInts):
            raise LoweringError(f"{src.name}: block tables are row integers")
        return self.out.buffer(f"ints:{src.name}", "u32", self.rows * src.kind.count), src.kind.count

    def cache(self, s: int) -> tuple[str, object, bool]:
        """A ring's or a paged pool's buffer ([slots][kv heads][length][d] or
        [blocks][kv heads][block size][d]), its layout, whether bf16."""
        src = self.p.source(s)
        if not isinstance(src.kind, SCache) or not isinstance(src.kind.layout, (Ring, Paged)):
            raise LoweringError(f"{src.name}: the prefill attention takes ring caches and paged pools")
        lay = src.kind.layout
        bf16 = src.kind.elem == CACHE_BF16
        if isinstance(lay, Ring):
            count = (lay.slots + self.scratch) * lay.kv_heads * lay.length * lay.head_dim
        else:
            count = (lay.blocks + self.scratch) * lay.kv_heads * lay.block_size * lay.head_dim
        return self.out.buffer(f"cache:{src.name}", "bf16" if bf16 else "f16", count), lay, bf16

    def rope(self, spec, d: int, rows: int) -> str:
        name = f"rope:{spec.theta!r}:{d}:{spec.rotated}:{rows}"
        self.out.buffer(name, "f32", rows * spec.rotated * 2)
        self.out.constants[name] = ("rope", float(spec.theta), d, spec.rotated, rows)
        return name

    def launch(self, step: Step, entry: str, groups: int, threads: int, bind: dict, params: dict,
               lds: int = 0) -> None:
        self.out.launches.append(Launch(step.name, entry, groups, threads, bind, params, {}, lds))

    # Values in their layouts -------------------------------------------------------

    def rows_value(self, step: Step, v: int) -> str:
        """v's f32 rows, gathering them the first time when v is an embedding."""
        got = self.rows_of.get(v)
        if got is not None:
            return got
        node = self.producer.get(v)
        if node is None or not isinstance(node.op, Gather):
            raise LoweringError(f"{step.name}: {self.p.value(v).name} is not made as rows before this step")
        table, t, dims = self.weight_source(node.op.table)
        tname, ttype = self.weight_plain(node.op.table)
        if ttype not in (F16, F32) or dims[1] != self.width(v) or dims[1] % 4:
            raise LoweringError(f"{step.name}: a gather from {table.name} {ttype}{list(dims)}")
        buf = self.value_rows(v)
        self.launch(step, "fk_prefill_gather", self.rows // 4, 256,
                    {"table": tname, "tokens": self.ints(node.op.tokens), "x": buf},
                    {"rows": self.rows, "width": dims[1], "table_rows": dims[0], "table_f16": int(ttype == F16),
                     "factor": float(np.float32(node.op.factor))})
        self.rows_of[v] = buf
        return buf

    def tiled_input(self, step: Step, x: int, rec: dict) -> str:
        """The GEMM's A: x tiled, made here from x's RMSNorm when the plan
        recomputes it."""
        got = self.tiled_of.get(x)
        if got is not None:
            return got
        node = rec.get(x)
        if node is None or not isinstance(node.op, RmsNorm):
            raise LoweringError(f"{step.name}: the anchors' input {self.p.value(x).name} is neither tiled nor an "
                                f"RMSNorm this step makes")
        op = node.op
        width = self.width(op.x)
        if self.p.value(op.x).shape.segment != width:
            raise LoweringError(f"{step.name}: an RMSNorm in segments narrower than the row")
        src = self.rows_value(step, op.x)
        bind = {"x": src, "gamma": None, "y": self.value_tiled(x)}
        if op.gamma is not None:
            gname, gt = self.weight_plain(op.gamma)
            if gt != F32:
                raise LoweringError(f"{step.name}: a gamma of {gt}; the kernels read f32 gammas")
            bind["gamma"] = gname
        entry = f"fk_prefill_norm_pack_w{width}" if width in NORM_PACK_HELD else "fk_prefill_norm_pack"
        self.launch(step, entry, self.rows // 4, 256, bind,
                    {"rows": self.rows, "width": width, "eps": float(np.float32(op.eps)),
                     "factor": float(np.float32(op.factor)), "has_gamma": int(op.gamma is not None)})
        self.tiled_of[x] = bind["y"]
        return bind["y"]

    # Steps -------------------------------------------------------------------------

    def step(self, step: Step) -> None:
        kinds = {w.kind for w in step.work}
        anchors = [self.p.node(w.node) for w in step.work if w.kind == ANCHOR]
        if anchors and all(isinstance(a.op, Linear) for a in anchors):
            return self.linear_step(step, anchors)
        if len(anchors) == 1 and isinstance(anchors[0].op, Attend):
            return self.attend_step(step, anchors[0])
        if anchors:
            raise LoweringError(f"{step.name}: anchors of mixed or unknown kinds")
        if EFFECT in kinds or STAGE in kinds:
            return self.store_step(step)
        if COMBINE in kinds or LAND in kinds:
            return self.combine_step(step)
        return self.light_step(step)

    def recomputes(self, step: Step) -> dict:
        return {self.p.node(w.node).outputs[0]: self.p.node(w.node) for w in step.work if w.kind == RECOMPUTE}

    def silu_pair(self, outs: list) -> Optional[tuple]:
        """The SiLU·mul node two anchor outputs feed, and nothing else does:
        (node, gate index, up index)."""
        if len(outs) != 2:
            return None
        readers = {n.id: n for v in outs for n in self.readers[v]}
        if len(readers) != 1:
            return None
        node = next(iter(readers.values()))
        if not (isinstance(node.op, GeluMul) and node.op.form in ACT and {node.op.a, node.op.b} == set(outs)):
            return None
        if any(o.value in outs for o in self.p.outputs):
            return None
        return node, outs.index(node.op.a), outs.index(node.op.b)

    def linear_step(self, step: Step, anchors: list) -> None:
        if len(anchors) > 3:
            raise LoweringError(f"{step.name}: {len(anchors)} anchors; the GEMM takes up to 3")
        xs = {a.op.x for a in anchors}
        if len(xs) != 1:
            raise LoweringError(f"{step.name}: anchors of different inputs")
        x = xs.pop()
        rec = self.recomputes(step)
        k = self.width(x)
        if k % GEMM_K:
            raise LoweringError(f"{step.name}: an input row of {k}, not a multiple of {GEMM_K}")
        a_buf = self.tiled_input(step, x, rec)
        outs = [a.outputs[0] for a in anchors]
        bind = {"a": a_buf, "b0": None, "b1": None, "b2": None, "c0": None, "c1": None, "c2": None, "r0": None}
        m = self.rows
        epis = [self.p.node(w.node) for w in step.work if w.kind == EPILOGUE]

        sp = self.silu_pair(outs)
        if sp is not None and not epis:
            node, gi, ui = sp
            gsrc, gt, gdims = self.weight_source(anchors[gi].op.weight)
            usrc, ut, udims = self.weight_source(anchors[ui].op.weight)
            if gt != F16 or ut != F16 or gdims != udims or gdims[0] % (SLAB // 2) or gdims[1] != k:
                raise LoweringError(f"{step.name}: gate {gsrc.name} and up {usrc.name} do not pair")
            n = gdims[0]
            pname = self.out.buffer(f"pair:{gsrc.name}|{usrc.name}", "f16", 2 * n * k)
            self.out.layouts[pname] = ("pair", (gsrc.name, usrc.name))
            act = node.outputs[0]
            bind.update(b0=pname, c0=self.value_tiled(act))
            self.tiled_of[act] = bind["c0"]
            self.launch(step, "fk_gemm_f16_silu_mul", (m // SLAB) * (n // (SLAB // 2)), 256, bind,
                        {"m": m, "k": k, "n_anchors": 1, "first_col": [0, n, n, n], "ldc": [n, 0, 0],
                         "act": ACT[node.op.form]}, GEMM_LDS)
            return

        rows, first = [], [0]
        for j, a in enumerate(anchors):
            wname, n, kk = self.weight_tiled(a.op.weight)
            if kk != k or n != self.width(a.outputs[0]):
                raise LoweringError(f"{step.name}: weight of {a.name} is [{n}, {kk}] for a row of {k}")
            bind[f"b{j}"] = wname
            rows.append(n)
            first.append(first[-1] + n)
        first += [first[-1]] * (4 - len(first))
        params = {"m": m, "k": k, "n_anchors": len(anchors), "first_col": first, "ldc": (rows + [0, 0, 0])[:3]}
        groups = (m // SLAB) * (sum(rows) // SLAB)
        if len(epis) == 1 and len(anchors) == 1 and isinstance(epis[0].op, Softcap) and epis[0].op.x == outs[0]:
            # The tile stored as rows, then the softcap over them into the
            # capped value's rows.
            cap = float(np.float32(epis[0].op.cap))
            if not 0 < cap < float("inf"):
                raise LoweringError(f"{step.name}: a softcap of {epis[0].op.cap}")
            bind["c0"] = self.value_rows(outs[0])
            self.rows_of[outs[0]] = bind["c0"]
            self.launch(step, "fk_gemm_f16_store", groups, 256, bind, params, GEMM_LDS)
            capped = epis[0].outputs[0]
            count = self.rows * rows[0]
            self.launch(step, "fk_prefill_softcap", min(max(1, count // 1024), 4096), 256,
                        {"x": bind["c0"], "y": self.value_rows(capped)}, {"count": count, "cap": cap})
            self.rows_of[capped] = self.value_rows(capped)
            return
        if epis:
            if len(epis) != 1 or len(anchors) != 1 or not isinstance(epis[0].op, Add):
                raise LoweringError(f"{step.name}: epilogues other than one residual add or softcap on one anchor")
            op = epis[0].op
            tile = outs[0]
            if tile not in (op.a, op.b):
                raise LoweringError(f"{step.name}: an epilogue off its anchor's tile")
            other = op.b if op.a == tile else op.a
            bind["r0"] = self.rows_value(step, other)
            bind["c0"] = self.value_rows(epis[0].outputs[0])
            self.rows_of[epis[0].outputs[0]] = bind["c0"]
            self.launch(step, "fk_gemm_f16_add", groups, 256, bind, params, GEMM_LDS)
            return
        for j, v in enumerate(outs):
            bind[f"c{j}"] = self.value_rows(v)
            self.rows_of[v] = bind[f"c{j}"]
        self.launch(step, "fk_gemm_f16_store", groups, 256, bind, params, GEMM_LDS)

    def store_step(self, step: Step) -> None:
        for w in step.work:
            node = self.p.node(w.node)
            if w.kind in (EFFECT, STAGE):
                if not isinstance(node.op, KvStore):
                    raise LoweringError(f"{step.name}: an effect other than a KV store")
                self.pending.append(node)
                if w.kind == STAGE:
                    self.staged.add(node.id)
            elif w.kind != RECOMPUTE or not isinstance(node.op, Rope):
                raise LoweringError(f"{step.name}: {w.kind} {node.name} in a store step")

    def roped(self, step: Step, v: int) -> tuple[int, object]:
        """(the value RoPE turns, its Rope op), for v made by a Rope."""
        node = self.producer.get(v)
        if node is None or not isinstance(node.op, Rope):
            raise LoweringError(f"{step.name}: {self.p.value(v).name} is not RoPE'd; the prefill attention "
                                f"takes RoPE'd queries and keys")
        return node.op.x, node.op

    def attend_step(self, step: Step, anchor) -> None:
        op = anchor.op
        spec = op.spec
        if spec.reach is not None:
            raise LoweringError(f"{step.name}: attention with a reach")
        if spec.head_dim != HEAD_DIM or spec.heads % spec.kv_heads or spec.heads // spec.kv_heads not in (1, 2, 4):
            raise LoweringError(f"{step.name}: {spec.heads} heads over {spec.kv_heads} of {spec.head_dim}; the "
                                f"prefill attention takes heads of {HEAD_DIM}, 1, 2 or 4 a kv head")
        kname, klay, kbf = self.cache(op.to.keys)
        vname, vlay, vbf = self.cache(op.to.values)
        if klay != vlay or kbf != vbf or klay.kv_heads != spec.kv_heads or klay.head_dim != HEAD_DIM:
            raise LoweringError(f"{step.name}: key and value caches of different layouts")
        paged = isinstance(klay, Paged)
        if paged:
            table, table_len = self.tables(op.to.sequences)
            length = table_len * klay.block_size   # the positions a row's table covers
            paging = {"block_size": klay.block_size, "table_len": table_len, "blocks": klay.blocks + self.scratch}
        else:
            length, paging = klay.length, None
            if klay.length % ATTEND_KEYS:
                raise LoweringError(f"{step.name}: a ring of {klay.length}; the prefill attention reads keys by "
                                    f"blocks of {ATTEND_KEYS} that must not wrap")
        stores = {}
        for n in self.pending:
            at = n.op.at
            if at.cache in (op.to.keys, op.to.values):
                if (at.positions, at.sequences) != (op.to.positions, op.to.sequences):
                    raise LoweringError(f"{step.name}: a store at other positions than the attention reads")
                stores[at.cache] = n
        if set(stores) != {op.to.keys, op.to.values} or len(self.pending) != 2:
            raise LoweringError(f"{step.name}: the attention's key and value stores are not the steps before it")
        self.pending = []
        staged = {stores[c].id in self.staged for c in stores}
        if len(staged) != 1:
            raise LoweringError(f"{step.name}: one of the attention's stores staged, the other not")
        staged = staged.pop()
        if staged and paged:
            raise LoweringError(f"{step.name}: staged stores into paged pools")
        k_raw, k_rope = self.roped(step, stores[op.to.keys].op.x)
        q_raw, q_rope = self.roped(step, op.q)
        v_raw = stores[op.to.values].op.x
        if q_rope.spec != k_rope.spec or q_rope.positions != op.to.positions or k_rope.positions != op.to.positions:
            raise LoweringError(f"{step.name}: q and k RoPE'd differently")
        rs = q_rope.spec
        if rs.axes != 1 or rs.pairs != ROPE_HALVES or 2 * rs.rotated > HEAD_DIM:
            raise LoweringError(f"{step.name}: RoPE other than NeoX halves on one axis")
        heads, kvh = spec.heads, spec.kv_heads
        if self.width(q_raw) != heads * HEAD_DIM or self.width(k_raw) != kvh * HEAD_DIM or \
                self.width(v_raw) != kvh * HEAD_DIM:
            raise LoweringError(f"{step.name}: q, k, v rows of other widths than the heads'")
        pos = self.ints(op.to.positions)
        seq = table if paged else self.ints(op.to.sequences)
        qr = self.out.buffer(f"qrot:{self.p.value(op.q).name}", "f16", heads * HEAD_DIM * self.rows)
        ks = vs = None
        if staged:
            elem = "bf16" if kbf else "f16"
            ks = self.out.buffer(f"staged:{kname[len('cache:'):]}", elem, self.rows * kvh * HEAD_DIM)
            vs = self.out.buffer(f"staged:{vname[len('cache:'):]}", elem, self.rows * kvh * HEAD_DIM)
            self.landing[stores[op.to.keys].id] = (ks, kname)
            self.landing[stores[op.to.values].id] = (vs, vname)
        self.launch(step, "fk_prefill_rope_store_paged" if paged else "fk_prefill_rope_store", self.rows, 256,
                    {"q": self.rows_value(step, q_raw), "k": self.rows_value(step, k_raw),
                     "v": self.rows_value(step, v_raw), "position": pos, "table" if paged else "slot": seq,
                     "rope": self.rope(rs, HEAD_DIM, length), "qr": qr, "kc": ks or kname, "vc": vs or vname},
                    dict({"rows": self.rows, "heads": heads, "kv_heads": kvh, "head_dim": HEAD_DIM,
                          "rotated": rs.rotated, "rope_rows": length, "length": length,
                          "slots": 0 if paged else klay.slots + self.scratch, "cache_bf16": int(kbf),
                          "staged": int(staged)},
                         **(paging or {})))
        outv = anchor.outputs[0]
        obuf = self.value_tiled(outv)
        self.tiled_of[outv] = obuf
        g = heads // kvh
        params = {"rows": self.rows, "heads": heads, "kv_heads": kvh, "length": length,
                  "slots": 0 if paged else klay.slots + self.scratch, "window": spec.window or 0,
                  "cache_bf16": int(kbf),
                  "scale": float(np.float32(spec.scale)), "staged": int(staged), "run_rows": self.run_rows}
        if paged:
            # f16 pools under 4 GiB with tables of at most 256 blocks: each
            # block's rows straight into LDS
            pool_bytes = paging["blocks"] * kvh * paging["block_size"] * HEAD_DIM * 2
            direct = not kbf and paging["table_len"] <= 256 and pool_bytes < 1 << 32
            form = "fk_prefill_attend_paged_f16_g" if direct else "fk_prefill_attend_paged_g"
            self.launch(step, f"{form}{g}", (self.rows // QBLOCK) * kvh, 64 * g,
                        {"qr": qr, "kc": kname, "vc": vname, "position": pos, "table": seq, "out": obuf},
                        dict(params, **paging))
        else:
            # f16 rings without staged rows: each block's rows straight into LDS
            form = "fk_prefill_attend_g" if kbf or staged else "fk_prefill_attend_f16_g"
            self.launch(step, f"{form}{g}", (self.rows // QBLOCK) * kvh, 64 * g,
                        {"qr": qr, "kc": kname, "vc": vname, "position": pos, "slot": seq, "out": obuf,
                         "ks": ks, "vs": vs}, params)

    def combine_step(self, step: Step) -> None:
        # The prefill attention finishes its rows in one launch: nothing to
        # combine; staged stores land here, after the last attention reading
        # the ring (Plan.hs:41-50).
        lands = []
        for w in step.work:
            node = self.p.node(w.node)
            if w.kind == LAND and isinstance(node.op, KvStore) and node.id in self.landing:
                lands.append(node)
            elif w.kind != COMBINE or not isinstance(node.op, Attend) or node.outputs[0] not in self.tiled_of:
                raise LoweringError(f"{step.name}: {w.kind} {node.name} in a combine step")
        if not lands:
            return
        if len(lands) != 2 or lands[0].op.at.positions != lands[1].op.at.positions or \
                lands[0].op.at.sequences != lands[1].op.at.sequences:
            raise LoweringError(f"{step.name}: lands of other than one key and value pair")
        (ks, kname), (vs, vname) = (self.landing.pop(n.id) for n in lands)
        _, lay, _ = self.cache(lands[0].op.at.cache)
        self.launch(step, "fk_prefill_land", self.rows, 256,
                    {"ks": ks, "vs": vs, "position": self.ints(lands[0].op.at.positions),
                     "slot": self.ints(lands[0].op.at.sequences), "kc": kname, "vc": vname},
                    {"rows": self.rows, "kv_heads": lay.kv_heads, "head_dim": lay.head_dim, "length": lay.length,
                     "slots": lay.slots + self.scratch})

    def light_step(self, step: Step) -> None:
        rec = self.recomputes(step)
        for v, node in rec.items():
            if isinstance(node.op, ArgMax):
                width = self.width(node.op.x)
                self.launch(step, "fk_prefill_argmax", self.rows // 4, 256,
                            {"x": self.rows_value(step, node.op.x), "out": self.value_rows(v)},
                            {"rows": self.rows, "width": width})
                self.rows_of[v] = self.value_rows(v)
            else:
                raise LoweringError(f"{step.name}: a light step of {type(node.op).__name__}")


# Weights and rows ---------------------------------------------------------------------


def weight_image(lowered: Lowered, name: str, weights: dict) -> np.ndarray:
    """The contents of weight buffer `name` from the host weights (source
    name -> array): as given, tiled, or the gate/up pair tiled."""
    kind, srcs = lowered.layouts[name]
    if kind == "plain":
        return np.asarray(weights[srcs[0]])
    dims = [tuple(lowered.program.source_named(s).kind.dims) for s in srcs]
    mats = [np.asarray(weights[s], np.float16).reshape(d) for s, d in zip(srcs, dims)]
    if kind == "tiled":
        return pack(mats[0])
    return pack(pair(mats[0], mats[1]))


def check_rows(positions, slots, qblock: int = QBLOCK, first_rows: bool = False) -> None:
    """The attention's contract on a step's rows: every block of `qblock`
    rows is one sequence's (one slot) at consecutive positions.  With
    `first_rows`, rows of slot -1 are rows that fill the step out: a block's
    real rows come first, and its filling rows continue their positions."""
    pos = np.asarray(positions, np.int64).reshape(-1)
    sl = np.asarray(slots, np.int64).reshape(-1)
    if pos.size != sl.size or pos.size % qblock:
        raise LoweringError(f"{pos.size} rows: the prefill attention takes blocks of {qblock}")
    pb, sb = pos.reshape(-1, qblock), sl.reshape(-1, qblock)
    if first_rows:
        fill = sb < 0
        if np.any(fill[:, :-1] & ~fill[:, 1:]) or np.any(np.where(fill, sb[:, :1], sb) != sb[:, :1]):
            raise LoweringError(f"a block of {qblock} rows whose real rows are not first, or of two sequences")
    elif np.any(sb != sb[:, :1]):
        raise LoweringError(f"rows of a block of {qblock} are not one sequence's")
    if np.any(pb - pb[:, :1] != np.arange(qblock)):
        raise LoweringError(f"rows of a block of {qblock} are not one sequence's consecutive positions")


def run_of(seq_rows: int) -> int:
    """The rows a sequence's run takes in a step: its rows rounded up to
    whole query blocks, so that a step's tiles are whole runs (32, 64, 128
    or 256 rows, or a multiple of 256)."""
    if seq_rows < 1:
        raise LoweringError(f"a run of {seq_rows} rows")
    if seq_rows > SLAB:
        return -(-seq_rows // SLAB) * SLAB
    run = QBLOCK
    while run < seq_rows:
        run *= 2
    return run


class _RowsSession:
    """A step of many rows through the prefill kernels, its rows placed:
    ``place`` gives each row of the step (padded out to whole tiles) its
    position and slot; rows that only fill the step out store into the
    caches' scratch slot, one past the program's, and their outputs are
    never read.  The KV caches are the decode step's (the same names,
    layout and rounding), with that slot after them."""

    def _setup(self, device, kernels, dims, program, sequence_rows: int, rows: int, run_rows: int,
               positions, slots, real, scratch: bool, paging=None, tables=None) -> None:
        from .engine import Engine
        from .program.check import check_program
        from .program.plan import PlanOptions, plan

        self.device, self.kernels, self.dims = device, kernels, dims
        self.program = program
        self.checked = check_program(self.program)
        self.plan = plan(PlanOptions(sequence_rows=sequence_rows), self.checked)
        self.lowered = lower_prefill(self.checked, self.plan, rows, run_rows=run_rows, scratch_slot=scratch)
        self.engine = Engine(device, kernels, self.lowered)
        self.rows, self.run_rows = rows, run_rows
        self.real = np.asarray(real, np.int64)
        self.positions = np.asarray(positions, np.uint32)
        self.slots = np.asarray(slots, np.uint32)
        marks = np.where(np.isin(np.arange(rows), self.real), self.slots.astype(np.int64), -1)
        check_rows(self.positions, marks, QBLOCK, first_rows=True)
        # the real rows' positions and slots within their bounds; the
        # filling rows' positions continue their block's, past the bound
        bound = self.checked.program.source_named("position").kind.bound
        if np.any(self.positions[self.real] >= bound):
            raise LoweringError(f"positions {self.positions[self.real].tolist()} not below their bound {bound}")
        self.engine.write("ints:position", self.positions)
        if paging is None:
            self.engine.set_ints("slot", self.slots, dims.slots + int(scratch))
        else:
            block_size, pool_blocks = paging
            self.tables = np.asarray(tables, np.uint32)
            self.engine.set_ints("blocks", self.tables, pool_blocks + int(scratch))

    def weight_buffers(self):
        return [name for name in self.lowered.layouts]

    def write_weights(self, weights: dict) -> None:
        """Host weights (source name -> array), each into its buffer's layout."""
        for name in self.lowered.layouts:
            self.engine.write(name, weight_image(self.lowered, name, weights))

    def init_synthetic(self, seed: int = 2026, std: float = 0.02) -> None:
        """Weights std · N(0, 1) on the device (a layout permutes them, so the
        draw is the same in any layout), norm gains 1."""
        for i, name in enumerate(sorted(self.lowered.layouts)):
            kind, srcs = self.lowered.layouts[name]
            dims = self.lowered.program.source_named(srcs[0]).kind.dims
            if kind == "plain" and len(dims) == 1:
                self.engine.write(name, np.ones(dims[0], np.float32))
            else:
                self.engine.init_normal(name, seed + 7919 * i, std)
        self.device.sync()

    def set_tokens(self, tokens) -> None:
        """The real rows' tokens, in order (the filling rows take token 0)."""
        t = np.zeros(self.rows, np.uint32)
        t[self.real] = np.asarray(tokens, np.uint32).reshape(-1)
        self.engine.set_ints("tokens", t, self.dims.vocab)

    def set_rows(self, x: np.ndarray) -> None:
        """The real rows' inputs, in order (the filling rows zero)."""
        x = np.asarray(x, np.float32).reshape(len(self.real), -1)
        full = np.zeros((self.rows, x.shape[1]), np.float32)
        full[self.real] = x
        self.engine.write("value:x", full.reshape(-1))

    def run(self, stream=None) -> None:
        self.engine.enqueue(stream)

    def graph(self, stream=None):
        return self.engine.capture(stream=stream)

    @property
    def staged(self) -> bool:
        return any(L.entry == "fk_prefill_land" for L in self.lowered.launches)

    def logits(self) -> np.ndarray:
        """The real rows' logits, in order."""
        return self.engine.read("value:logits").reshape(self.rows, -1)[self.real]

    def tokens(self) -> np.ndarray:
        return self.engine.read("value:token")[self.real]

    def cache(self, name: str) -> np.ndarray:
        return self.engine.read(f"cache:{name}")

    def close(self) -> None:
        self.engine.close()


class PrefillSession(_RowsSession):
    """The prefill of `seqs` sequences of `seq_rows` rows each (positions 0 ..
    seq_rows - 1, sequence i in ring slot i) through one decoder program:
    gated, planned with steps of the sequence's rows, lowered to the prefill
    kernels and resident on one GPU.  The KV caches it fills are the decode
    step's (the same names, layout and rounding)."""

    def __init__(self, device, kernels, dims, seqs: int, seq_rows: int, layers: Optional[int] = None,
                 embed: bool = True, rope_rotated: Optional[int] = None, position_bound: Optional[int] = None,
                 paging: Optional[tuple] = None, tables: Optional[np.ndarray] = None):
        from .program.decoder import decoder_step

        if seqs < 1 or seqs > dims.slots:
            raise LoweringError(f"{seqs} sequences for caches of {dims.slots} slots")
        self.seqs, self.seq_rows = seqs, seq_rows
        self.embed = embed
        # Each sequence's rows take a run of whole query blocks, and the step
        # whole tiles of runs: rows past a sequence's (and whole runs past
        # the sequences) fill them out, in the scratch slot.
        rows, run, positions, slots, real = prefill_placement(seqs, seq_rows, dims.slots)
        pad = rows != seqs * seq_rows
        rows_tables = None
        if paging is not None:
            # Paged pools (paging = (block size, pool blocks)): sequence i's
            # block table is row i of `tables` (default: distinct blocks in a
            # scrambled order), every row of the sequence carrying it; the
            # filling rows' tables hold the scratch block.
            block_size, pool_blocks = paging
            table_len = dims.context // block_size
            if tables is None:
                if seqs * table_len > pool_blocks:
                    raise LoweringError(f"{seqs} tables of {table_len} blocks in a pool of {pool_blocks}")
                perm = np.random.default_rng(0).permutation(pool_blocks)[:seqs * table_len]
                tables = perm.reshape(seqs, table_len)
            tables = np.asarray(tables, np.uint32).reshape(seqs, table_len)
            rows_tables = np.full((rows, table_len), pool_blocks, np.uint32)
            for i in range(seqs):
                rows_tables[i * run:i * run + seq_rows] = tables[i]
        # Positions below `position_bound` (the rows' own, seq_rows, by
        # default): a bound past what the ring holds beyond a step's rows
        # makes the plan stage the KV stores.
        program = decoder_step(dims, "prefill", embed, layers, position_bound=position_bound or seq_rows,
                               rope_rotated=rope_rotated, paging=paging)
        self._setup(device, kernels, dims, program, seq_rows, rows, run, positions, slots, real, pad, paging,
                    rows_tables)
        if paging is not None:
            self.tables = tables



class DecodeRows(_RowsSession):
    """A decode step of several rows (Eval.hs:126-140: each row a sequence
    at its own position and slot) through the prefill kernels: row i is the
    first row of query block i, whose other 31 rows continue its positions
    in the scratch slot (their outputs unread), the step filled out to whole
    tiles likewise.  The program is the decode step's (``decoder_step``,
    positions below the context), planned one row a sequence."""

    def __init__(self, device, kernels, dims, positions, slots, layers: Optional[int] = None, embed: bool = True):
        from .program.decoder import decoder_step

        self.embed = embed
        rows, pos, sl, real = decode_placement(positions, slots, dims.slots)
        program = decoder_step(dims, "decode", embed, layers, position_bound=dims.context)
        self._setup(device, kernels, dims, program, 1, rows, QBLOCK, pos, sl, real, True)


def decode_placement(positions, slots, n_slots: int) -> tuple:
    """A decode step's rows in a step of whole tiles: (rows, each row's
    position, its slot, the real rows).  Row i is the first row of query
    block i; the rest of each block continues its positions in the scratch
    slot (`n_slots`), and blocks past the rows fill the tiles out there."""
    positions = np.asarray(positions, np.uint32).reshape(-1)
    slots = np.asarray(slots, np.uint32).reshape(-1)
    m = positions.size
    if m < 1 or slots.size != m or np.any(slots >= n_slots):
        raise LoweringError(f"{m} rows in slots {slots.tolist()} of {n_slots}")
    rows = -(-m * QBLOCK // SLAB) * SLAB
    pos = np.zeros(rows, np.uint32)
    sl = np.full(rows, n_slots, np.uint32)
    for b in range(rows // QBLOCK):
        pos[b * QBLOCK:(b + 1) * QBLOCK] = (positions[b] if b < m else 0) + np.arange(QBLOCK, dtype=np.uint32)
    real = np.arange(m) * QBLOCK
    sl[real] = slots
    return rows, pos, sl, real


def prefill_placement(seqs: int, seq_rows: int, n_slots: int) -> tuple:
    """A prefill's rows in a step of whole tiles: (rows, the run of each
    sequence, each row's position, its slot, the real rows).  Sequence i's
    rows (positions 0 .. seq_rows - 1, slot i) start run i; the run's rest,
    and runs past the sequences, continue positions in the scratch slot
    (`n_slots`)."""
    run = run_of(seq_rows)
    rows = -(-seqs * run // SLAB) * SLAB
    positions = np.tile(np.arange(run, dtype=np.uint32), rows // run)
    slots = np.full(rows, n_slots, np.uint32)
    real = np.concatenate([np.arange(i * run, i * run + seq_rows) for i in range(seqs)])
    for i in range(seqs):
        slots[i * run:i * run + seq_rows] = i
    return rows, run, positions, slots, real
