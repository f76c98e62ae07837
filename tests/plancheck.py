"""A plan's dependencies, checked apart from the planner by its rules
(test/Test/FuryKernel/PlanCheck.hs restated): every step reads only what
earlier steps stored or what its own work makes; epilogues are elementwise on
one linear layer's tile; combines read their attention's partials in a light
step; stores into caches land before the attention that reads them and after
those before; staging iff a ring lacks room; every anchor, effect and stage
placed once; every output stored; gated routes stored by an earlier light step.
"""

from __future__ import annotations

from furykernel_amd.program.graph import (
    Add, Attend, GeluMul, Input, KvStore, Linear, LinearRouted, Ring, SCache, ScaleBy, Softcap, SRowInts,
    Standardize, op_values)
from furykernel_amd.program.plan import (
    ANCHOR, COMBINE, EFFECT, EPILOGUE, LAND, PARTIALS, RECOMPUTE, STAGE, Plan, PlanOptions)


def _is_linear(op):
    return isinstance(op, (Linear, LinearRouted))


def _elementwise(op):
    return isinstance(op, (Add, ScaleBy, GeluMul, Softcap, KvStore, Standardize))


def _attended(op):
    return [op.to.keys, op.to.values] if isinstance(op, Attend) else []


def _written(op):
    return [op.at.cache] if isinstance(op, KvStore) else []


def plan_issues(opts: PlanOptions, pl: Plan) -> list[str]:
    p = pl.program
    steps = pl.steps
    nodes = {n.id: n for n in p.nodes}

    def op_of(n):
        return nodes[n].op if n in nodes else Input(0)

    def outs_of(n):
        return list(nodes[n].outputs) if n in nodes else []

    def node_name(n):
        return nodes[n].name if n in nodes else "?"

    def value_name(v):
        val = p.value(v)
        return val.name if val else "?"

    def is_input(v):
        prod = p.producer(v)
        return prod is not None and isinstance(prod.op, Input)

    inputs = {v.id for v in p.values if is_input(v.id)}

    def places(w):
        return w.kind in (ANCHOR, EFFECT, STAGE) or (w.kind == EPILOGUE and isinstance(op_of(w.node), KvStore))

    def writes(w):
        if w.kind == STAGE:
            return []
        if w.kind == LAND:
            return _written(op_of(w.node))
        return _written(op_of(w.node)) if places(w) else []

    staged_nodes = {w.node for s in steps for w in s.work if w.kind == STAGE}

    def stage_of(n):
        op = op_of(n)
        return (op.x, op.at.cache) if isinstance(op, KvStore) else None

    def staged_into(c):
        return [(n, stage_of(n)) for n in sorted(staged_nodes) if stage_of(n) and stage_of(n)[1] == c]

    order = {n.id: k for k, n in enumerate(p.nodes)}
    issues: list[str] = []
    elems, partials, stages = set(inputs), set(), set()
    placed: dict[int, list[int]] = {}
    stored_by: dict[int, list[int]] = {}

    for s in steps:
        found: list[str] = []
        local, tile = set(), {}
        read_e, read_p, read_s = set(), set(), set()

        def read_one(what, v):
            if v in local:
                return
            if v in elems:
                read_e.add(v)
            elif v in tile:
                found.append(f"{what} reads {value_name(v)}, on the tile of {node_name(tile[v])}")
            else:
                found.append(f"{what} reads {value_name(v)}, which no earlier step stored and the step doesn't compute")

        for w in s.work:
            op = op_of(w.node)
            if w.kind == RECOMPUTE:
                for v in op_values(op):
                    read_one(f"recompute {node_name(w.node)}", v)
                local |= set(outs_of(w.node))
            elif w.kind == COMBINE:
                if isinstance(op, Attend):
                    outs = outs_of(w.node)
                    if all(v in partials for v in outs):
                        read_p |= set(outs)
                    else:
                        found.append(f"combine {node_name(w.node)} of partials no earlier step stored")
                    if s.anchors:
                        found.append(f"combine {node_name(w.node)} in a step of anchors")
                    local |= set(outs)
                else:
                    found.append(f"combine of {node_name(w.node)}, which isn't attention")
            elif w.kind == ANCHOR:
                for v in op_values(op):
                    read_one(f"anchor {node_name(w.node)}", v)
                for c in dict.fromkeys(_attended(op)):
                    for store, key in staged_into(c):
                        if order.get(store, -1) < order.get(w.node, -1):
                            if key in stages:
                                read_s.add(key)
                            else:
                                found.append(f"anchor {node_name(w.node)} reads the values {node_name(store)} "
                                             f"stages, which no earlier step staged")
                for v in outs_of(w.node):
                    tile[v] = w.node
            elif w.kind == EPILOGUE:
                ins = op_values(op)
                tiled = [(v, tile[v]) for v in ins if v in tile]
                if not _elementwise(op):
                    found.append(f"epilogue {node_name(w.node)} isn't elementwise")
                for v in ins:
                    if v not in [t for t, _ in tiled]:
                        read_one(f"epilogue {node_name(w.node)}", v)
                anchors = list(dict.fromkeys(a for _, a in tiled))
                if len(anchors) == 1:
                    a = anchors[0]
                    if not _is_linear(op_of(a)):
                        found.append(f"epilogue {node_name(w.node)} on the tile of {node_name(a)}, which holds partials")
                    for v in outs_of(w.node):
                        tile[v] = a
                elif not anchors:
                    found.append(f"epilogue {node_name(w.node)} on no tile")
                else:
                    found.append(f"epilogue {node_name(w.node)} on several tiles")
            elif w.kind in (EFFECT, STAGE):
                for v in op_values(op):
                    read_one(f"{w.kind} {node_name(w.node)}", v)
            elif w.kind == LAND:
                if s.anchors:
                    found.append(f"land {node_name(w.node)} in a step of anchors")
                key = stage_of(w.node)
                if key is None:
                    found.append(f"land of {node_name(w.node)}, which isn't a store")
                elif key in stages:
                    read_s.add(key)
                else:
                    found.append(f"land {node_name(w.node)} of values no earlier step staged")
        for st in s.stores:
            if st.form == PARTIALS:
                a = tile.get(st.value)
                if a is None or not isinstance(op_of(a), Attend):
                    found.append(f"stores {value_name(st.value)} as partials, which aren't its attention's")
            elif st.form[0] == "elements":
                val = p.value(st.value)
                if val is None or val.type != st.form[1]:
                    found.append(f"stores {value_name(st.value)} as another type")
                if st.value in local:
                    pass
                elif st.value in tile:
                    if not _is_linear(op_of(tile[st.value])):
                        found.append(f"stores {value_name(st.value)} as elements, from the partials of "
                                     f"{node_name(tile[st.value])}")
                else:
                    found.append(f"stores {value_name(st.value)}, which it doesn't compute")
            else:
                keys = [stage_of(w.node) for w in s.work if w.kind == STAGE]
                if (st.value, st.form[1]) not in keys:
                    found.append(f"stores {value_name(st.value)} staged, which none of its stages keeps")
        listed_e = {st.value for st in s.reads if st.form[0] == "elements"}
        listed_p = {st.value for st in s.reads if st.form == PARTIALS}
        listed_s = {(st.value, st.form[1]) for st in s.reads if st.form[0] == "staged"}
        if listed_e != read_e or listed_p != read_p:
            found.append(f"lists the reads {sorted(listed_e)} and partials {sorted(listed_p)}, but its work reads "
                         f"{sorted(read_e)} and partials {sorted(read_p)}")
        if listed_s != read_s:
            found.append("lists other stages than its work reads")
        for w in s.work:
            if w.kind == STAGE:
                x, c = stage_of(w.node)
                if not any(st.value == x and st.form == ("staged", c) for st in s.stores):
                    found.append("stages and doesn't store their values")
        stores_c = [c for w in s.work for c in writes(w)]
        attends = [c for w in s.work if w.kind == ANCHOR for c in _attended(op_of(w.node))]
        if any(c in attends for c in stores_c):
            found.append("stores into a cache its attention reads")
        if len(stores_c) != len(set(stores_c)):
            found.append("stores into one cache twice")
        issues += [f"{s.name}: {f}" for f in found]
        elems |= {st.value for st in s.stores if st.form[0] == "elements"}
        partials |= {st.value for st in s.stores if st.form == PARTIALS}
        stages |= {(st.value, st.form[1]) for st in s.stores if st.form[0] == "staged"}
        for w in s.work:
            if places(w):
                placed.setdefault(w.node, []).append(s.index)
        for st in s.stores:
            if st.form[0] == "elements":
                stored_by.setdefault(st.value, []).append(s.index)

    def placed_once(n):
        v = placed.get(n, [])
        return v[0] if len(v) == 1 else None

    for a in p.nodes:
        if not isinstance(a.op, Attend):
            continue
        for k in p.nodes:
            if not any(c in _attended(a.op) for c in _written(k.op)):
                continue
            sa, sk = placed_once(a.id), placed_once(k.id)
            if sa is None or sk is None:
                continue
            if order[k.id] < order[a.id]:
                if not sk < sa:
                    issues.append(f"{k.name} and {a.name}: a store before attention in the program, not in an earlier step")
            elif not sk > sa:
                issues.append(f"{k.name} and {a.name}: a store after attention in the program, not in a later step")

    def bound(s):
        src = p.source(s)
        return src.kind.bound if src is not None and isinstance(src.kind, SRowInts) else 0

    for i, n in enumerate(p.nodes):
        if not isinstance(n.op, KvStore):
            continue
        c = n.op.at.cache
        is_staged = n.id in staged_nodes
        rooms = []
        src = p.source(c)
        if src is not None and isinstance(src.kind, SCache) and isinstance(src.kind.layout, Ring):
            length = src.kind.layout.length
            for r in p.nodes[i + 1:]:
                if isinstance(r.op, Attend) and c in (r.op.to.keys, r.op.to.values):
                    reads = bound(r.op.to.positions) if r.op.spec.window is None else r.op.spec.window
                    rooms.append(0 if reads > length else length - reads + 1)
        if is_staged != any(opts.sequence_rows > room for room in rooms):
            issues.append(f"{n.name}: " + ("staged, though its ring has room for a step's rows of one sequence"
                                           if is_staged else
                                           "stored first, though its ring hasn't room for a step's rows of one sequence"))

    for n in sorted(staged_nodes):
        lands = [s.index for s in steps for w in s.work if w.kind == LAND and w.node == n]
        key = stage_of(n)
        if key is None:
            continue
        if len(lands) == 1:
            for a in p.nodes:
                if key[1] in _attended(a.op) and order[n] < order[a.id]:
                    sa = placed_once(a.id)
                    if sa is not None and lands[0] <= sa:
                        issues.append(f"{node_name(n)}: lands in a step no later than {a.name}'s, which reads its ring")
        else:
            issues.append(f"{node_name(n)}: lands {len(lands)} times")

    for n in p.nodes:
        if isinstance(n.op, (Linear, LinearRouted, Attend, KvStore)) and placed_once(n.id) is None:
            issues.append(f"{n.name}: placed {len(placed.get(n.id, []))} times")
    for o in p.outputs:
        if not is_input(o.value) and o.value not in stored_by:
            issues.append(f"output {o.name} is never stored")
    if opts.gated:
        light = {s.index for s in steps if s.is_light}
        for s in steps:
            for n in s.anchors:
                op = op_of(n)
                if isinstance(op, LinearRouted) and not is_input(op.ids):
                    if not any(i < s.index and i in light for i in stored_by.get(op.ids, [])):
                        issues.append(f"gated: {node_name(n)} reads its route {value_name(op.ids)}, which no "
                                      f"earlier light step stored")
    return issues
