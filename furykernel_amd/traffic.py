"""Algorithmic HBM bytes of a lowered launch: what it must read and write, once
each, at a given decode position — the figure a kernel's achieved GB/s is
quoted against.

Counted per launch, from its parameters and the buffer types it binds:

- GEMV step: every weight row of its anchors, the input row (the stored
  f32 row, both rows of a SiLU·mul, or the gathered table row and its
  token), the norm gains, the stored tiles, the residual row read and the
  epilogue row written;
- KV store: each stored row read (f32) and written to the cache (f16/bf16),
  and the RoPE table row;
- attention: K and V of every position the query reads (the ring up to the
  position, or the window), the query rows, the RoPE row and the partials
  written; with the store folded in, the new rows read and stored;
- combine: the partials read and the combined rows written;
- argmax, SiLU·mul: their rows; a folded SiLU·mul its stored row, a folded
  argmax its threadgroups' 64-bit keys, the token launch those keys read and
  the token written.
"""

from __future__ import annotations

from .lower import EPI_ADD_GATHER, EPI_ADD_STORED, EPI_ARGMAX, EPI_SILU_MUL, EPI_SOFTCAP, PRO_COMBINE, PRO_GATHER, \
    PRO_GATHER_RMSNORM, PRO_SILU_MUL, Launch, Lowered

_ELT = {"f32": 4, "u32": 4, "f16": 2, "bf16": 2, "u16": 2, "u64": 8}


def _elt(lowered: Lowered, name: str) -> int:
    return _ELT[lowered.buffers[name].dtype]


def positions_read(length: int, window: int, position: int) -> int:
    """Cache positions an attention at `position` reads: up to the ring's
    length, or the window's."""
    n = min(position + 1, length)
    return min(n, window) if window else n


def launch_bytes(lowered: Lowered, launch: Launch, position: int) -> int:
    b, p, e = launch.bind, launch.params, launch.entry
    if e.startswith("fk_step_gemv"):
        k = p["k"]
        rows = p["rows"][:p["n_anchors"]]
        total = sum(r * k * _elt(lowered, b[f"w{j}"]) for j, r in enumerate(rows))
        if p["pro_mode"] in (PRO_GATHER, PRO_GATHER_RMSNORM):
            total += k * _elt(lowered, b["table"]) + 4
        elif p["pro_mode"] == PRO_COMBINE:
            total += (k // p["head_dim"]) * p["splits"] * (p["head_dim"] + 2) * 4
        else:
            total += k * 4 * (2 if p["pro_mode"] == PRO_SILU_MUL else 1)
        if p["has_gamma"]:
            total += k * 4
        if p["store_tile"]:
            total += sum(rows) * 4
        if p["epi_mode"] == EPI_ADD_STORED:
            total += rows[0] * 4 * 2
        elif p["epi_mode"] == EPI_ADD_GATHER:
            total += rows[0] * _elt(lowered, b["res_table"]) + 4 + rows[0] * 4
        elif p["epi_mode"] == EPI_SILU_MUL:
            total += rows[0] * 4
        elif p["epi_mode"] == EPI_ARGMAX:
            total += 8 * launch.groups
        elif p["epi_mode"] == EPI_SOFTCAP:
            total += rows[0] * 4 + (8 * launch.groups if p.get("arg_slots") else 0)
        return total
    if e == "fk_step_token":
        return 8 * p["slots"] + 4
    if e == "fk_step_store":
        row = p["kv_heads"] * p["head_dim"]
        cache = 2 if p["cache_bf16"] or lowered.buffers[b["c0"]].dtype == "f16" else 4
        total = p["n_stores"] * row * (4 + cache) + 8
        if p["rope"] != [0, 0]:
            total += p["rotated"] * 8
        return total
    if e in ("fk_step_attend", "fk_step_attend_wide"):
        n = positions_read(p["length"], p["window"], position)
        elt = _elt(lowered, b["kc"])
        d = p["head_dim"]
        total = 2 * p["kv_heads"] * n * d * elt + p["heads"] * d * 4 + 8
        partials = p["heads"] * -(-n // p["split"]) * (d + 2) * 4
        total += partials
        if p["rope"] or p["krope"]:
            total += p["rotated"] * 8
        if p["store"]:
            total += 2 * p["kv_heads"] * d * (4 + elt)
        return total
    if e == "fk_step_combine":
        d = p["head_dim"]
        return p["heads"] * p["splits"] * (d + 2) * 4 + p["heads"] * d * 4
    if e == "fk_step_argmax":
        return p["n"] * 4 + 4
    if e == "fk_step_act_mul":
        return p["n"] * 4 * 3
    if e.startswith("fk_gemv_p4_"):
        eb = 4 if e.endswith("f32") else 2
        return p["n"] * p["k"] * eb + p["k"] * 4 + p["n"] * 4
    if e == "fk_step_elementwise":
        if p["op"] == 2:      # standardize: the row, bias and scale in, the row out
            return p["n"] * 8 + p["width"] * 8
        if p["op"] == 1:      # scale: the row and the factor in, the row out
            return p["n"] * 8 + 4
        return p["n"] * 12 if p["op"] == 0 else p["n"] * 8
    if e.startswith("fk_step_gather_"):
        eb = 4 if e.endswith("f32") else 2
        return p["rows"] * p["width"] * (p["count"] * eb + 4) + p["rows"] * p["count"] * 4
    if e == "fk_prefill_softcap":
        return p["count"] * 4 * 2
    raise ValueError(f"no byte count for {e}")


def step_bytes(lowered: Lowered, position: int) -> int:
    return sum(launch_bytes(lowered, launch, position) for launch in lowered.launches)
