"""Every memory access a GEMV step launch makes, computed on the CPU the way
fk_step_gemv.h computes it (the prologue's loads, each wavefront's blocks of
rows and their weight loads, the residual loads, the stores, the argmax
slots, the LDS slots), and checked against the sizes of the buffers the
launch binds.  A launch is never sent to the GPU with a grid or a shape
whose accesses this finds out of bounds.
"""

from __future__ import annotations

import numpy as np

WAVE = 64
THREADS = 512
PRO_STORED, PRO_RMSNORM, PRO_GATHER, PRO_GATHER_RMSNORM, PRO_SILU_MUL, PRO_COMBINE = range(6)
COMBINE_SPLITS = 8
EPI_NONE, EPI_ADD_STORED, EPI_ADD_GATHER, EPI_SILU_MUL, EPI_ARGMAX, EPI_SOFTCAP = range(6)
ELT = {"f32": 4, "f16": 2, "bf16": 2, "u32": 4, "u16": 2, "u64": 8}


def shape_of(entry: str) -> tuple[int, int, int, int]:
    """(weight bytes, pack elements P, rows a block R, packs a lane KPL)."""
    parts = entry.split("_")  # fk step gemv <wt> k<K> r<R> p<> e<>
    wt, kmax, r = parts[3], int(parts[4][1:]), int(parts[5][1:])
    eb = 4 if wt == "f32" else 2
    p = 16 // eb
    return eb, p, r, kmax // (WAVE * p)


def modes_of(entry: str) -> tuple[int, int]:
    """(prologue, epilogue) from the entry's `_p<pro>_e<epi>` suffix."""
    parts = entry.split("_")
    if not (parts[-2].startswith("p") and parts[-1].startswith("e")):
        raise Bad(f"{entry}: no _p<prologue>_e<epilogue> suffix")
    return int(parts[-2][1:]), int(parts[-1][1:])


class Bad(AssertionError):
    pass


def check_launch(launch, buffers: dict, groups: int | None = None) -> None:
    """Raises Bad naming the first access out of bounds; `buffers` maps a
    logical buffer to its BufferSpec, `groups` overrides the launch's grid."""
    prm, bind = launch.params, launch.bind
    groups = launch.groups if groups is None else groups
    if launch.threads != THREADS:
        raise Bad(f"{launch.entry}: {launch.threads} threads")
    eb, P, R, KPL = shape_of(launch.entry)
    # The kernel is specialised on the modes its entry's name carries
    # (<shape>_p<prologue>_e<epilogue>); its parameter struct's modes are
    # never read on the device.
    pro, epi = modes_of(launch.entry)
    k, n_anchors, rows, first = prm["k"], prm["n_anchors"], prm["rows"], prm["first_row"]
    blocks = prm["blocks"]
    C = P // 4
    NPK = max(1, KPL * P // 32)
    XT = WAVE * P * KPL // 4
    packs, packs4 = k // P, k // 4
    gather = pro in (PRO_GATHER, PRO_GATHER_RMSNORM)
    norm = pro in (PRO_RMSNORM, PRO_GATHER_RMSNORM)

    # Element sizes the kernel reads each buffer at: the weights and the
    # gathered tables as the entry's weight type, the argmax slots as u64, the
    # tokens as u32, every row as f32.
    at_size = {**{f"w{j}": eb for j in range(3)}, "table": eb, "res_table": eb, "arg": 8}

    def elems(name: str) -> int:
        """The buffer's extent in elements of the size the kernel reads it at
        (an unbound buffer is address 0: any access to it is out of bounds)."""
        if bind.get(name) is None:
            raise Bad(f"{launch.entry}: {name} is read or written but not bound (address 0)")
        spec = buffers[bind[name]]
        return spec.count * ELT[spec.dtype] // at_size.get(name, 4)

    def need(name: str, idx: np.ndarray, what: str, width: int = 1) -> None:
        n = elems(name)
        idx = np.asarray(idx)
        if idx.size and (idx.min() < 0 or idx.max() + width > n):
            raise Bad(f"{launch.entry}: {what} reads/writes {name}[{int(idx.min())}..{int(idx.max()) + width - 1}] "
                      f"of {n}")

    # LDS: the kernel's dynamic LDS holds xt[XT] float4s (and gt[XT] for the norm).
    if launch.lds_bytes < XT * 16 * (2 if norm else 1):
        raise Bad(f"{launch.entry}: {launch.lds_bytes} bytes of LDS for {XT} float4s")
    if k > WAVE * P * KPL or k % P or k % 4:
        raise Bad(f"{launch.entry}: k = {k} for packs of {P}, {KPL} a lane")
    if n_anchors < 1 or n_anchors > 3 or any(rows[a] < 1 for a in range(n_anchors)):
        raise Bad(f"{launch.entry}: anchors {rows}")

    # Prologue loads (thread t, m < NPK): j = min(t + 512 m, packs4 - 1).
    t = np.arange(THREADS)
    j = np.minimum(t[:, None] + THREADS * np.arange(NPK)[None, :], packs4 - 1).ravel()
    if gather:
        table_rows = prm["table_rows"]
        need("token", np.array([0]), "the token")
        tok = table_rows - 1  # the largest row a clamped token reaches
        need("table", tok * k + 4 * j, "the gathered row", 4)
    elif pro == PRO_COMBINE:
        # Head h = 4j div d, dimensions i = 4j mod d: each split's (clamped)
        # accumulators (4 floats) and its (max, sum) pair.
        d, splits = prm["head_dim"], prm["splits"]
        heads = k // d
        if not 1 <= splits <= COMBINE_SPLITS or d % 4 or k % d:
            raise Bad(f"{launch.entry}: a combine of {splits} splits of heads of {d}")
        h, i = (4 * j) // d, (4 * j) % d
        tc = np.minimum(np.arange(COMBINE_SPLITS), splits - 1)
        need("src", ((h[:, None] * splits + tc[None, :]) * d + i[:, None]).ravel(), "the partials", 4)
        need("src", (heads * splits * d + (h[:, None] * splits + tc[None, :]) * 2).ravel(), "the splits' stats", 2)
    else:
        need("src", 4 * j, "the stored row", 4)
    if pro == PRO_SILU_MUL:
        need("src2", prm.get("src2_off", 0) + 4 * j, "the second row", 4)
    if norm:
        need("gamma", 4 * j, "the gains", 4)
    # LDS writes: xt_at(j) for j < max(packs4, XT) within t + 512 m.
    jj = (t[:, None] + THREADS * np.arange(NPK)[None, :]).ravel()
    jj = jj[jj < max(packs4, XT)]
    pk = jj // C
    at = ((pk // WAVE) * C + jj % C) * WAVE + pk % WAVE
    if at.size and at.max() >= XT:
        raise Bad(f"{launch.entry}: LDS slot {int(at.max())} of {XT}")

    if epi == EPI_ADD_GATHER:
        # The residual's token is read before the first block, by every thread.
        need("res_token", np.array([0]), "the residual's token")

    # Blocks: wavefront gw takes b = gw, gw + total, ... while b < blocks, and
    # issues its first block's loads (clamped) even when gw is past the blocks.
    total_waves = groups * (THREADS // WAVE)
    issued = np.unique(np.concatenate([np.arange(total_waves), np.arange(blocks)]))
    if epi == EPI_SILU_MUL and R == 1:
        # every wavefront of a threadgroup runs as many blocks as its first:
        # blocks up to the next multiple of the threadgroup's wavefronts
        waves = THREADS // WAVE
        issued = np.unique(np.concatenate([issued, np.arange(-(-blocks // waves) * waves)]))

    lanes = np.arange(WAVE)
    jl = np.minimum(lanes[:, None] + WAVE * np.arange(KPL)[None, :], packs - 1).ravel()
    for q in range(R):
        b = issued
        if epi == EPI_SILU_MUL and R == 1:
            a = b & 1
            row = b >> 1
            live = (b < blocks) & (row < rows[0])
        elif epi == EPI_SILU_MUL:
            H = max(R // 2, 1)
            a = np.where(q < H, 0, 1)
            a = np.full(b.shape, a)
            row = b * H + q % H
            live = (b < blocks) & (row < rows[0])
        else:
            g = b * R + q
            a = ((n_anchors > 1) & (g >= first[1])).astype(int) + ((n_anchors > 2) & (g >= first[2])).astype(int)
            row = g - np.array(first)[a]
            live = (b < blocks) & (g < first[n_anchors])
        for an in range(n_anchors):
            sel = a == an
            if not sel.any():
                continue
            n = rows[an]
            r = np.minimum(row[sel], n - 1)
            need(f"w{an}", (r[:, None] * k + jl[None, :] * P).ravel(), f"anchor {an}'s weights", P)
            lv = live[sel]
            rl = row[sel][lv]
            if rl.size:
                if prm["store_tile"]:
                    need(f"y{an}", rl, f"anchor {an}'s tile")
                if epi in (EPI_ADD_STORED, EPI_ADD_GATHER):
                    need("epi_out", rl, "the epilogue row")
                    if epi == EPI_ADD_STORED:
                        need("res", np.minimum(rl, n - 1), "the residual")
                if epi == EPI_SILU_MUL and an == 0:
                    need("epi_out", rl, "the SiLU·mul row")
                if epi == EPI_SOFTCAP:
                    need("epi_out", rl, "the softcap row")
            # The residual of every block below `blocks` is loaded (its row
            # clamped into the anchor), live or not.
            ran = row[sel][b[sel] < blocks]
            if ran.size and epi == EPI_ADD_STORED:
                need("res", np.minimum(ran, n - 1), "the residual (clamped)")
            if ran.size and epi == EPI_ADD_GATHER:
                need("res_table", (prm["table_rows"] - 1) * n + np.minimum(ran, n - 1), "the gathered residual")
    if epi == EPI_ARGMAX or (epi == EPI_SOFTCAP and prm.get("arg_slots", 0)):
        slots = prm["arg_slots"]
        if slots > elems("arg"):
            raise Bad(f"{launch.entry}: {slots} argmax slots in a buffer of {elems('arg')}")
    if epi == EPI_SILU_MUL and (n_anchors != 2 or rows[0] != rows[1] or (R == 1 and blocks != 2 * rows[0])):
        raise Bad(f"{launch.entry}: the SiLU·mul epilogue on anchors {rows[:n_anchors]}, {blocks} blocks of {R}")
