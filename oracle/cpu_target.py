"""The CPU target of the oracle: a lowered plan's launches run by the C
restatement, each kernel's loops in the order its gfx950 kernel computes, its
buffers numpy arrays named as the engine names its device buffers.

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker of the GPU engine (same launch
list, same arithmetic, compared bit for bit) and as the CPU baseline.

``width`` is the SIMD width of the reductions: 64 for the gfx950 kernels'
bits, 32 for the reference CPU target's.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import fkref

NP = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "u32": np.uint32, "u16": np.uint16,
      "u64": np.uint64}
EPI_SILU_MUL, EPI_ARGMAX, EPI_SOFTCAP = 3, 4, 5
PRO_COMBINE = 5
TYPE = {"f16": fkref.F16, "bf16": fkref.BF16, "f32": fkref.F32}


class CpuTarget:
    def __init__(self, lowered, width: int = 64):
        self.lowered = lowered
        self.width = width
        self.buffers = {name: np.zeros(spec.count, NP[spec.dtype]) for name, spec in lowered.buffers.items()}

    def write(self, name: str, values) -> None:
        a = np.asarray(values, dtype=self.buffers[name].dtype).reshape(-1)
        if a.size != self.buffers[name].size:
            raise ValueError(f"{name}: {a.size} elements for {self.buffers[name].size}")
        self.buffers[name][:] = a

    def read(self, name: str) -> np.ndarray:
        return self.buffers[name].copy()

    def _p(self, name):
        return None if name is None else self.buffers[name].ctypes.data

    def _pool(self, addr: str):
        """A paged pool's blocks as this target holds them: an array of the
        blocks' host addresses, in order in the pool's buffer (the device's
        address table, which the engine writes, read here as that)."""
        kind, pool, block_bytes = self.lowered.constants[addr]
        base = self.buffers[pool].ctypes.data
        n = self.lowered.buffers[addr].count
        return (ctypes.c_void_p * n)(*[base + i * block_bytes for i in range(n)])

    def _reach(self, b, p, pos: int) -> int:
        return int(self.buffers[b["reach"]][0]) if p.get("has_reach") else pos

    def run(self) -> None:
        for launch in self.lowered.launches:
            self.run_launch(launch)

    def run_launch(self, launch) -> None:
        L = fkref.lib()
        b, p = launch.bind, launch.params
        e = launch.entry
        if e.startswith("fk_step_gemv"):
            wt = e.split("_")[3]
            n = p["n_anchors"]
            src = self._p(b["src"])
            pro = p["pro_mode"]
            if pro == PRO_COMBINE:
                # The combine prologue: the combine kernel's row, then the
                # GEMV step on it as a stored row.
                d = p["head_dim"]
                row = np.zeros(p["k"], np.float32)
                st = L.fkref_step_combine(src, row.ctypes.data, p["k"] // d, d, p["splits"])
                if st:
                    raise ValueError(f"{launch.step} ({e}): the oracle refused its combine (status {st})")
                src, pro = row.ctypes.data, 0
            epi = p["epi_mode"]
            folded = epi in (EPI_SILU_MUL, EPI_ARGMAX, EPI_SOFTCAP)
            # A folded epilogue reads the anchors' tiles: kept here whether or not
            # the step stores them.
            tiles = [self.buffers[b[f"y{j}"]] if b[f"y{j}"] else np.zeros(p["rows"][j], np.float32)
                     for j in range(n)]
            ws = (ctypes.c_void_p * 3)(*[self._p(b[f"w{j}"]) for j in range(3)])
            ys = (ctypes.c_void_p * 3)(*([t.ctypes.data for t in tiles] + [None] * (3 - n)))
            rows = (ctypes.c_int * 3)(*p["rows"])
            tok = int(self.buffers[b["token"]][0]) if b["token"] else 0
            rtok = int(self.buffers[b["res_token"]][0]) if b["res_token"] else 0
            st = L.fkref_step_gemv(ws, TYPE[wt], ys, rows, n, p["k"], pro, src,
                                   self._p(b["src2"]), self._p(b["gamma"]) if p["has_gamma"] else None,
                                   self._p(b["table"] or b["res_table"]), tok, p["table_rows"], p["seg"], p["eps"],
                                   p["factor"], p["gfactor"], 0 if folded else epi, self._p(b["res"]),
                                   self._p(b["res_table"]), rtok, None if folded else self._p(b["epi_out"]),
                                   launch.threads, self.width, p.get("act", 0), p.get("src2_off", 0))
            if not st and epi == EPI_SILU_MUL:
                st = L.fkref_act_mul(tiles[0].ctypes.data, tiles[1].ctypes.data, self._p(b["epi_out"]), p["rows"][0],
                                     p.get("act", 0))
            keyed = None
            if not st and epi == EPI_SOFTCAP:
                out = self.buffers[b["epi_out"]]
                for i, v in enumerate(tiles[0][:p["rows"][0]]):
                    out[i] = L.fkref_softcap(float(v), p["cap"])
                keyed = out if p.get("arg_slots", 0) else None
            if not st and epi == EPI_ARGMAX:
                keyed = tiles[0]
            if keyed is not None:
                # Each threadgroup's largest key into its slot: row blocks of
                # `rows_per_block` rows, block b taken by wavefront b mod (all
                # wavefronts), of 64 threads each.
                n_rows = p["rows"][0]
                keys = np.array([L.fkref_argmax_key(float(v), i) for i, v in enumerate(keyed[:n_rows])],
                                np.uint64)
                rows_per_block = -(-n_rows // p["blocks"])
                waves = launch.threads // 64
                total_waves = launch.groups * waves
                blocks = np.arange(n_rows) // rows_per_block
                group = (blocks % total_waves) // waves
                arg = self.buffers[b["arg"]]
                arg[:] = 0
                np.maximum.at(arg, group, keys)
        elif e == "fk_step_token":
            top = int(self.buffers[b["arg"]][:p["slots"]].max())
            t = 0xFFFFFFFF - (top & 0xFFFFFFFF)
            self.buffers[b["out"]][0] = t
            if p["advance"]:
                self.buffers[b["token"]][0] = t
                pos = self.buffers[b["position"]]
                pos[0] = (int(pos[0]) + p["step"]) % p["context"]
            st = 0
        elif e == "fk_step_store":
            st = L.fkref_step_store(self._p(b["x0"]), self._p(b["x1"]), self._p(b["c0"]), self._p(b["c1"]),
                                    p["n_stores"], p["rope"][0], p["rope"][1], p["kv_heads"], p["head_dim"],
                                    p["length"], p["slots"], p["rotated"], launch.meta["theta"],
                                    int(self.buffers[b["position"]][0]), int(self.buffers[b["slot"]][0]),
                                    p["cache_bf16"])
        elif e == "fk_step_attend":
            # The store the launch may do first, then the attention.
            pos, slot = int(self.buffers[b["position"]][0]), int(self.buffers[b["slot"]][0])
            st = 0
            if p["store"]:
                st = L.fkref_step_store(self._p(b["knew"]), self._p(b["vnew"]), self._p(b["kc"]), self._p(b["vc"]),
                                        2, p["krope"], 0, p["kv_heads"], p["head_dim"], p["length"], p["slots"],
                                        p["rotated"], launch.meta["store_theta"], pos, slot, p["cache_bf16"])
            st = st or L.fkref_step_attend_reach(self._p(b["q"]), self._p(b["kc"]), self._p(b["vc"]),
                                                 self._p(b["partials"]), p["heads"], p["kv_heads"], p["head_dim"],
                                                 p["length"], p["slots"], p["splits"], p["split"], p["rope"],
                                                 p["rotated"], launch.meta["theta"], p["scale"], p["window"], pos,
                                                 slot, self._reach(b, p, pos), p["cache_bf16"])
        elif e == "fk_step_attend_paged":
            pos = int(self.buffers[b["position"]][0])
            kp, vp = self._pool(b["kpool"]), self._pool(b["vpool"])
            st = 0
            if p["store"]:
                st = L.fkref_step_store_paged(self._p(b["knew"]), self._p(b["vnew"]), kp, vp, 2, p["krope"], 0,
                                              p["kv_heads"], p["head_dim"], p["block_size"], self._p(b["table"]),
                                              p["table_len"], p["blocks"], p["rotated"], launch.meta["store_theta"],
                                              pos, p["cache_bf16"])
            st = st or L.fkref_step_attend_paged(self._p(b["q"]), kp, vp, self._p(b["partials"]), p["heads"],
                                                 p["kv_heads"], p["head_dim"], p["block_size"], self._p(b["table"]),
                                                 p["table_len"], p["blocks"], p["splits"], p["split"], p["rope"],
                                                 p["rotated"], launch.meta["theta"], p["scale"], p["window"], pos,
                                                 self._reach(b, p, pos), p["cache_bf16"])
        elif e == "fk_step_store_paged":
            pools = [self._pool(b["p0"]), self._pool(b["p1"]) if b["p1"] else None]
            st = L.fkref_step_store_paged(self._p(b["x0"]), self._p(b["x1"]), pools[0], pools[1], p["n_stores"],
                                          p["rope"][0], p["rope"][1], p["kv_heads"], p["head_dim"], p["block_size"],
                                          self._p(b["table"]), p["table_len"], p["blocks"], p["rotated"],
                                          launch.meta["theta"], int(self.buffers[b["position"]][0]), p["cache_bf16"])
        elif e == "fk_step_attend_wide":
            pos, slot = int(self.buffers[b["position"]][0]), int(self.buffers[b["slot"]][0])
            st = 0
            if p["store"]:
                st = L.fkref_step_store(self._p(b["knew"]), self._p(b["vnew"]), self._p(b["kc"]), self._p(b["vc"]),
                                        2, p["krope"], 0, p["kv_heads"], p["head_dim"], p["length"], p["slots"],
                                        p["rotated"], launch.meta["store_theta"], pos, slot, p["cache_bf16"])
            st = st or L.fkref_step_attend_wide(self._p(b["q"]), self._p(b["kc"]), self._p(b["vc"]),
                                                self._p(b["partials"]), p["heads"], p["kv_heads"], p["head_dim"],
                                                p["length"], p["slots"], p["splits"], p["split"], p["rope"],
                                                p["rotated"], launch.meta["theta"], p["scale"], p["window"], pos,
                                                slot, p["cache_bf16"])
        elif e == "fk_step_combine":
            st = L.fkref_step_combine(self._p(b["partials"]), self._p(b["out"]), p["heads"], p["head_dim"],
                                      p["splits"])
        elif e == "fk_step_argmax":
            self.buffers[b["out"]][0] = L.fkref_argmax(self._p(b["x"]), p["n"])
            st = 0
        elif e == "fk_step_act_mul":
            half = p.get("half", 0)
            if half:
                # segments of 2 half of one row: each element's act·mul as the
                # contiguous form computes it
                a = self.buffers[b["a"]]
                i = np.arange(p["n"])
                at = (i // half) * 2 * half + i % half
                aa, bb = np.ascontiguousarray(a[at]), np.ascontiguousarray(a[at + half])
                y = np.zeros(p["n"], np.float32)
                st = L.fkref_act_mul(aa.ctypes.data, bb.ctypes.data, y.ctypes.data, p["n"], p.get("act", 0))
                self.buffers[b["y"]][:p["n"]] = y
            else:
                off = p.get("b_off", 0)
                bb = self.buffers[b["b"]][off:]
                st = L.fkref_act_mul(self._p(b["a"]), bb.ctypes.data, self._p(b["y"]), p["n"], p.get("act", 0))
        elif e == "fk_rmsnorm_f32":
            st = L.fkref_rmsnorm(self._p(b["x"]), self._p(b["gamma"]) if p["has_gamma"] else None, self._p(b["y"]),
                                 p["rows"], p["width"], p["seg"], p["eps"], p["factor"], launch.threads, 64, 4)
        elif e == "fk_step_route":
            st = L.fkref_route(self._p(b["x"]), self._p(b["scale"]) if p["has_scale"] else None, self._p(b["ids"]),
                               self._p(b["ws"]), p["n"], p["k"], p["has_scale"])
        elif e.startswith("fk_gemv_routed_"):
            wt = e.split("_")[3]
            kind, pool, entry_bytes = self.lowered.constants[b["table"]]
            table, ids = self.buffers[pool], self.buffers[b["ids"]]
            x, y = self.buffers[b["x"]], self.buffers[b["y"]]
            n, k = p["n"], p["k"]
            st = 0
            for r in range(p["ranks"]):
                ent = min(int(ids[r]), p["entries"] - 1)
                w = table.ctypes.data + ent * entry_bytes
                xr = x.ctypes.data + (0 if p["shared"] else r * k * 4)
                yr = y.ctypes.data + r * n * 4
                st = st or L.fkref_gemv(w, TYPE[wt], xr, fkref.F32, yr, None, n, k, 1, 64, 4 if wt == "f32" else 8, 1)
        elif e.startswith("fk_gemv_p4_"):
            # a wavefront a row, packs of 4: the reference GEMV's order at
            # width 64, pack 4, split 1
            wt = e[len("fk_gemv_p4_"):]
            st = L.fkref_gemv(self._p(b["w"]), TYPE[wt], self._p(b["x"]), fkref.F32, self._p(b["y"]), None, p["n"],
                              p["k"], 1, self.width, 4, 1)
        elif e == "fk_step_elementwise":
            # fk_step.h's elementwise operations, each a binary32 operation
            # in the evaluator's order (Eval.hs:336-355, 536-544)
            n, op = p["n"], p["op"]
            a = self.buffers[b["a"]]
            y = self.buffers[b["y"]]
            if op == 0:
                y[:n] = a[:n] + self.buffers[b["b"]][:n]
            elif op == 1:
                y[:n] = a[:n] * self.buffers[b["b"]][0]
            elif op == 2:
                w = p["width"]
                bias, scale = self.buffers[b["b"]][:w], self.buffers[b["c"]][:w]
                f = np.float32(p["factor"])
                y[:n] = ((f * a[:n].reshape(-1, w) - bias) * scale).reshape(-1)
            else:
                wa, wb = p["width"], p["width_b"]
                rows = n // (wa + wb)
                y[:n] = np.concatenate([a[:rows * wa].reshape(rows, wa),
                                        self.buffers[b["b"]][:rows * wb].reshape(rows, wb)], axis=1).reshape(-1)
            st = 0
        elif e.startswith("fk_step_gather_"):
            # each row's tokens' table rows summed from +0 in order, then
            # times the factor, in binary32
            wt = e[len("fk_step_gather_"):]
            t = self.buffers[b["table"]]
            table = (t.astype(np.uint32) << 16).view(np.float32) if wt == "bf16" else t.astype(np.float32)
            rows, width, count = p["rows"], p["width"], p["count"]
            table = table[:p["table_rows"] * width].reshape(p["table_rows"], width)
            toks = np.minimum(self.buffers[b["tokens"]][:rows * count].reshape(rows, count), p["table_rows"] - 1)
            acc = np.zeros((rows, width), np.float32)
            for c in range(count):
                acc = acc + table[toks[:, c]]
            self.buffers[b["y"]][:rows * width] = (acc * np.float32(p["factor"])).reshape(-1)
            st = 0
        elif e == "fk_step_combine_ranks":
            st = L.fkref_combine_ranks(self._p(b["w"]), self._p(b["x"]), self._p(b["res"]), self._p(b["y"]), p["seg"],
                                       p["ranks"], p["residual"])
        else:
            raise ValueError(f"the CPU target has no kernel {e}")
        if st:
            raise ValueError(f"{launch.step} ({e}): the oracle refused it (status {st})")
