"""Runs a lowered plan on the GPU: the executor of a planned step.

Everything a step reads or writes lives in one arena of HBM, allocated once
and resident across steps: the weights, the KV caches, the values steps store
for later steps, the attention partials, the row integers.  Each launch's
kernarg bytes are built once (the buffers never move), so a step is a list of
``fk_launch`` calls, which ``capture`` records into a HIP graph and
``Graph.replay`` runs as one.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from . import kernels as K
from . import runtime
from .lower import Launch, Lowered, rope_table

_NP = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "u32": np.uint32, "u16": np.uint16,
       "u64": np.uint64}
_STRUCTS = {
    "fk_step_store": K.StepStoreParams,
    "fk_step_attend": K.StepAttendParams,
    "fk_step_attend_wide": K.StepAttendParams,
    "fk_step_attend_paged": K.StepAttendPagedParams,
    "fk_step_store_paged": K.StepStorePagedParams,
    "fk_step_combine": K.StepCombineParams,
    "fk_step_argmax": K.CountParams,
    "fk_step_act_mul": K.ActMulParams,
    "fk_step_route": K.RouteParams,
    "fk_rmsnorm_f32": K.RmsNormParams,
    "fk_step_combine_ranks": K.CombineRanksParams,
    "fk_gemv_routed_f16_r1": K.GemvRoutedParams,
    "fk_gemv_routed_f16_r2": K.GemvRoutedParams,
    "fk_gemv_routed_f32_r1": K.GemvRoutedParams,
    "fk_gemv_routed_bf16_r1": K.GemvRoutedParams,
    "fk_gemv_routed_bf16_r2": K.GemvRoutedParams,
    "fk_step_elementwise": K.ElementwiseParams,
    "fk_gemv_p4_f32": K.GemvParams,
    "fk_gemv_p4_f16": K.GemvParams,
    "fk_gemv_p4_bf16": K.GemvParams,
    "fk_step_gather_f32": K.GatherParams,
    "fk_step_gather_f16": K.GatherParams,
    "fk_step_gather_bf16": K.GatherParams,
    "fk_prefill_softcap": K.PrefillSoftcapParams,
    "fk_step_token": K.StepTokenParams,
    "fk_gemm_f16_store": K.GemmParams,
    "fk_gemm_f16_store_keys": K.GemmParams,
    "fk_gemm_f16_add": K.GemmParams,
    "fk_gemm_f16_silu_mul": K.GemmParams,
    "fk_gemm_f16_qkv_rope": K.GemmQkvParams,
    "fk_gemm_f16_qkv_rope_paged": K.GemmQkvPagedParams,
    **{f"{form}{g}": K.PrefillAttendPagedParams for form in ("fk_prefill_attend_paged_g", "fk_prefill_attend_paged_f16_g")
       for g in (1, 2, 4)},
    "fk_prefill_gather": K.PrefillGatherParams,
    "fk_prefill_norm_pack": K.PrefillNormParams,
    **{f"fk_prefill_norm_pack_w{w}": K.PrefillNormParams for w in K.NORM_PACK_HELD},
    "fk_prefill_rope_store": K.PrefillRopeParams,
    "fk_prefill_rope_store_paged": K.PrefillRopePagedParams,
    **{f"{form}{g}": K.PrefillAttendParams for form in ("fk_prefill_attend_g", "fk_prefill_attend_f16_g")
       for g in (1, 2, 4)},
    "fk_prefill_argmax": K.PrefillArgmaxParams,
    "fk_prefill_argmax_keys": K.PrefillArgmaxKeysParams,
    "fk_prefill_land": K.PrefillLandParams,
}


def widen(wtype: str, w) -> np.ndarray:
    """Weights of type `wtype` (bf16 as uint16 bits) as exact f32 values."""
    a = np.asarray(w)
    if wtype == "bf16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def params_struct(launch: Launch) -> ctypes.Structure:
    """The launch's parameter struct from its flat parameters (a paged
    entry's paging fields go to its ``g``, the rest to its inner struct)."""
    cls = K.StepGemvParams if launch.entry.startswith("fk_step_gemv") else _STRUCTS[launch.entry]
    s = cls()
    names = [f[0] for f in cls._fields_]
    inner = None
    if "g" in names:
        inner = getattr(s, names[0])
    paging = {f[0] for f in K.Paging._fields_}
    for name, value in launch.params.items():
        target = s if inner is None else (s.g if name in paging else inner)
        field = getattr(type(target), name, None)
        if field is None:
            raise K.LaunchError(f"{launch.entry}: no parameter {name}")
        if isinstance(value, (list, tuple)):
            arr = getattr(target, name)
            for i, v in enumerate(value):
                arr[i] = v
        else:
            setattr(target, name, value)
    return s


_ELT = {"f32": 4, "f16": 2, "bf16": 2, "u32": 4, "u16": 2, "u64": 8}


def _gemv_needs(launch: Launch) -> dict:
    """Bytes (and element type) each buffer of a GEMV step launch must hold
    for every access its kernel makes: the weights and the gathered tables
    are read as the entry's weight type, the rows as f32."""
    p = launch.params
    _, wt, _, _, _, epi = K.gemv_entry(launch.entry)
    wb = _ELT[wt]
    n, rows, k = p["n_anchors"], p["rows"], p["k"]
    widest = max(rows[:n])
    _, _, _, _, pro, _ = K.gemv_entry(launch.entry)
    src_bytes = k * 4
    if pro == K.PRO_COMBINE:
        src_bytes = (k // p["head_dim"]) * p["splits"] * (p["head_dim"] + 2) * 4
    need = {"src": (src_bytes, "f32"), "src2": ((k + p.get("src2_off", 0)) * 4, "f32"), "gamma": (k * 4, "f32"),
            "table": (p.get("table_rows", 1) * k * wb, wt), "token": (4, "u32"), "res_token": (4, "u32"),
            "res": (widest * 4, "f32"), "res_table": (p.get("table_rows", 1) * widest * wb, wt),
            "epi_out": ((rows[0] if epi in (K.EPI_SILU_MUL, K.EPI_SOFTCAP) else widest) * 4, "f32"),
            "arg": (p.get("arg_slots", 0) * 8, "u64")}
    for j in range(n):
        need[f"w{j}"] = (rows[j] * k * wb, wt)
        need[f"y{j}"] = (rows[j] * 4, "f32")
    return need


def _attend_needs(launch: Launch) -> dict:
    p = launch.params
    d, kv, heads = p["head_dim"], p["kv_heads"], p["heads"]
    cache = "bf16" if p["cache_bf16"] else "f16"
    out = {"q": (heads * d * 4, "f32"), "knew": (kv * d * 4, "f32"), "vnew": (kv * d * 4, "f32"),
           "position": (4, "u32"), "rope": (p["rope_rows"] * p["rotated"] * 8, "f32"),
           "partials": (heads * p["splits"] * (d + 2) * 4, "f32"), "reach": (4, "u32")}
    if launch.entry == "fk_step_attend_paged":
        out.update(kpool=(p["blocks"] * 8, "u64"), vpool=(p["blocks"] * 8, "u64"), table=(p["table_len"] * 4, "u32"))
    else:
        out.update(kc=(p["slots"] * kv * p["length"] * d * 2, cache), vc=(p["slots"] * kv * p["length"] * d * 2, cache),
                   slot=(4, "u32"))
    return out


def check_launch(launch: Launch, specs: dict) -> None:
    """Refuses (LaunchError) a launch whose kernel would dereference a buffer
    it has not bound, whose entry's modes disagree with its parameters, or
    (for the GEMV step and attention families) whose buffers are smaller or of
    another type than what its kernel reads: every check made before a
    launch's kernarg is built.  `specs` maps logical buffers to BufferSpecs."""
    e = launch.entry
    abi = K.ABIS.get(e)
    if abi is None:
        raise K.LaunchError(f"{e}: no such kernel")
    if abi.threads and launch.threads != abi.threads:
        raise K.LaunchError(f"{e} is compiled for {abi.threads} threads, not {launch.threads}")
    extra = set(launch.bind) - set(abi.buffers)
    if extra:
        raise K.LaunchError(f"{e}: binds {sorted(extra)}, which the kernel does not take")
    if e.startswith("fk_step_gemv"):
        _, _, kmax, r, pro, epi = K.gemv_entry(e)
        p = launch.params
        if (p.get("pro_mode"), p.get("epi_mode")) != (pro, epi):
            raise K.LaunchError(f"{e} runs prologue {pro} and epilogue {epi}; its parameters say "
                                f"{p.get('pro_mode')} and {p.get('epi_mode')}")
        if p["k"] > kmax or not 1 <= p["n_anchors"] <= 3:
            raise K.LaunchError(f"{e}: k = {p['k']} past {kmax}, or {p['n_anchors']} anchors")
        if epi == K.EPI_SILU_MUL and (p["n_anchors"] != 2 or p["rows"][0] != p["rows"][1]
                                      or (r == 1 and p["blocks"] != 2 * p["rows"][0])):
            raise K.LaunchError(f"{e}: the SiLU·mul epilogue on anchors {p['rows']}, {p['blocks']} blocks of {r}")
        if epi == K.EPI_SOFTCAP and (p["n_anchors"] != 1 or not 0 < p.get("cap", 0) < float("inf")):
            raise K.LaunchError(f"{e}: a softcap of {p.get('cap')} on {p['n_anchors']} anchors")
        if pro == K.PRO_COMBINE and (not 1 <= p.get("splits", 0) <= K.COMBINE_SPLITS or not p.get("head_dim")
                                     or p["head_dim"] % 4 or p["k"] % p["head_dim"]):
            raise K.LaunchError(f"{e}: a combine of {p.get('splits')} splits of heads of {p.get('head_dim')}")
        if p.get("act", 0) not in (K.ACT_SILU, K.ACT_GELU_TANH) or p.get("src2_off", 0) % 4:
            raise K.LaunchError(f"{e}: activation {p.get('act')}, second row at {p.get('src2_off')}")
    reads = K.launch_reads(e, launch.params)
    unbound = sorted(b for b in reads if launch.bind.get(b) is None)
    if unbound:
        raise K.LaunchError(f"{e}: reads or writes {unbound}, which the launch leaves unbound")
    needs = _gemv_needs(launch) if e.startswith("fk_step_gemv") else \
        _attend_needs(launch) if e in ("fk_step_attend", "fk_step_attend_wide", "fk_step_attend_paged") else {}
    for b in sorted(reads & set(needs)):
        spec = specs[launch.bind[b]]
        nbytes, dtype = needs[b]
        if spec.dtype != dtype:
            raise K.LaunchError(f"{e}: {b} is {spec.name} of {spec.dtype}; the kernel reads {dtype}")
        if spec.nbytes < nbytes:
            raise K.LaunchError(f"{e}: {b} is {spec.name}, {spec.nbytes} bytes; the kernel touches {nbytes}")
    arg = launch.bind.get("arg")
    if arg is not None and launch.params.get("arg_slots", 0) > specs[arg].count:
        raise K.LaunchError(f"{e}: {launch.params['arg_slots']} argmax slots in a buffer of {specs[arg].count}")


class Engine:
    def __init__(self, device: runtime.Device, ks: K.Kernels, lowered: Lowered, extra_bytes: int = 0):
        self.device = device
        self.kernels = ks
        self.lowered = lowered
        specs = lowered.buffers
        total = sum((spec.nbytes + 255) // 256 * 256 for spec in specs.values()) + 4096 + extra_bytes
        self.arena = device.arena(total)
        self.buffers: dict[str, runtime.Buffer] = {}
        for name, spec in specs.items():
            self.buffers[name] = self.arena.alloc(spec.nbytes, 256)
        for name, what in lowered.constants.items():
            if what[0] == "rope":
                self.write(name, rope_table(*what[1:]))
            elif what[0] == "zero":
                self.zero(name)
            elif what[0] == "ones":
                self.write(name, np.ones(specs[name].count, np.float32))
            elif what[0] == "addresses":
                # a paged pool's blocks, in order in its buffer
                pool, block_bytes = self.buffers[what[1]], what[2]
                self.write(name, pool.ptr + block_bytes * np.arange(specs[name].count, dtype=np.uint64))
            else:
                raise ValueError(f"{name}: no constant {what[0]}")
        # The step's launches in a native launch table: each checked once
        # (here, against the buffers' types; in the library, against the
        # kernel's manifest) and kept with its kernarg.
        self.table = runtime.Table(device)
        for launch in lowered.launches:
            self._add(launch)
        self._advance: dict = {}

    def _add(self, launch: Launch) -> int:
        check_launch(launch, self.lowered.buffers)
        spans = []
        for b in K.ABIS[launch.entry].buffers:
            name = launch.bind.get(b)
            spans.append((0, 0) if name is None else (self.buffers[name].ptr, self.lowered.buffers[name].nbytes))
        return self.table.add(self.kernels.fn(launch.entry), launch.groups, launch.threads, launch.lds_bytes, spans,
                              params_struct(launch))

    # State -------------------------------------------------------------------

    def spec(self, name: str):
        return self.lowered.buffers[name]

    def write(self, name: str, values: np.ndarray) -> None:
        spec = self.spec(name)
        a = np.ascontiguousarray(values, dtype=_NP[spec.dtype]).reshape(-1)
        if a.size != spec.count:
            raise ValueError(f"{name}: {a.size} elements for a buffer of {spec.count}")
        self.buffers[name].write(a)

    def write_weights(self, weights: dict) -> None:
        """Host weights by source name (bf16 ones as their uint16 bits) into
        the buffers the step reads them from: as given, and widened exactly to
        f32 where the lowering keeps an f32 copy (an RMSNorm's gains)."""
        for src, w in weights.items():
            if f"weight:{src}" in self.lowered.buffers:
                self.write(f"weight:{src}", w)
            if f"table:{src}" in self.lowered.buffers:  # a table's entries, in order
                self.write(f"table:{src}", w)
            wide = f"widen:{src}"
            if wide in self.lowered.buffers:
                self.write(wide, widen(self.lowered.program.source_named(src).kind.type, w))

    def read(self, name: str) -> np.ndarray:
        spec = self.spec(name)
        return self.buffers[name].read(_NP[spec.dtype], spec.count)

    def set_ints(self, source: str, values, bound: Optional[int] = None) -> None:
        a = np.asarray(values, dtype=np.uint32).reshape(-1)
        if bound is not None and np.any(a >= bound):
            raise ValueError(f"{source}: {a.tolist()} not below its bound {bound}")
        self.write(f"ints:{source}", a)

    def init_normal(self, name: str, seed: int, std: float) -> None:
        """Synthetic values on the device: std * N(0, 1), SplitMix64 + Box-Muller."""
        spec = self.spec(name)
        codes = {"f32": 0, "f16": 1, "bf16": 2}
        if spec.dtype not in codes:
            raise ValueError(f"{name}: normals of {spec.dtype}")
        buf = self.buffers[name]
        groups = min(max(spec.count // 256, 1), 65536)
        self.kernels.launch("fk_init_normal", groups, 256, {"dst": buf.ptr},
                            K.InitNormalParams(spec.count, seed & 0xFFFFFFFFFFFFFFFF, std, codes[spec.dtype]))

    def zero(self, name: str) -> None:
        self.kernels.fill_u32(self.buffers[name], 0, (self.spec(name).nbytes + 3) // 4)

    # Running -----------------------------------------------------------------

    def enqueue(self, stream: runtime.Stream | None = None, only: Optional[list] = None,
                advance: Optional[dict] = None) -> None:
        """Queues every launch of the step (or those at the indices `only`),
        in plan order; with `advance`, then the next step's token and
        position (see ``enqueue_advance``)."""
        n = len(self.lowered.launches)
        picks = list(range(n)) if only is None else list(only)
        last = n - 1
        folded = advance is not None and self.lowered.launches[last].entry == "fk_step_token" and \
            (not picks or picks[-1] == last)
        if folded:
            picks[-1] = self._advance_index(**advance)
        # runs of consecutive indices go to the table in one call each
        i = 0
        while i < len(picks):
            j = i
            while j + 1 < len(picks) and picks[j + 1] == picks[j] + 1:
                j += 1
            self.table.enqueue(picks[i], j - i + 1, stream)
            i = j + 1
        if advance is not None and not folded:
            self.enqueue_advance(stream=stream, **advance)

    def _advance_index(self, token_out: str, token_in: str, position: str, context: int, step: int = 1) -> int:
        """The token launch that also advances (the greedy token it makes is
        the next step's token, the position `step` on), added to the table
        once per set of arguments."""
        key = (token_out, token_in, position, context, step)
        if key not in self._advance:
            launch = self.lowered.launches[-1]
            if launch.bind["out"] != token_out:
                raise ValueError(f"the step's token is {launch.bind['out']}, not {token_out}")
            bind = dict(launch.bind, token=token_in, position=position)
            params = dict(launch.params, context=context, step=step, advance=1)
            self._advance[key] = self._add(Launch(launch.step, launch.entry, launch.groups, launch.threads, bind,
                                                  params))
        return self._advance[key]

    def enqueue_advance(self, token_out: str, token_in: str, position: str, context: int, step: int = 1,
                        stream: runtime.Stream | None = None) -> None:
        """The next decode step's inputs on the device: the greedy token in,
        the position `step` on."""
        self.kernels.launch("fk_step_advance", 1, 64,
                            {"next_token": self.buffers[token_out].ptr, "token": self.buffers[token_in].ptr,
                             "position": self.buffers[position].ptr},
                            K.AdvanceParams(context, step), stream)

    def capture(self, advance: Optional[dict] = None, stream: runtime.Stream | None = None,
                only: Optional[list] = None) -> runtime.Graph:
        """A graph of the step's launches (or those at the indices `only`; and
        the advance, if given), to replay."""
        with self.device.capture(stream) as out:
            self.enqueue(stream, only, advance)
        return out[0]

    def close(self) -> None:
        self.table.destroy()
        self.arena.destroy()
