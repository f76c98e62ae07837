"""Decode throughput of the planned 1B-class f16 step on one MI355X.

The workload: the decoder step program (d_model 2048, 16 layers, 32 query
heads and 8 KV heads of 64, FFN 8192 SiLU-gated, vocab 32000, a KV ring of
4096 positions, batch 1), gated, planned, lowered to the gfx950 step kernels
and resident in HBM — weights, KV caches, values and partials — with a HIP
graph of the whole step (every launch, then the device-side advance of the
greedy token).  Each timed step decodes one token at position 4095, so its
attention reads all 4096 cached positions of every layer.  Weights are
N(0, 0.02) and caches N(0, 1), generated on the device.

Prints one JSON line: tokens/s (``value``), the step's algorithmic HBM
bytes and achieved GB/s against 8 TB/s, the roofline of the kernel with the
largest share of the step (its launches replayed alone, timed with HIP
events on the stream they run on), and the CPU baseline: the oracle's CPU
target (the C restatement of the reference CPU target's execution model,
SIMD width 32, one thread) timed on a bounded sample of the same step.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--eager]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tokens/sec + achieved HBM GB/s (% of ~8 TB/s) for planned step, 1 GPU"
HBM_PEAK_GBPS = 8000.0
POSITION = 4095


def _plan_options():
    from furykernel_amd.program.plan import PlanOptions

    # The SiLU·mul stored once (folded into the gate/up step) rather than
    # recomputed by every threadgroup of the down projection.
    return PlanOptions(store_gelus=True)


PLAN = None


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=20, help="replays of each kernel's launches for its roofline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU time to spend on the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--untuned", action="store_true",
                    help="shape the GEMV steps by the lowering's defaults, not the committed selections")
    ap.add_argument("--eager", action="store_true",
                    help="queue each step's launches on the stream instead of replaying a HIP graph")
    ap.add_argument("--workload", choices=("decode", "prefill", "kernels"), default="decode",
                    help="decode (the headline metric) or the 1B prefill of 4 x 2048 rows")
    ap.add_argument("--paged", action="store_true",
                    help="prefill workload: the KV caches as paged pools (blocks of 64 positions, each sequence's "
                         "rows through a scrambled block table) instead of rings")
    ap.add_argument("--calibrate", action="store_true",
                    help="only read and write 1 GiB with the streaming kernels (the known sizes that scale the "
                         "HBM counters FETCH_SIZE and WRITE_SIZE)")
    return ap.parse_args()


CALIBRATE_BYTES = 1 << 30


def calibrate() -> int:
    """Three fills (1 GiB written) and three streaming reads (1 GiB read) of one
    buffer, each its own dispatch: what FETCH_SIZE and WRITE_SIZE count for a
    known size, per dispatch."""
    from furykernel_amd import kernels, runtime

    dev = runtime.Device(0)
    ks = kernels.Kernels(dev)
    buf = dev.alloc(CALIBRATE_BYTES)
    out = dev.alloc(1 << 20)
    for _ in range(3):
        ks.fill_u32(buf, 0x3C003C00)
    for _ in range(3):
        ks.stream_read(buf, out, 4096)
    dev.sync()
    print(json.dumps({"calibrate": {"fk_fill_u32": {"dispatches": 3, "bytes_written": CALIBRATE_BYTES},
                                    "fk_stream_read": {"dispatches": 3, "bytes_read": CALIBRATE_BYTES}}}), flush=True)
    buf.free()
    out.free()
    dev.close()
    return 0


def log(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def lowered_for(dims, layers=None):
    from furykernel_amd.lower import lower_plan
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import decoder_step
    from furykernel_amd.program.plan import plan

    checked = check_program(decoder_step(dims, embed=True, layers=layers))
    return lower_plan(checked, plan(_plan_options(), checked))


def kernel_table(session, reps: int, eager: bool) -> dict:
    """Each kernel entry's launches of the step, alone and in plan order (a
    graph of them, or queued eagerly), run `reps` times between two HIP
    events on their stream: the average launch duration (consecutive
    launches, so the gap between dispatches is inside it) and the
    algorithmic bytes per launch.  An entry with fewer than 16 launches a
    step has them repeated to at least 16 in its graph, so that a graph
    launch's own cost is not counted against one or two kernels."""
    from furykernel_amd.traffic import launch_bytes

    dev, eng, low = session.device, session.engine, session.lowered
    by_entry: dict = {}
    for i, launch in enumerate(low.launches):
        by_entry.setdefault(launch.entry, []).append(i)
    table = {}
    start, end = dev.event(), dev.event()
    for entry, idx in by_entry.items():
        picks = idx * max(1, -(-16 // len(idx)))
        if eager:
            run = lambda: eng.enqueue(only=picks)  # noqa: E731
        else:
            g = eng.capture(only=picks)
            run = g.replay
        run()
        dev.sync()
        start.record()
        for _ in range(reps):
            run()
        end.record()
        end.synchronize()
        if not eager:
            g.destroy()
        avg_us = start.elapsed_ms(end) * 1e3 / (reps * len(picks))
        nbytes = sum(launch_bytes(low, low.launches[i], POSITION) for i in idx) / len(idx)
        table[entry] = {"launches": len(idx), "avg_us": round(avg_us, 3), "bytes_per_launch": int(nbytes),
                        "gbps": round(nbytes / avg_us / 1e3, 1), "us_per_step": round(avg_us * len(idx), 2)}
    return table


TRAFFIC_PROFILE = ROOT / "profiles" / "traffic_decode_1b_f16.md"
PREFILL_TRAFFIC_PROFILE = ROOT / "profiles" / "traffic_prefill_1b_f16.md"


def measured_traffic(entry: str, profile: Path = TRAFFIC_PROFILE):
    """HBM bytes a launch of `entry` moves, as the committed rocprofv3 counter
    runs measured them (FETCH_SIZE and WRITE_SIZE, each scaled by what it
    reads for a copy of known size); None if the profile has no row for it."""
    if not profile.exists():
        return None
    for line in profile.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and cells[0] == entry:
            return int(cells[4])
    return None


def cpu_baseline(dims, seconds: float) -> dict:
    """The oracle's CPU target (width 32, one thread) on layer 0's launches and
    the head's, repeated for about `seconds`; a token costs the layers' launches
    once per layer and the head's once."""
    import numpy as np

    from furykernel_amd.lower import rope_table
    from oracle import fkref
    from oracle.cpu_target import CpuTarget

    one = lowered_for(dims, layers=1)
    per_layer = len(lowered_for(dims, layers=2).launches) - len(one.launches)
    cpu = CpuTarget(one, 32)
    rng = np.random.default_rng(2026)
    block = rng.standard_normal(1 << 20).astype(np.float32)
    for name, spec in one.buffers.items():
        buf = cpu.buffers[name]
        if name.startswith("weight:"):
            buf[:] = 1 if spec.count == dims.d_model else np.resize(block * np.float32(0.02), spec.count)
        elif name.startswith("cache:"):
            buf[:] = np.resize(block, spec.count)
    for name, what in one.constants.items():
        if what[0] == "rope":
            cpu.write(name, rope_table(*what[1:]))
    cpu.write("ints:position", [POSITION])
    cpu.write("ints:tokens", [7])
    layer, head = one.launches[:per_layer], one.launches[per_layer:]

    def sample(threads: int, budget: float):
        fkref.lib().fkref_set_threads(threads)
        t_layer = t_head = 0.0
        reps = 0
        while reps == 0 or t_layer + t_head < budget:
            t0 = time.perf_counter()
            for launch in layer:
                cpu.run_launch(launch)
            t1 = time.perf_counter()
            for launch in head:
                cpu.run_launch(launch)
            t_head += time.perf_counter() - t1
            t_layer += t1 - t0
            reps += 1
        fkref.lib().fkref_set_threads(1)
        return (t_layer * dims.layers + t_head) / reps, reps, t_layer + t_head

    # One thread (the CPU target: threadgroups one after another), then the
    # GEMVs' rows spread over the host's cores (the box's share of them).
    per_token, reps, spent = sample(1, seconds)
    cores = max(1, min(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)), os.cpu_count() or 1))
    per_token_all, reps_all, spent_all = sample(cores, seconds / 2)
    return {"value": round(1.0 / per_token, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"layer 0's {len(layer)} launches and the head's {len(head)} of the same step at position "
                      f"{POSITION}, run {reps} times ({spent:.1f} s); a token = {dims.layers} x layer + head",
            "host_cpus": os.cpu_count(),
            "omp": {"value": round(1.0 / per_token_all, 4), "unit": "tokens/s", "cores": cores, "kind": "port",
                    "sample": f"the same sample with the GEMVs' rows spread over {cores} threads (each row's "
                              f"arithmetic unchanged), run {reps_all} times ({spent_all:.1f} s)"}}


MFMA_PEAK_TFLOPS = 2500.0
PREFILL_METRIC = "prefill tokens/sec + MFMA utilization (% of 2.5 PFLOP/s f16 dense), 1 GPU"
PREFILL_SEQS, PREFILL_ROWS = 4, 2048


def launch_flops(low, launch) -> float:
    """Matrix-core arithmetic of a launch: 2 m k n for a GEMM (n the gate and
    up columns together for SiLU·mul); for the attention, the causal
    QKᵀ and PV products its rows' positions call for (2 · 2 · 64 per
    query head and attended position)."""
    p = launch.params
    if launch.entry.startswith("fk_gemm_f16_"):
        n = 2 * p["ldc"][0] if launch.entry.endswith("silu_mul") else p["first_col"][p["n_anchors"]]
        return 2.0 * p["m"] * p["k"] * n
    if launch.entry.startswith("fk_prefill_attend"):
        per_seq = PREFILL_ROWS * (PREFILL_ROWS + 1) / 2
        return 2.0 * 2.0 * 64 * p["heads"] * per_seq * (p["rows"] / PREFILL_ROWS)
    return 0.0


def prefill_cpu_baseline(dims, seconds: float, rows: int = 64) -> dict:
    """The oracle (the vectorised binary64 evaluator, numpy on the host's
    cores) on one layer of the same decoder program and `rows` rows of one
    sequence, with the head, repeated for about `seconds`; a token costs that
    layer 16 times, the embedding and the head once."""
    import numpy as np

    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import decoder_step
    from oracle.eval import Bindings, evaluate_fast

    checked = check_program(decoder_step(dims, "prefill", True, 1, position_bound=rows))
    rng = np.random.default_rng(5)
    weights = {}
    for src in checked.program.sources:
        if type(src.kind).__name__ == "SWeight":
            d = src.kind.dims
            weights[src.name] = np.ones(d[0]) if len(d) == 1 else rng.standard_normal(d) * 0.02
    caches = {}
    for src in checked.program.sources:
        if type(src.kind).__name__ == "SCache":
            lay = src.kind.layout
            caches[src.name] = {0: np.zeros(lay.kv_heads * lay.length * lay.head_dim)}
    b = Bindings(rows, weights=weights, caches=caches,
                 row_ints={"tokens": rng.integers(0, dims.vocab, (rows, 1)), "position": np.arange(rows)[:, None],
                           "slot": np.zeros((rows, 1), np.int64)})
    runs = 0
    t0 = time.perf_counter()
    while runs == 0 or time.perf_counter() - t0 < seconds:
        evaluate_fast(checked, b)
        runs += 1
    total = time.perf_counter() - t0
    one = total / runs
    # the head and embedding share of the one-layer run, measured alone
    b0 = time.perf_counter()
    x = rng.standard_normal((rows, dims.d_model))
    _ = x @ weights["lm_head"].T
    head = time.perf_counter() - b0
    per_token = ((one - head) * dims.layers + head) / rows
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(1.0 / per_token, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the binary64 evaluator (oracle/eval.py evaluate_fast, numpy) on layer 0 of the 1B prefill "
                      f"program for {rows} rows of one sequence with the head, {runs} runs in {total:.1f} s; the "
                      f"layer's time counted {dims.layers} times a token"}


def main_prefill(args) -> int:
    import numpy as np

    from furykernel_amd import kernels, runtime
    from furykernel_amd.prefill import PrefillSession
    from furykernel_amd.program.decoder import ONE_B_PREFILL as D

    dev = runtime.Device(0)
    ks = kernels.Kernels(dev)
    paging = (64, PREFILL_SEQS * D.context // 64) if args.paged else None
    s = PrefillSession(dev, ks, D, PREFILL_SEQS, PREFILL_ROWS, paging=paging)
    rows = s.rows
    s.init_synthetic()
    s.set_tokens(np.random.default_rng(3).integers(0, D.vocab, rows))
    low = s.lowered
    log(f"prefill of {PREFILL_SEQS} x {PREFILL_ROWS} rows: {len(low.launches)} launches in one graph")
    graph = s.graph()
    for _ in range(args.warmup):
        graph.replay()
    dev.sync()
    start, end = dev.event(), dev.event()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        graph.replay()
    end.record()
    dev.sync()
    elapsed = time.perf_counter() - t0
    graph.destroy()
    ms = elapsed * 1e3 / args.steps
    flops = sum(launch_flops(low, l) for l in low.launches)
    log(f"{args.steps} timed prefills: {ms:.3f} ms each, {flops / 1e12:.2f} TFLOP")

    by_entry: dict = {}
    for i, launch in enumerate(low.launches):
        by_entry.setdefault(launch.entry, []).append(i)
    table = {}
    for entry, idx in by_entry.items():
        g = s.engine.capture(only=idx)
        g.replay()
        dev.sync()
        start.record()
        for _ in range(args.kernel_reps):
            g.replay()
        end.record()
        end.synchronize()
        g.destroy()
        avg_us = start.elapsed_ms(end) * 1e3 / (args.kernel_reps * len(idx))
        fl = sum(launch_flops(low, low.launches[i]) for i in idx) / len(idx)
        row = {"launches": len(idx), "avg_us": round(avg_us, 2), "us_per_prefill": round(avg_us * len(idx), 1)}
        if fl:
            row.update(flops_per_launch=fl, tflops=round(fl / avg_us / 1e6, 1))
        table[entry] = row
        log(f"{entry}: {len(idx)} launches, {avg_us:.1f} us a launch" +
            (f", {fl / avg_us / 1e6:.1f} TFLOP/s" if fl else ""))
    gemms = {e: r for e, r in table.items() if "tflops" in r}
    dominant = max(gemms, key=lambda e: gemms[e]["us_per_prefill"])
    dom = table[dominant]
    tflops = flops / (ms * 1e-3) / 1e12
    line = {
        "metric": PREFILL_METRIC,
        "value": round(rows / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: weights N(0, 0.02) (norm gains 1) generated on the device, random tokens",
        "config": {"workload": "1B-class f16 prefill via the planner: 4 sequences x 2048 rows (positions 0..2047) "
                               + ("into a paged pool of 256 blocks of 64 positions through scrambled block tables"
                                  if args.paged else "into 4 ring slots of 4096")
                               + ", logits and greedy token for every row",
                   "d_model": D.d_model, "layers": D.layers, "heads": D.heads, "kv_heads": D.kv_heads,
                   "head_dim": D.head_dim, "ffn": D.ffn, "vocab": D.vocab, "kv_length": D.context,
                   "rows": rows, "launches": len(low.launches), "launch": "one HIP graph per prefill"},
        "mfma": {"flops_per_prefill": flops, "achieved_tflops": round(tflops, 1),
                 "frac_of_peak": round(tflops / MFMA_PEAK_TFLOPS, 4), "peak_tflops": MFMA_PEAK_TFLOPS},
        "roofline": {"kernel": dominant, "bound": "mfma", "achieved": dom["tflops"], "peak": MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(dom["tflops"] / MFMA_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(dominant, PREFILL_TRAFFIC_PROFILE),
                     "traffic_source": "read from profiles/traffic_prefill_1b_f16.md (the committed rocprofv3 "
                                       "FETCH_SIZE and WRITE_SIZE runs of this workload: bytes leaving the L2s, "
                                       "which the memory-side cache may serve), not measured in this run",
                     "avg_launch_us": dom["avg_us"], "flops_per_launch": dom["flops_per_launch"],
                     "launches_per_step": dom["launches"]},
        "kernels": table,
    }
    s.close()
    dev.close()
    line["cpu_baseline"] = None if args.no_cpu_baseline else prefill_cpu_baseline(D, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


KERNELS_METRIC = "standalone kernels: achieved HBM GB/s (% of ~8 TB/s), 1 GPU"
COPY_BYTES = 512 << 20   # inputs a kernel's launches cycle through: twice the 256 MB memory-side cache


def gemv_variants(wtype: str, n: int, k: int) -> list:
    """The (rows a wavefront, threads) the committed selection picks for the
    standalone GEMV class, or every rows a wavefront at 256 threads."""
    from furykernel_amd import tuning
    pick = tuning.gemv_pick(wtype, n, k)
    log(f"gemv_{wtype} n{n}_k{k}: " + (f"the committed selection's r{pick[0]}_t{pick[1]}" if pick else
                                       "no valid committed selection; every rows a wavefront"))
    return [pick] if pick else [(r, 256) for r in (1, 2, 4)]


def main_kernels(args) -> int:
    """The standalone kernels at their configurations' sizes: f32 matvec
    W[4096 × 4096]·x, RMSNorm and row softmax over [64 × 4096] f32, and the
    int8 weight-only matvec W[8192 × 8192] with per-row f32 scales and f16 x.
    Each launch of a kernel reads its own copy of the inputs — 512 MB of
    copies, twice the memory-side cache, so that every launch reads HBM —
    and the launches run back to back in one HIP graph, timed with HIP
    events on its stream: the average launch, gaps between dispatches
    included (with --eager the launches are queued one by one instead, so
    the average also holds each launch's host cost).  Algorithmic bytes: every input element read once and every
    output written once.  The CPU baseline: the oracle's C GEMV (the
    reference GEMV's order, one thread) on the f32 matvec."""
    import numpy as np

    from furykernel_amd import kernels, runtime

    dev = runtime.Device(0)
    ks = kernels.Kernels(dev)

    def normal(buf, seed, f16):
        cnt = buf.size // (2 if f16 else 4)
        ks.launch("fk_init_normal", min(max(cnt // 256, 1), 65536), 256, {"dst": buf.ptr},
                  kernels.InitNormalParams(cnt, seed, 1.0, 1 if f16 else 0))

    def timed(launches: list, reps: int) -> float:
        if args.eager:   # queued one by one, each launch a dispatch of its own in a kernel trace
            def replay():
                for run in launches:
                    run()
            finish = None
        else:
            with dev.capture() as g:
                for run in launches:
                    run()
            replay, finish = g[0].replay, g[0].destroy
        replay()
        dev.sync()
        start, end = dev.event(), dev.event()
        start.record()
        for _ in range(reps):
            replay()
        end.record()
        end.synchronize()
        if finish is not None:
            finish()
        return start.elapsed_ms(end) * 1e3 / (reps * len(launches))

    table = {}
    bufs = []

    def copies_of(nbytes: int) -> int:
        return max(2, -(-COPY_BYTES // nbytes))

    # f32 matvec 4096 × 4096: the variant of rows a wavefront with the best rate.
    n = k = 4096
    cw = copies_of(n * k * 4)
    ws = [dev.alloc(n * k * 4) for _ in range(cw)]
    x, y = dev.alloc(k * 4), dev.alloc(n * 4)
    for i, w in enumerate(ws):
        normal(w, 100 + i, False)
    normal(x, 99, False)
    bufs += ws + [x, y]
    nbytes = n * k * 4 + k * 4 + n * 4
    best = None
    for r, t in gemv_variants("f32", n, k):
        us = timed([lambda w=w, r=r, t=t: ks.gemv(w, x, y, n, k, "f32", rows_per_wave=r, threads=t) for w in ws], 20)
        log(f"fk_gemv_f32_f32_r{r} 4096 x 4096, {t} threads: {us:.2f} us a launch, {nbytes / us / 1e3:.1f} GB/s")
        if best is None or us < best[1]:
            best = (f"fk_gemv_f32_f32_r{r}", us)
    table["matvec_f32_4096x4096"] = {"kernel": best[0], "avg_us": round(best[1], 3), "bytes": nbytes,
                                     "gbps": round(nbytes / best[1] / 1e3, 1),
                                     "frac": round(nbytes / best[1] / 1e3 / HBM_PEAK_GBPS, 4)}

    # RMSNorm and softmax over 64 × 4096 f32.
    rows, width = 64, 4096
    cr = copies_of(rows * width * 4)
    xs = [dev.alloc(rows * width * 4) for _ in range(cr)]
    gamma, out = dev.alloc(width * 4), dev.alloc(rows * width * 4)
    for i, b in enumerate(xs):
        normal(b, 300 + i, False)
    normal(gamma, 298, False)
    bufs += xs + [gamma, out]
    for name, entry, run, nb in (
            ("rmsnorm_64x4096", "fk_rmsnorm_f32", lambda b, t: ks.rmsnorm(b, gamma, out, rows, width, threads=t),
             2 * rows * width * 4 + width * 4),
            ("softmax_64x4096", "fk_softmax_f32", lambda b, t: ks.softmax(b, out, rows, width, threads=t),
             2 * rows * width * 4)):
        best = None
        for t in (256, 512, 1024):
            us = timed([lambda b=b, t=t: run(b, t) for b in xs], 20)
            log(f"{entry} 64 x 4096, {t} threads a row: {us:.2f} us a launch, {nb / us / 1e3:.1f} GB/s")
            if best is None or us < best[1]:
                best = (t, us)
        t, us = best
        table[name] = {"kernel": entry, "threads": t, "avg_us": round(us, 3), "bytes": nb,
                       "gbps": round(nb / us / 1e3, 1), "frac": round(nb / us / 1e3 / HBM_PEAK_GBPS, 4)}

    # int8 weight-only matvec 8192 × 8192.
    n = k = 8192
    ci = copies_of(n * k)
    wi = [dev.alloc(n * k) for _ in range(ci)]
    scale, xh, yi = dev.alloc(n * 4), dev.alloc(k * 2), dev.alloc(n * 4)
    for i, w in enumerate(wi):
        ks.fill_u32(w, 0x05fb11ef ^ (i * 0x01010101), n * k // 4)
    normal(scale, 297, False)
    normal(xh, 296, True)
    bufs += wi + [scale, xh, yi]
    nbytes = n * k + n * 4 + k * 2 + n * 4
    best = None
    for r, t in gemv_variants("i8", n, k):
        us = timed([lambda w=w, r=r, t=t: ks.gemv(w, xh, yi, n, k, "i8", rows_per_wave=r, threads=t, scale=scale)
                    for w in wi], 20)
        log(f"fk_gemv_i8_f16_r{r} 8192 x 8192, {t} threads: {us:.2f} us a launch, {nbytes / us / 1e3:.1f} GB/s")
        if best is None or us < best[1]:
            best = (f"fk_gemv_i8_f16_r{r}", us)
    table["matvec_i8_8192x8192"] = {"kernel": best[0], "avg_us": round(best[1], 3), "bytes": nbytes,
                                    "gbps": round(nbytes / best[1] / 1e3, 1),
                                    "frac": round(nbytes / best[1] / 1e3 / HBM_PEAK_GBPS, 4)}
    for b in bufs:
        b.free()
    table.update(ir_gemv_table(dev, timed, copies_of))
    table.update(paged_routed_table(dev, ks, args.eager))

    head = table["matvec_f32_4096x4096"]
    line = {
        "metric": KERNELS_METRIC, "value": head["gbps"], "unit": "GB/s", "n_gpus": 1, "steps": 20, "warmup": 1,
        "ms_per_step": round(head["avg_us"] / 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: N(0, 1) matrices, vectors and rows generated on the device; int8 weights a fixed "
                "byte pattern",
        "config": {"workload": "standalone kernels: f32 matvec 4096 x 4096, RMSNorm and row softmax over 64 x 4096 "
                               "f32, int8 weight-only matvec 8192 x 8192 (per-row scales, f16 x), and the IR "
                               "target's bf16 GEMV family (lowered to HIP, compiled by hipRTC) at 8192 x 2048 and "
                               "2048 x 8192; each launch on its own copy of the inputs (512 MB of copies)"},
        "roofline": {"kernel": head["kernel"], "bound": "hbm", "achieved": head["gbps"], "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": head["frac"], "traffic": None, "avg_launch_us": head["avg_us"],
                     "bytes_per_launch": head["bytes"]},
        "kernels": table,
        "cpu_baseline": None if args.no_cpu_baseline else matvec_cpu_baseline(args.cpu_seconds),
    }
    print(json.dumps(line), flush=True)
    return 0


# The IR target's bf16 GEMV family at the 1B decode's FFN shapes: a few
# variants each (rows a SIMD group, threads, pack, split-K).
# The variants of the IR GEMV family timed a shape: the fastest of a sweep of
# rows a SIMD group 1-8, threads 256-1024 and splits 1-16 on the MI355X, and
# their neighbours.
IR_GEMV = {(8192, 2048): [(2, 256, 8, 4), (4, 256, 8, 4), (2, 512, 8, 4), (2, 1024, 8, 4)],
           (2048, 8192): [(4, 1024, 8, 16), (2, 1024, 8, 16), (2, 1024, 8, 4), (2, 256, 8, 4)]}


def ir_gemv_table(dev, timed, copies_of) -> dict:
    """The reference's bf16 GEMV family (test/Test/FuryKernel/Gemv.hs) built
    as IR, lowered by the MI355X backend to HIP and compiled by hipRTC: each
    shape's best variant, each launch on its own copy of W (bf16 N(0, 1)
    halves' bits), algorithmic bytes W + x + y."""
    import numpy as np

    from furykernel_amd.ir import rocm
    from furykernel_amd.ir.build import ROCM
    from furykernel_amd.ir.gate import check
    from furykernel_amd.ir.gemv import GemvShape, GemvVariant, gemv
    from furykernel_amd.ir.runtime import Unit

    kernels = []
    for (n, k), vs in IR_GEMV.items():
        for r, t, p, s in vs:
            name = f"ir_gemv_bf16_n{n}_k{k}_r{r}_t{t}_p{p}_s{s}"
            kern, problems = gemv(ROCM, name, GemvShape(n, k, 1), GemvVariant(r, t, p, s))
            assert not problems, problems
            kernels.append(((n, k), name, check(kern, ROCM)))
    unit = Unit(dev, rocm.lower([c for _, _, c in kernels]), "ir_gemv.hip")
    rng = np.random.default_rng(11)
    out = {}
    for (n, k) in IR_GEMV:
        wbits = (rng.standard_normal(n * k).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        ws = [dev.upload(wbits) for _ in range(copies_of(n * k * 2))]
        x = dev.upload((rng.standard_normal(k).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
        y = dev.alloc(n * 2)
        nbytes = n * k * 2 + k * 2 + n * 2
        best = None
        for shape, name, _ in kernels:
            if shape != (n, k):
                continue
            us = timed([lambda w=w, name=name: unit.launch(name, {}, {"x": x, "w": w, "y": y}) for w in ws], 20)
            log(f"{name}: {us:.2f} us a launch, {nbytes / us / 1e3:.1f} GB/s")
            if best is None or us < best[1]:
                best = (name, us)
        out[f"ir_gemv_bf16_{n}x{k}"] = {"kernel": best[0], "avg_us": round(best[1], 3), "bytes": nbytes,
                                         "gbps": round(nbytes / best[1] / 1e3, 1),
                                         "frac": round(nbytes / best[1] / 1e3 / HBM_PEAK_GBPS, 4)}
        for b in ws + [x, y]:
            b.free()
    return out


def paged_routed_table(dev, ks, eager: bool = False, reps: int = 50) -> dict:
    """Decode attention at the 1B step's shape (32 heads over 8, d 64, the
    row at position 4095 of 4096) over a ring and over a paged pool (64
    blocks of 64 positions through a scrambled block table, pool of 80
    blocks), and a routed-experts step (hidden 2048, 16 experts of FFN 1024,
    top 2, expert scales): each planned step lowered, its launches captured
    as one HIP graph (the step repeated to at least 16 launches) and
    replayed `reps` times between HIP events (with `eager`, the step's
    launches queued one by one `reps` times, each a dispatch of its own in a
    kernel trace).
    Algorithmic bytes: the K and V rows read (attention), the router and the
    two routed experts' weights (MoE), plus each step's inputs and outputs."""
    import math

    import numpy as np

    from furykernel_amd.engine import Engine
    from furykernel_amd.lower import lower_plan
    from furykernel_amd.program.build import program
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.graph import CACHE_F16, F16, F32, AttnSpec, Paged, Ring, RopeSpec, Shape, whole_row
    from furykernel_amd.program.plan import PlanOptions, plan

    heads, kv, d, positions, bs = 32, 8, 64, 4096, 64

    def attention(layout, seq_count, seq_bound):
        def body(b):
            q = b.input("q", Shape(heads * d, d), F32)
            k = b.input("k", Shape(kv * d, d), F32)
            v = b.input("v", Shape(kv * d, d), F32)
            pos = b.row_ints("position", 1, positions)
            sq = b.row_ints("blocks" if isinstance(layout, Paged) else "slot", seq_count, seq_bound)
            kc, vc = b.cache("kc", layout, CACHE_F16), b.cache("vc", layout, CACHE_F16)
            spec = RopeSpec(10000.0, d // 2)
            qr, kr = b.rope("qr", spec, pos, q), b.rope("kr", spec, pos, k)
            b.kv_store("store_k", kc, pos, sq, kr)
            b.kv_store("store_v", vc, pos, sq, v)
            b.output("o", b.attend("o", AttnSpec(heads, kv, d, None, 1.0 / math.sqrt(d), None), qr, kc, vc, pos, sq))
        return check_program(program("decode_attention", body))

    def moe():
        hidden, experts, ffn, k = 2048, 16, 1024, 2

        def body(b):
            x = b.input("x", whole_row(hidden), F32)
            g = b.weight("moe_norm", [hidden], F32)
            router = b.weight("router", [experts, hidden], F16)
            scale = b.weight("expert_scale", [experts], F32)
            gu = b.table("experts_gate_up", experts, [2 * ffn, hidden], F16)
            dn = b.table("experts_down", experts, [hidden, ffn], F16)
            cn = b.rmsnorm("moe_in", 1e-6, g, 1.0, x)
            ids, ws = b.route("route", k, scale, b.linear("router_logits", router, 0, cn))
            act = b.gated_gelu("experts_act", b.linear_routed("experts_gate_up_out", gu, ids, cn))
            s = b.combine_ranks("experts_sum", ws, b.linear_routed("experts_out", dn, ids, act))
            b.output("y", b.add("y", x, s))
        nbytes = (experts * hidden + k * 2 * ffn * hidden + k * hidden * ffn) * 2 + 3 * hidden * 4
        return check_program(program("moe", body)), nbytes

    def timed(eng, low) -> float:
        # the step repeated to at least 16 launches in its graph, so that the
        # graph launch's own cost does not dominate a step of a few launches
        n = len(low.launches)
        copies = 1 if eager else max(1, -(-16 // n))
        if eager:
            run, finish = eng.enqueue, None
        else:
            g = eng.capture(only=list(range(n)) * copies)
            run, finish = g.replay, g.destroy
        run()
        dev.sync()
        start, end = dev.event(), dev.event()
        start.record()
        for _ in range(reps):
            run()
        end.record()
        end.synchronize()
        if finish is not None:
            finish()
        return start.elapsed_ms(end) * 1e3 / (reps * copies)

    rng = np.random.default_rng(5)
    out = {}
    att_bytes = 2 * positions * kv * d * 2 + (heads + 2 * kv) * d * 4 + heads * d * 4
    for name, layout, count, bound in (("decode_attention_ring_4096", Ring(1, kv, positions, d), 1, 1),
                                       ("decode_attention_paged_4096_bs64", Paged(80, bs, kv, d), positions // bs, 80)):
        checked = attention(layout, count, bound)
        low = lower_plan(checked, plan(PlanOptions(), checked))
        eng = Engine(dev, ks, low)
        try:
            for v in ("q", "k", "v"):
                eng.init_normal(f"value:{v}", int(rng.integers(1 << 30)), 0.5)
            eng.init_normal("cache:kc", 71, 1.0)
            eng.init_normal("cache:vc", 72, 1.0)
            eng.set_ints("position", [positions - 1], positions)
            if isinstance(layout, Paged):
                eng.set_ints("blocks", rng.permutation(80)[:count], 80)
            else:
                eng.set_ints("slot", [0], 1)
            us = timed(eng, low)
        finally:
            eng.close()
        entries = [l.entry for l in low.launches]
        log(f"{name}: {entries}, {us:.2f} us a step, {att_bytes / us / 1e3:.1f} GB/s")
        out[name] = {"launches": entries, "avg_us": round(us, 3), "bytes": att_bytes,
                     "gbps": round(att_bytes / us / 1e3, 1), "frac": round(att_bytes / us / 1e3 / HBM_PEAK_GBPS, 4)}
    checked, nbytes = moe()
    low = lower_plan(checked, plan(PlanOptions(), checked))
    eng = Engine(dev, ks, low)
    try:
        for i, name in enumerate(sorted(n for n in low.buffers if n.startswith(("weight:", "table:")))):
            if low.buffers[name].dtype == "f32":
                eng.write(name, np.ones(low.buffers[name].count, np.float32))
            else:
                eng.init_normal(name, 300 + i, 0.05)
        eng.init_normal("value:x", 299, 1.0)
        us = timed(eng, low)
    finally:
        eng.close()
    entries = [l.entry for l in low.launches]
    log(f"moe_step_2048_e16_f1024_k2: {entries}, {us:.2f} us a step, {nbytes / us / 1e3:.1f} GB/s")
    out["moe_step_2048_e16_f1024_k2"] = {"launches": entries, "avg_us": round(us, 3), "bytes": nbytes,
                                         "gbps": round(nbytes / us / 1e3, 1),
                                         "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4)}
    return out


def matvec_cpu_baseline(seconds: float) -> dict:
    """The oracle's C GEMV (the reference GEMV's order at width 32, one
    thread) on an f32 4096 × 4096 matvec, repeated for about `seconds`."""
    import numpy as np

    from oracle import fkref

    rng = np.random.default_rng(1)
    w = rng.uniform(-1, 1, (4096, 4096)).astype(np.float32)
    x = rng.uniform(-1, 1, 4096).astype(np.float32)
    runs, t0 = 0, time.perf_counter()
    while True:
        fkref.gemv(w, x, 32, 4)
        runs += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    nbytes = w.nbytes + x.nbytes + 4096 * 4
    return {"value": round(nbytes * runs / el / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the oracle's C GEMV (oracle/fkref.c, width 32, pack 4) on the f32 4096 x 4096 matvec, "
                      f"{runs} runs in {el:.1f} s"}


def main() -> int:
    args = parse()
    if args.calibrate:
        return calibrate()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} (WORLD_SIZE {world}) is not run. "
              f"The decode step is one GPU's work at its real shape; sharding it is described, not built.",
              file=sys.stderr)
        return 2
    if args.workload == "prefill":
        return main_prefill(args)
    if args.workload == "kernels":
        return main_kernels(args)

    from furykernel_amd import kernels, runtime
    from furykernel_amd.decode import DecodeSession
    from furykernel_amd.program.decoder import ONE_B
    from furykernel_amd.traffic import step_bytes

    global PLAN
    PLAN = _plan_options()

    dev = runtime.Device(0)
    ks = kernels.Kernels(dev)
    session = DecodeSession(dev, ks, ONE_B, PLAN, embed=True, tuned=not args.untuned)
    from furykernel_amd import tuning
    tuned = {f: p for f, p in tuning.validated(dev.info.compute_units).items() if f.startswith("step_gemv")}

    def selection_label(used: dict):
        """The step GEMV picks the lowering used, each family's as class ->
        point, and the committed families it refused (stale or invalid)."""
        out: dict = {f: {c: "_".join(f"{a}{v}" for a, v in pt) for c, pt in p.items()} for f, p in used.items()}
        for f, problems in tuning.chooser_problems.items():
            if f.startswith("step_gemv"):
                out[f] = f"refused: {problems[0]}" + (f" (+{len(problems) - 1} more)" if len(problems) > 1 else "")
        return out or "none committed"

    log(f"GEMV step selections used: {sorted(tuned) or 'none'}"
        + (f"; refused: {tuning.chooser_problems}" if tuning.chooser_problems else ""))
    session.init_synthetic()
    session.set_position(POSITION, token=7)
    log(f"{len(session.lowered.launches)} launches a step resident in HBM; "
        f"{'eager launches' if args.eager else 'one graph'} per token")
    if args.eager:
        advance = dict(token_out="value:token", token_in="ints:tokens", position="ints:position",
                       context=ONE_B.context, step=0)

        def run():
            session.engine.enqueue(advance=advance)
    else:
        graph = session.graph(advance_position=False)
        run = graph.replay

    for _ in range(args.warmup):
        run()
    dev.sync()
    start, end = dev.event(), dev.event()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        run()
    end.record()
    dev.sync()
    elapsed = time.perf_counter() - t0
    event_ms = start.elapsed_ms(end)
    if not args.eager:
        graph.destroy()
    log(f"{args.steps} timed steps: {elapsed * 1e3 / args.steps:.4f} ms a step")

    tok_s = args.steps / elapsed
    nbytes = step_bytes(session.lowered, POSITION)
    table = kernel_table(session, args.kernel_reps, args.eager)
    for entry, row in table.items():
        log(f"{entry}: {row['launches']} launches a step, {row['avg_us']} us a launch, {row['gbps']} GB/s")
    dominant = max(table, key=lambda e: table[e]["us_per_step"])
    dom = table[dominant]
    achieved = dom["gbps"]

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: weights N(0, 0.02), KV caches N(0, 1), generated on the device (SplitMix64 + Box-Muller)",
        "config": {"workload": "1B-class f16 decode step via the planner, batch 1, one token at position 4095 "
                               "(attention over all 4096 cached positions)",
                   "d_model": ONE_B.d_model, "layers": ONE_B.layers, "heads": ONE_B.heads,
                   "kv_heads": ONE_B.kv_heads, "head_dim": ONE_B.head_dim, "ffn": ONE_B.ffn, "vocab": ONE_B.vocab,
                   "kv_length": ONE_B.context, "position": POSITION, "launches": len(session.lowered.launches),
                   "launch": "eager launches per token" if args.eager else "one HIP graph per token",
                   "gemv_selection": "untuned" if args.untuned else selection_label(tuned)},
        "hbm": {"step_bytes": nbytes, "achieved_gbps": round(nbytes * tok_s / 1e9, 1),
                "frac_of_peak": round(nbytes * tok_s / 1e9 / HBM_PEAK_GBPS, 4), "peak_gbps": HBM_PEAK_GBPS,
                "ms_per_step_events": round(event_ms / args.steps, 4)},
        "roofline": {"kernel": dominant, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(dominant),
                     "traffic_source": "read from profiles/traffic_decode_1b_f16.md (the committed rocprofv3 "
                                       "FETCH_SIZE and WRITE_SIZE runs of this workload), not measured in this run",
                     "avg_launch_us": dom["avg_us"], "bytes_per_launch": dom["bytes_per_launch"],
                     "launches_per_step": dom["launches"]},
        "kernels": table,
    }
    session.close()
    dev.close()
    line["cpu_baseline"] = None if args.no_cpu_baseline else cpu_baseline(ONE_B, args.cpu_seconds)
    log("CPU baseline done")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
