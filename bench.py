#!/usr/bin/env python3
"""Flash-attention forward benchmark on one MI355X (gfx950).

One step = one flash-attention forward of the headline workload (BH=8 S=1024 d=64 causal, f16 in,
f32 out) with Q/K/V already resident in HBM. Launches go through the C ABI (nc_flash_launch_async)
on one stream; the timed region is one replay of a HIP graph that holds the K timed launches back to
back between two HIP event-record nodes, with a device synchronize on both sides, so the average per
step is the kernel's average duration plus the (small) inter-kernel gap. Before it: --warmup untimed
steps and a wall-clock settle phase (--settle-ms) of graph replays, so that a short --warmup does
not time a GPU that is still raising its clock.

Prints ONE JSON line (rank 0, N=1) with the metric of the benchmark plan, a `roofline` object for
the flash kernel, a `cpu_baseline` object (the CPU oracle, a port of the reference's scalar CPU
reference, timed on this host on the same workload) and `extra_workloads`: the other configurations
timed the same way, each with its own parity check (c1 and c2, latency/HBM-bound, also as GB/s against
the 8 TB/s HBM peak; c4 and c5, MFMA-bound), and `mfma_ceiling`: the f16 MFMA rate the chip sustains
on operands drawn like the inputs (nc_util_mfma_ceiling).
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "not-cute-zig_amd"))

import numpy as np  # noqa: E402

import notcute_flash as nc  # noqa: E402
from flash_workloads import CONFIGS, HEADLINE  # noqa: E402

PEAK_F16_TFLOPS = 2516.6  # 256 CU x 4096 flop/clk x 2.4 GHz, dense
PEAK_HBM_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "flash_fwd_{workload}_traffic.txt")
MAX_TIMED_NODES = 20000  # launches captured into the one timed graph


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo ("unknown" where it is not readable)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(wl, q, k, v, budget_s: float, threads: int = 1) -> dict:
    """Time the CPU oracle (`threads` host threads over (slice, row)) on the full workload, repeated
    until `budget_s` passes."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import flash_oracle  # noqa: E402  (checker / CPU baseline only)

    o = np.zeros(wl.length("o"), dtype=np.float32)
    reps = 0
    t0 = time.perf_counter()
    while True:
        flash_oracle.flash_fwd(q, k, v, o, batch_heads=wl.batch_heads, seq_len=wl.seq_len, head_dim=wl.head_dim,
                               q_stride=wl.stride("q"), k_stride=wl.stride("k"), v_stride=wl.stride("v"),
                               o_stride=wl.stride("o"), scale=wl.scale, causal=wl.causal, threads=threads,
                               dtype=wl.dtype)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    flops = wl.work()["flops"]
    return {
        "value": flops * reps / el / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full {wl.name} workload ({wl.describe()}) x {reps} repetitions, {el:.1f} s, "
                  f"{'one thread' if threads == 1 else f'{threads} threads over (slice, row)'}, "
                  f"C restatement of src/main.zig:1271-1307 (-O3, no fast-math), on {cpu_model()}",
    }, o


def describe_dists(dists) -> str:
    """'N(0,1)' when Q, K and V share one distribution, else 'Q N(0,3) K N(0,3) V U(-1,1)'."""
    def one(d):
        if d[0] == "normal":
            return f"N({d[1]:g},{d[2]:g})"
        if d[0] == "uniform":
            return f"U({d[1]:g},{d[2]:g})"
        return f"((i*{d[1]}+{d[2]})%17)*{d[3]:g}"
    names = [one(d) for d in dists]
    return names[0] if len(set(names)) == 1 else " ".join(f"{t} {n}" for t, n in zip("QKV", names))


def calibrate_copy(mod: nc.Module, stream: nc.Stream, nbytes: int, iters: int) -> None:
    """Launch the plain copy kernel on a known byte count (for rocprofv3 counter calibration)."""
    n16 = nbytes // 16
    src = nc.DeviceBuffer(n16 * 16)
    dst = nc.DeviceBuffer(n16 * 16)
    src.memset(1)
    fn = mod.get_function("nc_util_copy_b128")
    import ctypes

    ps = [ctypes.c_void_p(src.ptr), ctypes.c_void_p(dst.ptr), ctypes.c_uint64(n16)]
    for _ in range(iters):
        fn.launch((1024,), (256,), ps, stream=stream.handle)
    stream.synchronize()
    src.free()
    dst.free()
    log(f"calibration copy: {iters} x {n16 * 16} bytes read + written")


def time_graph(stream, launch, steps: int, warmup: int, graph_batch: int, settle_ms: float,
               method: str = "nodes") -> dict:
    """Time exactly `steps` launches, back to back on the GPU, with a device synchronize on both sides.
    method "replays" times them as bench.py did before: events recorded on the stream around replays
    of graphs of `graph_batch` launches (time_graph_replays).

    The timed graph holds two untimed launches, a HIP event-record node, the `steps` launches and a
    second record node, so the event pair brackets exactly those launches, issued as the GPU runs a
    graph: neither the host's submission nor the graph's own launch cost (~7.7 us per replay on
    MI355X, measured as the difference between events around a replay and record nodes inside it:
    ~0.38 us of every step at 20 steps) falls between the two records. The untimed launches keep the
    GPU busy from the replay's start to the first record.

    Before the measured replay: `warmup` untimed steps as replays of a graph of up to `graph_batch`
    launches, one untimed replay of the timed graph (a new graph's first replay carries one-time
    set-up), then a clock-settle phase that keeps replaying the timed graph until `settle_ms` of wall
    time have passed (a GPU that has idled runs its first milliseconds of work on a lower clock, and
    a short --warmup alone would time that). At most 10 graphs are queued between synchronizes:
    under rocprofv3's kernel tracer, about 200 queued graphs of 100 launches each made the host
    runtime abort."""
    if method == "replays":
        return time_graph_replays(stream, launch, steps, warmup, graph_batch, settle_ms)
    if steps > MAX_TIMED_NODES:
        raise ValueError(f"--steps {steps}: at most {MAX_TIMED_NODES} launches are timed in one graph")
    gb = max(1, min(graph_batch, steps))
    graph = nc.Graph.capture(stream, lambda: [launch() for _ in range(gb)])
    # Timing-only events: their records skip the system-scope cache flush of a default event, which
    # would otherwise sit inside the event pair ahead of the first timed kernel.
    ev0, ev1 = nc.Event(timing_only=True), nc.Event(timing_only=True)

    def timed_body():
        launch()
        launch()
        ev0.record_node(stream.handle)
        for _ in range(steps):
            launch()
        ev1.record_node(stream.handle)

    timed = nc.Graph.capture(stream, timed_body)
    for i in range(warmup // gb):
        graph.launch(stream)
        if i % 10 == 9:
            stream.synchronize()
    timed.launch(stream)
    stream.synchronize()
    t0 = time.perf_counter()
    settle_graphs = 0
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(max(1, min(10, 100 // steps))):
            timed.launch(stream)
            settle_graphs += 1
        stream.synchronize()
    settled = (time.perf_counter() - t0) * 1e3
    nc.synchronize()
    timed.launch(stream)
    stream.synchronize()
    nc.synchronize()
    total_ms = nc.Event.elapsed(ev0, ev1)
    graph.destroy()
    timed.destroy()
    ev0.destroy()
    ev1.destroy()
    return {"ms_per_step": total_ms / steps, "total_ms": total_ms, "steps": steps,
            "settle_ms": round(settled, 1), "settle_launches": settle_graphs * (steps + 2)}


def time_graph_replays(stream, launch, steps: int, warmup: int, graph_batch: int, settle_ms: float) -> dict:
    """Time exactly `steps` launches as replays of graphs of up to `graph_batch` back-to-back launches,
    between HIP events recorded on the launch stream (so each graph's own launch cost, ~7.7 us, falls
    inside the pair), with two untimed replays queued ahead of the first event and a device
    synchronize on both sides; before them `warmup` steps and a clock-settle phase of replays. For
    runs under rocprofv3's kernel tracer, which executes a graph holding event-record nodes node by
    node (~67 us per launch on MI355X) but runs these graphs back to back."""
    gb = max(1, min(graph_batch, steps))
    full, rest = divmod(steps, gb)
    graph = nc.Graph.capture(stream, lambda: [launch() for _ in range(gb)])
    tail = nc.Graph.capture(stream, lambda: [launch() for _ in range(rest)]) if rest else None
    for i in range(warmup // gb):
        graph.launch(stream)
        if i % 10 == 9:
            stream.synchronize()
    stream.synchronize()
    t0 = time.perf_counter()
    settle_graphs = 0
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(10):
            graph.launch(stream)
        settle_graphs += 10
        stream.synchronize()
    settled = (time.perf_counter() - t0) * 1e3
    ev0, ev1 = nc.Event(timing_only=True), nc.Event(timing_only=True)
    nc.synchronize()
    graph.launch(stream)
    graph.launch(stream)
    ev0.record(stream.handle)
    for _ in range(full):
        graph.launch(stream)
    if tail is not None:
        tail.launch(stream)
    ev1.record(stream.handle)
    ev1.synchronize()
    nc.synchronize()
    total_ms = nc.Event.elapsed(ev0, ev1)
    graph.destroy()
    if tail is not None:
        tail.destroy()
    ev0.destroy()
    ev1.destroy()
    return {"ms_per_step": total_ms / steps, "total_ms": total_ms, "steps": steps,
            "settle_ms": round(settled, 1), "settle_launches": settle_graphs * gb}


def measure_mfma_ceiling(mod, stream, budget_ms: float, ops16) -> dict:
    """The f16 MFMA rate this chip sustains on operands drawn like the workloads' inputs: back-to-back
    32x32x16 MFMAs on all CUs (nc_util_mfma_ceiling, one 12-wave workgroup per CU, four independent
    accumulators per wave), launched for `budget_ms` after a 300 ms clock-settle period, HIP events
    around the timed launches. Under this load the clock settles where the matrix cores' power on
    such operands meets the chip's limit, so the rate is below the datasheet peak (which assumes
    the peak clock)."""
    import ctypes

    fn = mod.get_function("nc_util_mfma_ceiling")
    cus = nc.device_attributes().sm_count
    grid, threads, iters = cus, 768, 8192
    ops = nc.DeviceBuffer.from_array(ops16)
    out = nc.DeviceBuffer(grid * threads * 4)
    params = [ctypes.c_void_p(ops.ptr), ctypes.c_uint32(len(ops16) // 8), ctypes.c_void_p(out.ptr), ctypes.c_uint32(iters)]
    flops = 2.0 * 32 * 32 * 16 * 8 * iters * grid * (threads // 64)

    def run(ms_budget):
        ev0, ev1 = nc.Event(), nc.Event()
        n = 0
        t0 = time.perf_counter()
        ev0.record(stream.handle)
        while (time.perf_counter() - t0) * 1e3 < ms_budget:
            for _ in range(10):
                fn.launch((grid,), (threads,), params, stream=stream.handle)
            n += 10
            stream.synchronize()
        ev1.record(stream.handle)
        ev1.synchronize()
        el = nc.Event.elapsed(ev0, ev1)
        ev0.destroy()
        ev1.destroy()
        return n, el

    try:
        run(300.0)  # clock settle
        n, el = run(budget_ms)
    finally:
        ops.free()
        out.free()
    tflops = flops * n / (el * 1e-3) / 1e12
    log(f"bench: MFMA ceiling on f16 N(0,1) operands: {tflops:.1f} TFLOP/s ({100 * tflops / PEAK_F16_TFLOPS:.1f} % "
        f"of the datasheet peak), {n} launches in {el:.1f} ms")
    return {"tflops": round(tflops, 1), "pct_f16_peak": round(100.0 * tflops / PEAK_F16_TFLOPS, 2),
            "kernel": "nc_util_mfma_ceiling", "operands": "f16 N(0,1) (as the c3/c4 inputs)",
            "grid": grid, "threads": threads, "launches": n, "ms": round(el, 1),
            "timing": "HIP events around back-to-back launches after a 300 ms settle period",
            "note": "a lower bound of the sustainable rate: on all-zero operands this kernel reaches 91-94 % of "
                    "the datasheet rate at the 2.39 GHz it then runs at"}


def measure_extra(mod, name: str, args) -> dict:
    """One more workload timed exactly like the headline, with its own parity check (every query row
    up to S=1024, else sampled rows). Reported as extra keys of the one JSON line, with TFLOP/s and,
    for every workload, the algorithmic HBM rate (bytes of Q/K/V read once and O written once)."""
    wl = CONFIGS[name]
    if args.dtype != wl.dtype:
        wl = dataclasses.replace(wl, dtype=args.dtype)
    opts = wl.options()
    work = wl.work()
    sel = nc.select_kernel(opts)
    q, k, v = wl.make_inputs()
    dq, dk, dv = (nc.DeviceBuffer.from_array(x) for x in (q, k, v))
    do = nc.DeviceBuffer(wl.length("o") * 4)
    do.memset(0)
    stream = nc.Stream()
    try:
        def launch():
            nc.flash_launch(mod, dq, dk, dv, do, opts, stream=stream.handle)

        launch()
        stream.synchronize()
        max_abs = None
        rows = None if wl.seq_len <= 1024 else np.arange(0, wl.seq_len, 97)
        if not args.no_verify:
            import flashcheck  # noqa: E402  (checker only)

            ref = flashcheck.oracle(wl, q, k, v, rows=rows)
            max_abs, max_rel = flashcheck.errors(do.download(np.float32, wl.length("o")), ref,
                                                 flashcheck.active_index(wl, rows))
            bar_abs, bar_rel = flashcheck.parity_bar(wl.dtype)
            if not (max_abs <= bar_abs and max_rel <= bar_rel):
                raise RuntimeError(f"{name}: parity failure max-abs {max_abs} max-rel {max_rel}")
        t = time_graph(stream, launch, args.steps, args.warmup, args.graph_batch, args.settle_ms, args.timing)
        tflops = work["flops"] / (t["ms_per_step"] * 1e-3) / 1e12
        gbps = work["bytes"] / (t["ms_per_step"] * 1e-3) / 1e9
        log(f"bench: {wl.describe()} -> {sel.name.decode()}: {t['ms_per_step'] * 1e3:.2f} us/step, "
            f"{tflops:.1f} TFLOP/s ({100 * tflops / PEAK_F16_TFLOPS:.2f} % of f16 peak), {gbps:.1f} GB/s, "
            f"parity max-abs {max_abs}")
        return {"workload": f"{wl.name}: BH={wl.batch_heads} S={wl.seq_len} d={wl.head_dim} "
                            f"{'causal' if wl.causal else 'non-causal'}, Q/K/V {wl.dtype} {describe_dists(wl.dists)} "
                            f"seed {wl.seed}, scale {wl.scale:g}",
                "kernel": sel.name.decode(), "ms_per_step": round(t["ms_per_step"], 6), "steps": t["steps"],
                "settle_ms": t["settle_ms"], "tflops": round(tflops, 2),
                "pct_f16_mfma_peak": round(100.0 * tflops / PEAK_F16_TFLOPS, 3), "flops_per_step": work["flops"],
                "bound": "hbm" if work["flops"] / work["bytes"] * PEAK_HBM_GBPS / 1e3 < PEAK_F16_TFLOPS else "mfma",
                "bytes_per_step": work["bytes"], "gbps": round(gbps, 2),
                "pct_hbm_peak": round(100.0 * gbps / PEAK_HBM_GBPS, 4),
                "parity_max_abs": max_abs,
                "parity_rows": "every query row" if rows is None else "every 97th query row of every slice"}
    finally:
        for b in (dq, dk, dv, do):
            b.free()
        stream.destroy()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="timed steps (flash launches)")
    ap.add_argument("--warmup", type=int, default=5000,
                    help="untimed warmup steps: up to 50 eager launches, the rest graph replays")
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(CONFIGS))
    ap.add_argument("--graph-batch", type=int, default=100, help="launches captured per HIP graph")
    ap.add_argument("--timing", choices=("nodes", "replays"), default="nodes",
                    help="nodes: event-record nodes inside one graph around the timed launches; replays: events "
                         "around replays of --graph-batch graphs (for runs under rocprofv3's kernel tracer)")
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="untimed clock-settle replays of the timed graph, in wall-clock ms, after --warmup")
    ap.add_argument("--extra", default="c1,c2_causal,c2_full,c4,c5",
                    help="comma-separated extra workloads timed the same way (extra keys of the JSON line; '' for none)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget (0: skip)")
    ap.add_argument("--mfma-ceiling-ms", type=float, default=1000.0,
                    help="time the MFMA-ceiling kernel this long on N(0,1) f16 operands (0: skip)")
    ap.add_argument("--ref-iters", type=int, default=20, help="iterations of the per-launch event timing")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run the plain copy kernel on MIB MiB (profiling runs only)")
    ap.add_argument("--no-verify", action="store_true", help="skip the oracle check of the output")
    ap.add_argument("--dtype", choices=("f16", "bf16"), default="f16",
                    help="element type of Q/K/V (f16: the reference's and the headline's)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the path shards by (batch, head) slices with no exchange; see the design notes)", file=sys.stderr)
        return 2
    for var in ("RANK", "WORLD_SIZE"):
        if int(os.environ.get(var, "0") or 0) > (0 if var == "RANK" else 1):
            print("bench.py: multi-rank launch is not supported by this one-GPU build", file=sys.stderr)
            return 2

    wl = CONFIGS[args.workload]
    if args.dtype != wl.dtype:
        wl = dataclasses.replace(wl, dtype=args.dtype)
    opts = wl.options()
    work = wl.work()
    sel = nc.select_kernel(opts)
    log(f"bench: {wl.describe()} -> {sel.name.decode()} grid={sel.grid[0]} threads={sel.threads}")

    nc.init()
    mod = nc.Module.load_embedded()
    q, k, v = wl.make_inputs()
    dq, dk, dv = (nc.DeviceBuffer.from_array(x) for x in (q, k, v))
    do = nc.DeviceBuffer(wl.length("o") * 4)
    do.memset(0)
    stream = nc.Stream()

    def launch():
        nc.flash_launch(mod, dq, dk, dv, do, opts, stream=stream.handle)

    # correctness of what is timed
    launch()
    stream.synchronize()
    max_abs = None
    if not args.no_verify:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import flashcheck  # noqa: E402  (checker only)

        ref = flashcheck.oracle(wl, q, k, v, rows=None if wl.seq_len <= 1024 else np.arange(0, wl.seq_len, 97))
        idx = flashcheck.active_index(wl, None if wl.seq_len <= 1024 else np.arange(0, wl.seq_len, 97))
        out = do.download(np.float32, wl.length("o"))
        max_abs, max_rel = flashcheck.errors(out, ref, idx)
        log(f"bench: parity vs oracle max-abs {max_abs:.3e} max-rel {max_rel:.3e}")
        bar_abs, bar_rel = flashcheck.parity_bar(wl.dtype)
        if not (max_abs <= bar_abs and max_rel <= bar_rel):
            print(json.dumps({"error": "parity failure", "max_abs": max_abs, "max_rel": max_rel}))
            return 1

    # warmup, part 1 (eager)
    eager_warmup = min(args.warmup, 50)
    for _ in range(eager_warmup):
        launch()
    stream.synchronize()

    # reference semantics (src/benchmark.zig:35-92): one event pair per launch, mean/min/max
    fn = mod.get_function(sel.name.decode())
    ka = nc.pack_args(opts, sel, dq.ptr, dk.ptr, dv.ptr, do.ptr, module=mod)
    per_launch = nc.run_kernel(fn, tuple(sel.grid), (sel.threads,), nc.kernel_params(sel.name.decode(), ka),
                               warmup=5, iters=args.ref_iters,
                               bytes_=work["bytes"], flops=work["flops_reference"], stream=stream.handle)

    # timed region: graphs of back-to-back launches
    t = time_graph(stream, launch, args.steps, args.warmup - eager_warmup, args.graph_batch, args.settle_ms,
                   args.timing)
    ms, steps = t["ms_per_step"], t["steps"]
    log(f"bench: {steps} steps in {t['total_ms']:.3f} ms -> {ms * 1e3:.3f} us/step (after {t['settle_ms']:.0f} ms "
        f"of clock-settle replays); per-launch event timing mean {per_launch.mean_ms * 1e3:.2f} us "
        f"min {per_launch.min_ms * 1e3:.2f} us")

    # One event pair around 100 plain back-to-back launches (no graph), divided by 100.
    for _ in range(10):
        launch()
    stream.synchronize()
    ev0, ev1 = nc.Event(), nc.Event()
    ev0.record(stream.handle)
    for _ in range(100):
        launch()
    ev1.record(stream.handle)
    ev1.synchronize()
    b2b_ms = nc.Event.elapsed(ev0, ev1) / 100
    ev0.destroy()
    ev1.destroy()
    log(f"bench: 100 back-to-back launches without a graph: {b2b_ms * 1e3:.3f} us/launch")

    # Fixed per-launch cost: an empty kernel with the same grid and block, replayed the same way.
    empty = mod.get_function("nc_util_empty")
    tf_ = time_graph(stream, lambda: empty.launch(tuple(sel.grid), (sel.threads,), [ka], stream=stream.handle),
                     steps, 0, args.graph_batch, min(args.settle_ms, 50.0), args.timing)
    floor_ms = tf_["ms_per_step"]
    log(f"bench: empty kernel with the same grid: {floor_ms * 1e3:.3f} us/launch")

    if args.calibrate_copy:
        calibrate_copy(mod, stream, args.calibrate_copy << 20, 10)

    tflops = work["flops"] / (ms * 1e-3) / 1e12
    ai = work["flops"] / work["bytes"]
    roof_tflops = min(PEAK_F16_TFLOPS, ai * PEAK_HBM_GBPS / 1e3)
    bound = "hbm" if ai * PEAK_HBM_GBPS / 1e3 < PEAK_F16_TFLOPS else "mfma"
    traffic = None
    tf = TRAFFIC_FILE.format(workload=wl.name)
    if os.path.exists(tf):
        with open(tf) as f:
            rec_t = json.load(f)
        # only a figure measured on the kernel being timed is reported
        if rec_t.get("kernel") == sel.name.decode():
            traffic = rec_t.get("traffic_bytes_per_launch")
    if bound == "hbm":
        achieved = work["bytes"] / (ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                    "frac": round(achieved / PEAK_HBM_GBPS, 5), "traffic": traffic}
    else:
        roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(tflops / PEAK_F16_TFLOPS, 5), "traffic": traffic}

    extra = {}
    for name in filter(None, (x.strip() for x in args.extra.split(","))):
        if name != wl.name:
            extra[name] = measure_extra(mod, name, args)

    ceiling = None
    if args.mfma_ceiling_ms > 0:
        ceiling = measure_mfma_ceiling(mod, stream, args.mfma_ceiling_ms, nc.fill_normal(1 << 20, 7, 0, 0.0, 1.0))
        for x in extra.values():
            if x["bound"] == "mfma":
                x["pct_of_mfma_ceiling"] = round(100.0 * x["tflops"] / ceiling["tflops"], 2)

    cpu = cpu_all = None
    if args.cpu_seconds > 0:
        cpu, _ = cpu_baseline(wl, q, k, v, args.cpu_seconds)
        log(f"bench: cpu baseline {cpu['value'] * 1e3:.3f} GFLOP/s ({cpu['sample']})")
        # the same oracle threaded over (slice, row) on the host cores this job may use (16 on the box)
        nthr = max(1, min(16, len(os.sched_getaffinity(0))))
        if nthr > 1:
            cpu_all, _ = cpu_baseline(wl, q, k, v, args.cpu_seconds / 2, threads=nthr)
            log(f"bench: cpu baseline, {nthr} threads: {cpu_all['value'] * 1e3:.3f} GFLOP/s")

    rec = {
        "metric": "flash-attn fwd TFLOP/s + % f16 MFMA peak, BH=8 S=1024 d=64 causal",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic",
        "config": {"workload": f"{wl.name}: flash-attn fwd BH={wl.batch_heads} S={wl.seq_len} d={wl.head_dim} "
                               f"{'causal' if wl.causal else 'non-causal'}, Q/K/V {wl.dtype} "
                               f"{describe_dists(wl.dists)} seed {wl.seed}, scale {wl.scale:g}, "
                               f"f32 accumulate/out",
                   "batch_heads": wl.batch_heads, "seq_len": wl.seq_len, "head_dim": wl.head_dim,
                   "causal": wl.causal, "kernel": sel.name.decode(), "parallelism": "single-gpu"},
        "pct_f16_mfma_peak": round(100.0 * tflops / PEAK_F16_TFLOPS, 3),
        "pct_roofline": round(100.0 * tflops / roof_tflops, 3),
        "flops_per_step": work["flops"],
        "flops_per_step_reference_formula": work["flops_reference"],
        "bytes_per_step": work["bytes"],
        "timing": ("HIP event-record nodes inside one captured graph around exactly the timed back-to-back "
                   "launches (after two untimed ones), device synchronize before and after its replay; before "
                   "it --warmup steps and a wall-clock settle phase of replays of the same graph")
                  if args.timing == "nodes" else
                  ("HIP events on the launch stream around replays of graphs of --graph-batch back-to-back "
                   "launches (each graph's own launch cost inside the pair), after --warmup replays and a "
                   "wall-clock settle phase of replays"),
        "settle_ms": t["settle_ms"],
        "settle_launches": t["settle_launches"],
        "per_launch_event_ms": {"mean": per_launch.mean_ms, "min": per_launch.min_ms, "max": per_launch.max_ms,
                                "iters": args.ref_iters},
        "back_to_back_launch_ms": round(b2b_ms, 6),
        "launch_floor": {"ms_per_step": round(floor_ms, 6), "kernel": "nc_util_empty",
                         "grid": list(sel.grid), "threads": sel.threads,
                         "timing": "same graph replays as the timed region, empty kernel body"},
        "parity_max_abs": max_abs,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baseline_threads": cpu_all,
        "extra_workloads": extra,
        "mfma_ceiling": ceiling,
    }
    print(json.dumps(rec), flush=True)
    for b in (dq, dk, dv, do):
        b.free()
    stream.destroy()
    return 0


if __name__ == "__main__":
    sys.exit(main())
