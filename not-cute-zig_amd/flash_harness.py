#!/usr/bin/env python3
"""Command-line harness for the flash path, mirroring the reference's `flash`, `compare`,
`profile-flash` and flash-benchmark commands (src/main.zig:53-62) and the compare table of its
runner (modal_run.py:34-69), on one MI355X through the C ABI.

    python flash_harness.py flash                 # runFlashAttention's four cases (src/main.zig:189-194)
    python flash_harness.py compare               # runCompareDemo's flash shapes as JSONL (src/main.zig:141-170)
    python flash_harness.py baselines             # PyTorch SDPA on the same shapes (tools/pytorch_baselines.py)
    python flash_harness.py materialized          # rocBLAS QK^T -> softmax -> PV (tools/cuda_baselines.cu:689-759)
    python flash_harness.py profile-flash         # runProfileFlash (src/main.zig:81-130)
    python flash_harness.py profile-flash --counters DIR   # the same under rocprofv3 counter passes
                                                  # (the Nsight Compute run of modal_run.py:108-146)
    python flash_harness.py benchmark-flash       # runFlashBenchmark (src/main.zig:760-766)
    python flash_harness.py timeline --workload c3    # per-wave timeline of the selected kernel
    python flash_harness.py compare-table FILE... # the baseline-vs-not-cute table (modal_run.py:34-69)

Correctness here is checked against a float64 softmax(scale * Q K^T) V written in this file (the
reference checks against its f32 CPU loop; both are far inside the 0.008 / 0.02 tolerances it
applies). `baselines` times PyTorch's scaled_dot_product_attention backends on the same device,
shapes and inputs, in its own process: PyTorch brings its own HIP runtime, and this library is then
used only for its host-side input fills.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import math
import os
import re
import shutil
import subprocess
import sys
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import notcute_flash as nc  # noqa: E402
from flash_workloads import REFERENCE_COMPARE_SHAPES, REFERENCE_FILLS, Workload, reference_smoke_cases  # noqa: E402

# runFlashBenchmark's cases (src/main.zig:760-766) and their fills (src/main.zig:787-795):
# Q = ((3i+1) % 11) / 8, K = ((5i+2) % 13) / 16, V = ((7i+3) % 17) / 32.
BENCHMARK_SHAPES = [(2, 32, 16, False), (2, 32, 32, True), (2, 64, 16, False), (2, 64, 32, True), (2, 128, 32, True)]
BENCHMARK_FILLS = ((3, 1, 11, 0.125), (5, 2, 13, 0.0625), (7, 3, 17, 0.03125))

SMOKE_TOL = 0.008    # src/main.zig:279
COMPARE_TOL = 0.02   # src/main.zig:1042
BASELINE_TOL = 0.08  # tools/pytorch_baselines.py:205

# Keys of a compare record, in the reference's order (src/main.zig:873-880).
RECORD_KEYS = ("kernel", "implementation", "shape", "correct", "mean_ms", "min_ms", "max_ms", "gbps", "tflops",
               "bytes", "flops", "max_abs_error")


def shape_name(batch_heads: int, seq_len: int, head_dim: int, causal: bool) -> str:
    """src/main.zig:1044 / tools/pytorch_baselines.py:50."""
    return f"batch_heads={batch_heads},seq={seq_len},head={head_dim},causal={str(causal).lower()}"


def reference_work(batch_heads: int, seq_len: int, head_dim: int, causal: bool) -> Tuple[int, int]:
    """(flops, bytes) as src/main.zig:1032-1034: S(S+1)/2 score pairs when causal."""
    eff = seq_len * (seq_len + 1) // 2 if causal else seq_len * seq_len
    return batch_heads * 4 * eff * head_dim, batch_heads * seq_len * head_dim * (2 * 3 + 4)


def modular_fill(n: int, mul: int, add: int, mod: int, scale: float) -> np.ndarray:
    """f16 bit patterns of ((i*mul + add) % mod) * scale, i = 0..n-1."""
    i = np.arange(n, dtype=np.int64)
    return ((((i * mul + add) % mod).astype(np.float32)) * np.float32(scale)).astype(np.float16).view(np.uint16)


def decode(bits: np.ndarray, dtype: str = "f16") -> np.ndarray:
    """16-bit patterns of f16 or bf16 (the upper half of a binary32) as float64."""
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return bits.view(np.float16).astype(np.float64)


def attention_f64(wl: Workload, q: np.ndarray, k: np.ndarray, v: np.ndarray,
                  rows: Optional[np.ndarray] = None) -> np.ndarray:
    """softmax(scale * Q K^T, causal mask) V in float64 for every slice; returns O in the workload's
    f32 layout with unwritten (pad) positions left 0. `rows` restricts the query rows computed."""
    S, D = wl.seq_len, wl.head_dim
    out = np.zeros(wl.length("o"), dtype=np.float64)
    qf, kf, vf = (decode(x, wl.dtype) for x in (q, k, v))
    r_all = np.arange(S) if rows is None else np.asarray(rows)
    for b in range(wl.batch_heads):
        def mat(buf, which):
            base, rs = b * wl.stride(which), wl.row(which)
            idx = base + np.arange(S)[:, None] * rs + np.arange(D)[None, :]
            return buf[idx]
        Q, K, V = mat(qf, "q")[r_all], mat(kf, "k"), mat(vf, "v")
        s = (Q @ K.T) * float(np.float32(wl.scale))
        if wl.causal:
            s = np.where(np.arange(S)[None, :] > r_all[:, None], -np.inf, s)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        o = (p / p.sum(axis=1, keepdims=True)) @ V
        obase, ors = b * wl.stride("o"), wl.row("o")
        out[obase + r_all[:, None] * ors + np.arange(D)[None, :]] = o
    return out


def active_index(wl: Workload, rows: Optional[np.ndarray] = None) -> np.ndarray:
    S, D = wl.seq_len, wl.head_dim
    r = np.arange(S) if rows is None else np.asarray(rows)
    idx = [b * wl.stride("o") + r[:, None] * wl.row("o") + np.arange(D)[None, :] for b in range(wl.batch_heads)]
    return np.concatenate([x.ravel() for x in idx])


def make_record(implementation: str, shape: str, correct: bool, mean_ms: float, min_ms: float, max_ms: float,
                bytes_: int, flops: int, max_abs_error: float) -> Dict:
    """One compare record with the reference's fields and formulas (src/benchmark.zig:83-89)."""
    gbps = bytes_ / (mean_ms * 1.0e6) if mean_ms > 0 else 0.0
    tflops = flops / (mean_ms * 1.0e9) if mean_ms > 0 else 0.0
    vals = ("flash_attention", implementation, shape, bool(correct), float(mean_ms), float(min_ms), float(max_ms),
            gbps, tflops, int(bytes_), int(flops), float(max_abs_error))
    return dict(zip(RECORD_KEYS, vals))


def emit(rec: Dict, out=None) -> None:
    out = sys.stdout if out is None else out
    out.write(json.dumps(rec, separators=(",", ":")) + "\n")
    out.flush()


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Device:
    """Device buffers of one workload's inputs and output, uploaded once."""

    def __init__(self, wl: Workload, q, k, v, o_init=None):
        self.wl = wl
        self.bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v)]
        o = np.zeros(wl.length("o"), np.float32) if o_init is None else o_init
        self.bufs.append(nc.DeviceBuffer.from_array(o))

    def launch(self, module: nc.Module) -> None:
        q, k, v, o = self.bufs
        nc.flash_launch(module, q, k, v, o, self.wl.options())

    def output(self) -> np.ndarray:
        nc.synchronize()
        return self.bufs[3].download(np.float32, self.wl.length("o"))

    def time_selected(self, module: nc.Module, flops: int, bytes_: int, warmup: int = 5, iters: int = 20):
        """benchmark.runKernel over the selected kernel (src/main.zig:1033-1035)."""
        opts = self.wl.options()
        sel = nc.select_kernel(opts)
        fn = module.get_function(sel.name.decode())
        args = nc.pack_args(opts, sel, *[b.ptr for b in self.bufs], module=module)
        return sel, nc.run_kernel(fn, tuple(sel.grid), (sel.threads,), nc.kernel_params(sel.name.decode(), args),
                                  warmup=warmup, iters=iters,
                                  bytes_=bytes_, flops=flops)

    def free(self) -> None:
        for b in self.bufs:
            b.free()


# ---------------------------------------------------------------------------------------------
# flash: runFlashAttention (src/main.zig:189-287)
# ---------------------------------------------------------------------------------------------

def cmd_flash(module: nc.Module, _args) -> int:
    status = 0
    for wl in reference_smoke_cases():
        q, k, v = wl.make_inputs()
        dev = Device(wl, q, k, v)
        try:
            dev.launch(module)
            out = dev.output()
        finally:
            dev.free()
        ref = attention_f64(wl, q, k, v)
        idx = active_index(wl)
        diff = np.abs(out[idx] - ref[idx])
        bad = np.nonzero(diff > SMOKE_TOL)[0]
        pad = np.setdiff1d(np.arange(wl.length("o")), idx)
        if bad.size:
            i = int(idx[bad[0]])
            b = i // wl.stride("o")
            log(f"flash mismatch at batch {b} idx {i - b * wl.stride('o')}: expected {ref[i]}, got {out[i]}, "
                f"diff {abs(out[i] - ref[i])}")
            status = 1
        elif pad.size and np.any(out[pad] != 0):
            log(f"flash wrote outside the active region: batch_heads={wl.batch_heads}, seq={wl.seq_len}")
            status = 1
        else:
            log(f"flash attention OK: batch_heads={wl.batch_heads}, causal={str(wl.causal).lower()}, "
                f"Q/K/V/O={wl.seq_len}x{wl.head_dim} (max-abs {float(diff.max()):.2e})")
    return status


# ---------------------------------------------------------------------------------------------
# compare: compareFlash (src/main.zig:976-1047) + tools/pytorch_baselines.py
# ---------------------------------------------------------------------------------------------

def compare_workloads(which: str) -> List[Tuple[Workload, Optional[np.ndarray]]]:
    """(workload, checked rows or None for all)."""
    if which == "reference":
        return [(Workload(f"compare_bh{bh}_s{s}_d{d}", bh, s, d, c, 1.0 / math.sqrt(d), REFERENCE_FILLS), None)
                for (bh, s, d, c) in REFERENCE_COMPARE_SHAPES]
    from flash_workloads import CONFIGS, sample_rows
    out = []
    for name in ("c1", "c3", "c4", "c5"):
        wl = CONFIGS[name]
        out.append((wl, None if wl.seq_len <= 1024 else sample_rows(wl.seq_len, extra=16, seed=wl.seed)))
    return out


def torch_baselines(wl: Workload, q, k, v, ref: np.ndarray, idx: np.ndarray, shape: str, flops: int, bytes_: int,
                    warmup: int, iters: int) -> List[Dict]:
    """scaled_dot_product_attention backends on the same device and inputs (contiguous slices
    only). The math backend runs on float32 copies: its batched products in reduced precision take
    transposed views, which this pool's GPUs do not run reliably."""
    try:
        import torch
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel
    except Exception as exc:  # torch absent or too old
        log(f"baselines skipped: {exc}")
        return []
    if not torch.cuda.is_available():
        log("baselines skipped: torch sees no GPU")
        return []
    if any(wl.stride(x) != wl.seq_len * wl.head_dim for x in "qkvo"):
        log(f"baselines skipped for {shape}: padded slices")
        return []
    B, S, D = wl.batch_heads, wl.seq_len, wl.head_dim

    def t(x):
        return torch.from_numpy(x.view(np.float16).reshape(B, 1, S, D).copy()).to("cuda")

    tq, tk, tv = t(q), t(k), t(v)
    scale = float(np.float32(wl.scale))
    recs = []
    for impl, backend, dtype in (("torch_sdpa_flash", SDPBackend.FLASH_ATTENTION, torch.float16),
                                 ("torch_sdpa_mem_efficient", SDPBackend.EFFICIENT_ATTENTION, torch.float16),
                                 ("torch_sdpa_math_f32", SDPBackend.MATH, torch.float32)):
        a, b_, c_ = (x.to(dtype) for x in (tq, tk, tv))
        try:
            with sdpa_kernel(backend):
                for _ in range(warmup):
                    o = F.scaled_dot_product_attention(a, b_, c_, is_causal=wl.causal, scale=scale)
                torch.cuda.synchronize()
                samples = []
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                for _ in range(iters):
                    e0.record()
                    o = F.scaled_dot_product_attention(a, b_, c_, is_causal=wl.causal, scale=scale)
                    e1.record()
                    e1.synchronize()
                    samples.append(float(e0.elapsed_time(e1)))
        except Exception as exc:
            log(f"{impl} unavailable for {shape}: {str(exc).splitlines()[0][:160]}")
            continue
        got = o.to(torch.float32).reshape(-1).cpu().numpy().astype(np.float64)
        err = float(np.max(np.abs(got[idx] - ref[idx])))
        recs.append(make_record(impl, shape, err <= BASELINE_TOL, sum(samples) / len(samples), min(samples),
                                max(samples), bytes_, flops, err))
    return recs


def cmd_compare(module: nc.Module, args) -> int:
    status = 0
    for wl, rows in compare_workloads(args.shapes):
        shape = shape_name(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
        flops, bytes_ = reference_work(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
        q, k, v = wl.make_inputs()
        dev = Device(wl, q, k, v)
        try:
            dev.launch(module)
            out = dev.output()
            sel, res = dev.time_selected(module, flops, bytes_, args.warmup, args.iters)
        finally:
            dev.free()
        ref = attention_f64(wl, q, k, v, rows)
        idx = np.arange(wl.length("o")) if rows is None else active_index(wl, rows)
        err = float(np.max(np.abs(out[idx] - ref[idx])))
        ok = err <= COMPARE_TOL
        status |= 0 if ok else 1
        log(f"compare: not-cute flash {shape} -> {sel.name.decode()}")
        emit(make_record("not_cute", shape, ok, res.mean_ms, res.min_ms, res.max_ms, bytes_, flops, err))
    return status


def cmd_baselines(args) -> int:
    """tools/pytorch_baselines.py over the same shapes and inputs as `compare`."""
    import torch  # noqa: F401  (before any HIP use in this process)

    cases = compare_workloads(args.shapes)
    if args.limit:
        cases = cases[:args.limit]
    n = 0
    for wl, rows in cases:
        shape = shape_name(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
        flops, bytes_ = reference_work(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
        q, k, v = wl.make_inputs()
        ref = attention_f64(wl, q, k, v, rows)
        idx = np.arange(wl.length("o")) if rows is None else active_index(wl, rows)
        for rec in torch_baselines(wl, q, k, v, ref, idx, shape, flops, bytes_, args.warmup, args.iters):
            emit(rec)
            n += 1
    return 0 if n else 1


def materialized_record(plan: nc.Materialized, stream: nc.Stream, wl: Workload, q, k, v,
                        rows: Optional[np.ndarray], warmup: int, iters: int) -> Dict:
    """One `cublas_materialized` record (tools/cuda_baselines.cu:744-759): the output checked against
    the float64 reference, per-call event timing, bytes = inputs + output + workspace."""
    shape = shape_name(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
    flops, bytes_ = reference_work(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
    opts = wl.options()
    ws_bytes = nc.Materialized.workspace_bytes(opts)
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v)]
    bufs.append(nc.DeviceBuffer.from_array(np.zeros(wl.length("o"), np.float32)))
    bufs.append(nc.DeviceBuffer(ws_bytes))
    e0, e1 = nc.Event(), nc.Event()
    try:
        def run():
            plan.run(*bufs[:4], bufs[4], opts)

        run()
        stream.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
        for _ in range(warmup):
            run()
        stream.synchronize()
        samples = []
        for _ in range(iters):
            e0.record(stream.handle)
            run()
            e1.record(stream.handle)
            e1.synchronize()
            samples.append(nc.Event.elapsed(e0, e1))
    finally:
        e0.destroy()
        e1.destroy()
        for b in bufs:
            b.free()
    ref = attention_f64(wl, q, k, v, rows)
    idx = np.arange(wl.length("o")) if rows is None else active_index(wl, rows)
    err = float(np.max(np.abs(out[idx] - ref[idx])))
    rec = make_record("rocblas_materialized", shape, err <= BASELINE_TOL, sum(samples) / len(samples),
                      min(samples), max(samples), bytes_ + ws_bytes, flops, err)
    rec["workspace_bytes"] = ws_bytes
    return rec


def cmd_materialized(_module: nc.Module, args) -> int:
    """tools/cuda_baselines.cu:689-759 over the `compare` shapes and inputs, in this process."""
    cases = compare_workloads(args.shapes)
    if args.limit:
        cases = cases[:args.limit]
    stream = nc.Stream()
    plan = nc.Materialized(stream.handle)
    status = 0
    try:
        for wl, rows in cases:
            q, k, v = wl.make_inputs()
            rec = materialized_record(plan, stream, wl, q, k, v, rows, args.warmup, args.iters)
            status |= 0 if rec["correct"] else 1
            emit(rec)
    finally:
        plan.destroy()
        stream.destroy()
    return status


# ---------------------------------------------------------------------------------------------
# profile-flash: runProfileFlash (src/main.zig:81-130)
# ---------------------------------------------------------------------------------------------

def occupancy_report(module: nc.Module, opts) -> Dict:
    sel = nc.select_kernel(opts)
    fn = module.get_function(sel.name.decode())
    attrs = fn.attributes()
    dev = nc.device_attributes()
    threads = int(sel.threads)
    waves_per_block = threads // dev.warp_size
    by_threads = dev.max_threads_per_sm // threads
    regs_per_block = attrs.num_regs * threads
    by_regs = dev.max_registers_per_sm // regs_per_block if regs_per_block > 0 else by_threads
    by_lds = dev.max_shared_memory_per_sm // attrs.shared_size_bytes if attrs.shared_size_bytes > 0 else by_threads
    selected = fn.max_active_blocks(threads)
    return {
        "kernel": sel.name.decode(), "label": sel.label.decode(), "threads": threads,
        "grid": [int(x) for x in sel.grid], "regs_per_thread": attrs.num_regs,
        "static_lds": attrs.shared_size_bytes, "local": attrs.local_size_bytes, "const": attrs.const_size_bytes,
        "max_threads_per_block": attrs.max_threads_per_block, "binary_version": attrs.binary_version,
        "limit_by_threads": by_threads, "limit_by_regs": by_regs, "limit_by_lds": by_lds,
        "blocks_per_cu": selected, "waves_per_cu": selected * waves_per_block,
        "max_waves_per_cu": dev.max_threads_per_sm // dev.warp_size, "cu_count": dev.sm_count,
        "device": dev.name.decode(),
    }


def cmd_profile(module: nc.Module, args) -> int:
    bh, s, d, causal = 8, 1024, 64, True
    opts = nc.options(batch_heads=bh, seq_len=s, head_dim=d, scale=1.0 / math.sqrt(d), causal=causal)
    r = occupancy_report(module, opts)
    log(f"profile: not-cute flash batch_heads={bh} seq={s} head={d} causal=true")
    log(f"profile: selected kernel {r['kernel']} ({r['label']}), threads/block={r['threads']}, grid={r['grid'][0]}")
    log(f"profile: function attrs regs/thread={r['regs_per_thread']}, static_lds={r['static_lds']} B, "
        f"local={r['local']} B, const={r['const']} B, max_threads/block={r['max_threads_per_block']}, "
        f"binary={r['binary_version']}")
    log(f"profile: occupancy limits blocks/CU threads={r['limit_by_threads']}, regs={r['limit_by_regs']}, "
        f"lds={r['limit_by_lds']}, selected={r['blocks_per_cu']} (HIP occupancy API)")
    log(f"profile: selected occupancy waves/CU={r['waves_per_cu']} of max {r['max_waves_per_cu']} "
        f"on {r['cu_count']} CUs ({r['device']})")
    print(json.dumps({"profile": r}, separators=(",", ":")), flush=True)
    args.shapes = "single"
    wl = Workload("profile", bh, s, d, causal, 1.0 / math.sqrt(d), REFERENCE_FILLS)
    return _compare_one(module, wl, args)


# Counter passes of `profile-flash --counters`, the MI355X counterpart of the reference's Nsight
# Compute run (modal_run.py:108-146: speedOfLight, Occupancy, SchedulerStats, WarpStateStats and
# MemoryWorkloadAnalysis sections). rocprofv3 does not split counters over passes, so each pass is
# its own profiler run holding at most 8 SQ, 4 TCC (FETCH_SIZE takes 3, WRITE_SIZE 2) and 2 GRBM
# counters.
COUNTER_PASSES = [
    ("trace", ["--kernel-trace", "--stats"]),
    ("speed_of_light", ["--pmc", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F16",
                        "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_ACTIVE_INST_VALU", "SQ_INSTS_VALU", "SQ_INSTS_MFMA",
                        "GRBM_GUI_ACTIVE"]),
    ("scheduler", ["--pmc", "SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_ANY",
                   "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_WAIT_INST_LDS"]),
    ("lds", ["--pmc", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_ADDR_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_ACTIVE_INST_LDS"]),
    ("hbm_read", ["--pmc", "FETCH_SIZE"]),
    ("hbm_write", ["--pmc", "WRITE_SIZE"]),
    ("l2", ["--pmc", "TCC_HIT_sum", "TCC_MISS_sum"]),
]
SIMDS = 1024  # 256 CUs x 4 SIMDs
XCDS = 8      # GRBM_GUI_ACTIVE is reported summed over the XCDs


def _read_counters(outdir: str, kernel: str) -> Tuple[Dict[str, float], int]:
    """Per-dispatch means of every counter of `kernel` in a pass's counter_collection CSV files."""
    vals: Dict[str, List[float]] = {}
    for path in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                if row.get("Kernel_Name", "").split("(")[0].strip() == kernel:
                    vals.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
    n = max((len(v) for v in vals.values()), default=0)
    return {k: sum(v) / len(v) for k, v in vals.items()}, n


def _read_trace(outdir: str, kernel: str) -> Dict[str, float]:
    for path in glob.glob(os.path.join(outdir, "**", "*kernel_stats.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                if row["Name"].split("(")[0].strip() == kernel:
                    return {"calls": int(row["Calls"]), "average_ns": float(row["AverageNs"]),
                            "min_ns": float(row["MinNs"]), "max_ns": float(row["MaxNs"])}
    return {}


def cmd_profile_counters(args) -> int:
    """Run `profile-flash` once per counter pass under rocprofv3 (each pass a child process of its
    own, started before this process touches the GPU) and summarise the selected kernel's counters
    per dispatch."""
    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    kernel = nc.select_kernel(nc.options(batch_heads=8, seq_len=1024, head_dim=64, scale=0.125,
                                         causal=True)).name.decode()
    outroot = os.path.abspath(args.counters)
    env = dict(os.environ, TMPDIR="/tmp")
    child = [sys.executable, os.path.abspath(__file__), "profile-flash", "--warmup", str(args.warmup),
             "--iters", str(args.iters)]
    res: Dict[str, Dict] = {}
    for name, extra in COUNTER_PASSES:
        outdir = os.path.join(outroot, name)
        cmd = [rocprof, *extra, "-f", "csv", "-d", outdir, "-o", name, "--", *child]
        log(f"profile: pass {name}: {' '.join(cmd)}")
        try:
            p = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True, timeout=args.pass_timeout)
        except subprocess.TimeoutExpired:
            log(f"profile: pass {name} timed out after {args.pass_timeout} s")
            return 1
        # rocprofv3 may end with a segmentation fault after the program has finished and its files
        # are complete; the files decide.
        res[name] = _read_trace(outdir, kernel) if name == "trace" else dict(zip(("counters", "dispatches"),
                                                                                 _read_counters(outdir, kernel)))
        if not res[name] or (name != "trace" and not res[name]["dispatches"]):
            log(f"profile: pass {name} produced no record of {kernel} (rc {p.returncode}): {p.stderr[-400:]}")
            return 1
    c = {k: v for name, _ in COUNTER_PASSES[1:] for k, v in res[name]["counters"].items()}
    gui = c["GRBM_GUI_ACTIVE"] / XCDS  # GPU-busy cycles of one XCD during the dispatch
    summary = {
        "kernel": kernel, "dispatches": res["speed_of_light"]["dispatches"],
        "duration_us": res["trace"]["average_ns"] / 1e3,
        "grbm_gui_active_per_xcd": gui,
        "mfma_busy_pct": 100.0 * c["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * SIMDS),
        "mfma_flops": c["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512,
        "valu_mfma_coexec_pct_of_mfma": 100.0 * c["SQ_VALU_MFMA_COEXEC_CYCLES"] / max(c["SQ_VALU_MFMA_BUSY_CYCLES"], 1.0),
        "waves": c["SQ_WAVES"], "wait_any_pct_of_wave_cycles": 100.0 * c["SQ_WAIT_ANY"] / max(c["SQ_WAVE_CYCLES"], 1.0),
        "insts_per_wave": {k: c[k] / max(c["SQ_WAVES"], 1.0) for k in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_SALU",
                                                                      "SQ_INSTS_LDS")},
        "lds_bank_conflict_cycles": c["SQ_LDS_BANK_CONFLICT"],
        "fetch_kib": c["FETCH_SIZE"], "write_kib": c["WRITE_SIZE"],
        "l2_hit_pct": 100.0 * c["TCC_HIT_sum"] / max(c["TCC_HIT_sum"] + c["TCC_MISS_sum"], 1.0),
        "counters": c,
    }
    log(f"profile: {kernel}: {summary['duration_us']:.2f} us per dispatch, MFMA busy {summary['mfma_busy_pct']:.1f} % "
        f"of SIMD cycles, VALU co-issued with {summary['valu_mfma_coexec_pct_of_mfma']:.1f} % of MFMA cycles, "
        f"waves waiting {summary['wait_any_pct_of_wave_cycles']:.1f} % of their cycles, L2 hit {summary['l2_hit_pct']:.1f} %, "
        f"FETCH_SIZE {summary['fetch_kib']:.1f} KiB, WRITE_SIZE {summary['write_kib']:.1f} KiB")
    print(json.dumps({"profile_counters": summary}, separators=(",", ":")), flush=True)
    return 0


def _compare_one(module: nc.Module, wl: Workload, args) -> int:
    shape = shape_name(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
    flops, bytes_ = reference_work(wl.batch_heads, wl.seq_len, wl.head_dim, wl.causal)
    q, k, v = wl.make_inputs()
    dev = Device(wl, q, k, v)
    try:
        dev.launch(module)
        out = dev.output()
        _, res = dev.time_selected(module, flops, bytes_, args.warmup, args.iters)
    finally:
        dev.free()
    err = float(np.max(np.abs(out - attention_f64(wl, q, k, v))))
    emit(make_record("not_cute", shape, err <= COMPARE_TOL, res.mean_ms, res.min_ms, res.max_ms, bytes_, flops, err))
    return 0 if err <= COMPARE_TOL else 1


# ---------------------------------------------------------------------------------------------
# benchmark-flash: runFlashBenchmark (src/main.zig:760-857) with BenchmarkResult.print
# ---------------------------------------------------------------------------------------------

def cmd_benchmark(module: nc.Module, args) -> int:
    for (bh, s, d, causal) in BENCHMARK_SHAPES:
        n = bh * s * d
        q, k, v = (modular_fill(n, *f) for f in BENCHMARK_FILLS)
        wl = Workload("bench", bh, s, d, causal, 1.0 / math.sqrt(d), REFERENCE_FILLS)
        flops, bytes_ = reference_work(bh, s, d, causal)
        dev = Device(wl, q, k, v)
        try:
            sel, res = dev.time_selected(module, flops, bytes_, args.warmup, args.iters)
        finally:
            dev.free()
        print(f"--- Benchmark: {sel.label.decode()} seq={s} head={d} causal={str(causal).lower()} ---")
        print(f"  Time: mean={res.mean_ms:.3f}ms, min={res.min_ms:.3f}ms, max={res.max_ms:.3f}ms")
        print(f"  Bandwidth: {res.throughput_gbps:.2f} GB/s")
        print(f"  Compute:   {res.tflops:.2f} TFLOPs", flush=True)
    return 0


# ---------------------------------------------------------------------------------------------
# compare-table (modal_run.py:34-69)
# ---------------------------------------------------------------------------------------------

BASELINE_IMPLS = ("torch_sdpa_flash", "torch_sdpa_mem_efficient", "torch_sdpa_math", "torch_sdpa_math_f32",
                  "rocblas_materialized", "cublas_materialized", "cuda_wmma", "cuda_tiled")


# The table's columns (header, format spec): the layout of modal_run.py:34-69's printout, kept so
# that both read alike. TABLE_KEYS are the record fields a row needs.
TABLE_COLUMNS = (("kernel", "<18"), ("shape", "<40"), ("baseline", "<26"), ("not-cute ms", ">12"),
                 ("base ms", ">12"), ("speedup", ">9"), ("ok", ">5"))
TABLE_KEYS = ("kernel", "implementation", "shape", "mean_ms", "correct")


def read_records(lines: Iterable[str]) -> List[Dict]:
    """Compare records from JSONL mixed with other program output (the way modal_run.py:21-31 reads
    a remote run's stdout). A line that does not open a JSON object is other output and is passed
    over; one that opens an object but does not parse, or lacks a field the table needs, is
    reported on stderr with its line number and left out."""
    kept = []
    for number, text in enumerate(lines, 1):
        text = text.strip()
        if not text.startswith("{"):
            continue
        try:
            rec = json.loads(text)
        except json.JSONDecodeError as exc:
            log(f"compare-table: line {number} left out, not valid JSON ({exc.msg} at column {exc.colno})")
            continue
        absent = [key for key in TABLE_KEYS if key not in rec]
        if absent:
            log(f"compare-table: line {number} left out, no {'/'.join(absent)} field")
            continue
        kept.append(rec)
    return kept


def compare_table(records: Sequence[Dict]) -> str:
    """One row per (kernel, shape, baseline) that has both a not-cute record and a record of that
    baseline (BASELINE_IMPLS order within a case, cases sorted): both mean times, the baseline's
    time over not-cute's, and "yes" when both records passed their checks."""
    cases: Dict[Tuple[str, str], Dict[str, Dict]] = {}
    for rec in records:
        cases.setdefault((rec["kernel"], rec["shape"]), {})[rec["implementation"]] = rec
    rows = []
    for kernel, shape in sorted(cases):
        impls = cases[(kernel, shape)]
        ours = impls.get("not_cute")
        if ours is None:
            continue
        for name in (n for n in BASELINE_IMPLS if n in impls):
            theirs = impls[name]
            ratio = theirs["mean_ms"] / ours["mean_ms"] if ours["mean_ms"] else 0.0
            rows.append((kernel, shape, name, f"{ours['mean_ms']:.6f}", f"{theirs['mean_ms']:.6f}", f"{ratio:.2f}x",
                         "yes" if ours["correct"] and theirs["correct"] else "no"))
    header = tuple(title for title, _ in TABLE_COLUMNS)
    return "\n".join(["=== baselines vs not-cute ==="] +
                     [" ".join(format(cell, spec) for cell, (_, spec) in zip(row, TABLE_COLUMNS)) for row in (header, *rows)])


TIMELINE_WORDS = 13  # NC_TIMELINE_WORDS in csrc/flash_fwd.hip
TIMELINE_OBJECT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "flash_fwd_timeline_gfx950.hsaco")


def summarize_timeline(stamps: np.ndarray) -> dict:
    """Per-wave stamps of one launch ([workgroups, waves, TIMELINE_WORDS] u64, the layout written by
    the timeline code object) -> times in us from the first wave's start. Each wave's core-clock
    readings are placed on the chip-wide 100 MHz timebase through its 100 MHz reading at the end:
    with the clock over its life where it also read that counter at entry (word 12), else with its
    clock at the end (the two readings of both counters it takes there)."""
    st = stamps.astype(np.float64)
    anchored = st[..., 12] > 0
    cyc_per_tick = np.where(anchored, (st[..., 3] - st[..., 0]) / np.where(anchored, st[..., 5] - st[..., 12], 1.0),
                            (st[..., 4] - st[..., 3]) / (st[..., 6] - st[..., 5]))  # core cycles per 10 ns
    to_us = lambda word: (st[..., 5] - (st[..., 3] - st[..., word]) / cyc_per_tick) * 0.01  # noqa: E731
    start, loop0, loop1, end = to_us(0), to_us(1), to_us(2), to_us(3)
    t0 = start.min()
    start, loop0, loop1, end = start - t0, loop0 - t0, loop1 - t0, end - t0
    qblk = st[:, 0, 9].astype(np.int64)
    blocks = []
    for b in sorted(set(qblk.tolist())):
        m = qblk == b
        blocks.append({"query_block": b, "workgroups": int(m.sum()), "key_blocks": int(st[m][:, :, 8].max()),
                       "start": [round(float(start[m].min()), 3), round(float(start[m].max()), 3)],
                       "loop_start": [round(float(loop0[m].mean()), 3), round(float(loop0[m].max()), 3)],
                       "loop_end": [round(float(loop1[m].mean()), 3), round(float(loop1[m].max()), 3)],
                       "end": [round(float(end[m].mean()), 3), round(float(end[m].max()), 3)]})
    heavy = qblk == max(qblk.tolist(), key=lambda b: float(loop1[qblk == b].max() - loop0[qblk == b].min()))
    cyc = lambda a, b: float((st[heavy][:, :, b] - st[heavy][:, :, a]).mean())  # noqa: E731
    return {"clock_ghz": round(float(np.median(cyc_per_tick)) / 10.0, 3), "anchor": "start" if anchored.all() else "end",
            "wave_start_us": [round(float(np.percentile(start, q)), 3) for q in (0, 50, 100)],
            "span_us": round(float(end.max()), 3),
            "blocks": blocks,
            "heaviest_cycles": {"prologue": round(cyc(0, 1)), "key_loop": round(cyc(1, 2)), "epilogue": round(cyc(2, 3))}}


def cmd_timeline(args) -> int:
    """Per-wave timeline of the kernel the workload selects: the timeline code object's copy of it
    (csrc/flash_fwd.hip built with -DNC_TIMELINE) in the same graph replays of back-to-back launches
    as bench.py, stamps taken from the last launch. Prints the per-launch time of both copies (the
    stamped copy is slower by the ~1 us its last chip-clock read holds each wave) and, per query
    block, when its waves start, enter and leave their key loop and end."""
    from flash_workloads import CONFIGS

    wl = CONFIGS[args.workload]
    opts = wl.options()
    sel = nc.select_kernel(opts)
    name = sel.name.decode()
    if sel.scratch_bytes or not re.search(r"_q\d+s\d+p\d", name):
        print(f"timeline: {name} carries no stamps (only the pipelined kernels without scratch do)", file=sys.stderr)
        return 2
    nc.init()
    product = nc.Module.load_embedded()
    stamped = nc.Module.load_file(TIMELINE_OBJECT)
    q, k, v = wl.make_inputs()
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v)] + [nc.DeviceBuffer(wl.length("o") * 4)]
    grid = sel.grid[0] * sel.grid[1] * sel.grid[2]
    nw = sel.threads // 64
    words = grid * nw * TIMELINE_WORDS
    stamp_bufs = [nc.DeviceBuffer(words * 8) for _ in range(2)]
    stream = nc.Stream()
    result = {"workload": wl.describe(), "kernel": name, "launches": args.launches}
    try:
        for label, mod in (("product", product), ("stamped", stamped)):
            fn = mod.get_function(name)
            blocks = []
            for i in range(2):
                a = nc.pack_args(opts, sel, *[b.ptr for b in bufs])
                if label == "stamped":  # alternate buffers; bit 0 asks for the entry reading
                    a.scratch = stamp_bufs[i].ptr | (1 if args.anchor == "start" else 0)
                blocks.append(a)
            params = [nc.kernel_params(name, blk) for blk in blocks]
            graph = nc.Graph.capture(stream, lambda: [fn.launch(tuple(sel.grid), (sel.threads,), params[i % 2],
                                                                stream=stream.handle) for i in range(args.launches)])
            for i in range(args.warmup):
                graph.launch(stream)
                if i % 10 == 9:
                    stream.synchronize()
            stream.synchronize()
            ev0, ev1 = nc.Event(), nc.Event()
            ev0.record(stream.handle)
            for _ in range(10):
                graph.launch(stream)
            ev1.record(stream.handle)
            ev1.synchronize()
            result[f"{label}_us_per_launch"] = round(nc.Event.elapsed(ev0, ev1) * 1e3 / (10 * args.launches), 3)
            ev0.destroy()
            ev1.destroy()
            graph.destroy()
        last = (args.launches - 1) % 2
        stamps = stamp_bufs[last].download(np.uint64, words).reshape(grid, nw, TIMELINE_WORDS)
        result.update(summarize_timeline(stamps))
    finally:
        for b in bufs + stamp_bufs:
            b.free()
        stream.destroy()
    if args.json:
        print(json.dumps(result))
        return 0
    print(f"{result['workload']} -> {name}: {result['product_us_per_launch']} us per launch "
          f"({result['stamped_us_per_launch']} us stamped), clock {result['clock_ghz']} GHz, anchored at the "
          f"wave's {result['anchor']}")
    ws = result["wave_start_us"]
    print(f"waves start at {ws[0]} / {ws[1]} / {ws[2]} us (first / median / last); last wave ends at {result['span_us']} us")
    print(f"{'query block':>11} {'wgs':>4} {'key blocks':>10}  {'loop start':>15}  {'loop end':>15}  {'end':>15}  (us, mean / max)")
    for b in result["blocks"]:
        print(f"{b['query_block']:>11} {b['workgroups']:>4} {b['key_blocks']:>10}  {b['loop_start'][0]:>7.2f} / {b['loop_start'][1]:<5.2f}"
              f"  {b['loop_end'][0]:>7.2f} / {b['loop_end'][1]:<5.2f}  {b['end'][0]:>7.2f} / {b['end'][1]:<5.2f}")
    h = result["heaviest_cycles"]
    print(f"heaviest block, core cycles per wave: prologue {h['prologue']}, key loop {h['key_loop']}, epilogue {h['epilogue']}")
    return 0


def cmd_table(args) -> int:
    recs = []
    for path in args.files:
        with (sys.stdin if path == "-" else open(path)) as f:
            recs.extend(read_records(f))
    print(compare_table(recs))
    return 0


def main(argv: Optional[Sequence[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("flash", help="the reference's four flash smoke cases")
    p = sub.add_parser("compare", help="compare records (JSONL on stdout)")
    p.add_argument("--shapes", choices=("reference", "configs"), default="reference")
    b = sub.add_parser("baselines", help="torch SDPA records for the compare shapes (JSONL on stdout)")
    b.add_argument("--shapes", choices=("reference", "configs"), default="reference")
    b.add_argument("--limit", type=int, default=0, help="only the first N shapes")
    m = sub.add_parser("materialized", help="rocBLAS materialized-attention records for the compare shapes")
    m.add_argument("--shapes", choices=("reference", "configs"), default="reference")
    m.add_argument("--limit", type=int, default=0, help="only the first N shapes")
    for q in (p, b, m, sub.add_parser("profile-flash", help="attributes and occupancy of the c3 kernel"),
              sub.add_parser("benchmark-flash", help="runFlashBenchmark's five cases")):
        q.add_argument("--warmup", type=int, default=5)
        q.add_argument("--iters", type=int, default=20)
    pf = sub.choices["profile-flash"]
    pf.add_argument("--counters", metavar="DIR", default="",
                    help="run under rocprofv3 counter passes, writing them under DIR, and summarise")
    pf.add_argument("--pass-timeout", type=float, default=120.0, help="seconds per profiler pass")
    tl = sub.add_parser("timeline", help="per-wave timeline of the selected kernel (timeline code object)")
    tl.add_argument("--workload", default="c3")
    tl.add_argument("--launches", type=int, default=100, help="launches per graph; stamps come from the last")
    tl.add_argument("--warmup", type=int, default=300, help="untimed graph replays first")
    tl.add_argument("--anchor", choices=("end", "start"), default="end",
                    help="place waves on the chip clock from their end alone (short kernels) or also from a "
                         "reading at entry (long kernels, whose clock moves; costs ~1 us at each wave's start)")
    tl.add_argument("--json", action="store_true")
    t = sub.add_parser("compare-table", help="print the baseline table from JSONL files ('-' = stdin)")
    t.add_argument("files", nargs="+")
    args = ap.parse_args(argv)
    if args.cmd == "compare-table":
        return cmd_table(args)
    if args.cmd == "baselines":
        return cmd_baselines(args)
    if args.cmd == "timeline":
        return cmd_timeline(args)
    if args.cmd == "profile-flash" and args.counters:
        return cmd_profile_counters(args)  # before any GPU call: the passes are child processes
    nc.init()
    module = nc.Module.load_embedded()
    return {"flash": cmd_flash, "compare": cmd_compare, "profile-flash": cmd_profile,
            "benchmark-flash": cmd_benchmark, "materialized": cmd_materialized}[args.cmd](module, args)


if __name__ == "__main__":
    sys.exit(main())
