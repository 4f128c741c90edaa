"""GPU tests of the materialized-attention baseline (rocBLAS QK^T -> softmax kernel -> PV,
tools/cuda_baselines.cu:689-759) against the CPU oracle.

The baseline rounds the normalised probabilities to f16 before the PV product, so its error is
larger than the fused path's; the reference accepts it at 0.08 max-abs (tools/cuda_baselines.cu:759).
These tests hold it to the compare tolerance, 0.02 (src/main.zig:1042), and check that only the
active S x d region of each O slice is written.
"""

import math
import os
import subprocess
import sys

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import CONFIGS, Workload, reference_compare_cases, sample_rows

pytestmark = pytest.mark.gpu

TOL = 0.02
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def plan(gpu):
    stream = nc.Stream()
    p = nc.Materialized(stream.handle)
    yield p, stream
    p.destroy()
    stream.destroy()


def _run(plan, wl: Workload, rows=None):
    p, stream = plan
    print(f"[case] materialized {wl.describe()} rows={'all' if rows is None else len(rows)}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    opts = wl.options()
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    bufs.append(nc.DeviceBuffer(nc.Materialized.workspace_bytes(opts)))
    try:
        p.run(*bufs[:4], bufs[4], opts)
        stream.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
    idx = fc.active_index(wl, rows)
    ea, er = fc.errors(out, ref, idx)
    fc.assert_pads_untouched(out, o_init, wl, wl.name)
    print(f"[ok] materialized {wl.name}: max-abs {ea:.2e} max-rel {er:.2e}", flush=True)
    assert ea <= TOL, (wl.name, ea)
    return ea


@pytest.mark.parametrize("name", ["c1", "c2_causal", "c2_full", "c2_slicepad", "c3"])
def test_configs(plan, name):
    _run(plan, CONFIGS[name])


def test_c4_row_subset(plan):
    wl = CONFIGS["c4"]
    _run(plan, wl, rows=sample_rows(wl.seq_len, extra=16, seed=wl.seed))


@pytest.mark.parametrize("wl", reference_compare_cases(), ids=lambda w: w.name)
def test_reference_compare_cases(plan, wl):
    _run(plan, wl)


@pytest.mark.parametrize("d", [16, 32, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_ragged_and_softmax_geometries(plan, d, causal):
    """S across every softmax geometry (64 lanes x 1..8 scores, 256 x 4..32, 1024 x 16..32)."""
    for s in (1, 33, 65, 511, 513, 1000, 8193):
        bh = 2 if s < 4096 else 1
        wl = Workload(f"mat_s{s}_d{d}_{'c' if causal else 'n'}", bh, s, d, causal, 1.0 / math.sqrt(d),
                      (("normal", 0.0, 1.0),) * 3, seed=300 + s)
        rows = None if s <= 1000 else sample_rows(s, extra=8, seed=s)
        _run(plan, wl, rows=rows)


def test_row_padded_every_tensor(plan):
    wl = Workload("mat_rowpad", 3, 150, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=12,
                  q_row=72, k_row=64, v_row=80, o_row=68, q_stride=150 * 72 + 8, o_stride=150 * 68 + 12)
    _run(plan, wl)


def test_rejects_short_workspace_on_device(plan):
    p, _ = plan
    wl = CONFIGS["c1"]
    q, k, v = wl.make_inputs()
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v)] + [nc.DeviceBuffer(wl.length("o") * 4)]
    ws = nc.DeviceBuffer(nc.Materialized.workspace_bytes(wl.options()) - 2)
    try:
        with pytest.raises(nc.NcError) as ei:
            p.run(*bufs, ws, wl.options())
        assert ei.value.name == "InvalidValue"
    finally:
        for b in bufs + [ws]:
            b.free()


def test_harness_materialized_command():
    """`flash_harness.py materialized`: records with the reference's fields plus workspace_bytes."""
    import json

    cmd = [sys.executable, os.path.join(ROOT, "not-cute-zig_amd", "flash_harness.py"), "materialized",
           "--limit", "4", "--warmup", "1", "--iters", "3"]
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stderr
    recs = [json.loads(line) for line in p.stdout.splitlines() if line.startswith("{")]
    assert len(recs) == 4
    for r in recs:
        assert r["implementation"] == "rocblas_materialized" and r["correct"]
        bh, s = (int(x.split("=")[1]) for x in r["shape"].split(",")[:2])
        assert r["workspace_bytes"] == bh * s * s * 6
        assert r["min_ms"] <= r["mean_ms"] * (1 + 1e-6) and r["mean_ms"] <= r["max_ms"] * (1 + 1e-6)
