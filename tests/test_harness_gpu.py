"""GPU runs of the flash harness commands (not-cute-zig_amd/flash_harness.py) through the C ABI."""

import json
import re

import pytest

import flash_harness as fh
import notcute_flash as nc

pytestmark = pytest.mark.gpu


def _records(text):
    return [json.loads(line) for line in text.splitlines() if line.startswith("{")]


def test_flash_command(gpu, capsys):
    """runFlashAttention's four cases (src/main.zig:189-194) within 0.008, pads untouched."""
    assert fh.main(["flash"]) == 0
    assert capsys.readouterr().err.count("flash attention OK") == 4


def test_compare_command_reference_shapes(gpu, capsys):
    """runCompareDemo's 15 flash shapes (src/main.zig:141-170): one record each, max-abs <= 0.02."""
    assert fh.main(["compare", "--warmup", "2", "--iters", "3"]) == 0
    recs = _records(capsys.readouterr().out)
    assert len(recs) == 15
    for r in recs:
        assert tuple(r) == fh.RECORD_KEYS
        assert r["implementation"] == "not_cute" and r["correct"] and r["max_abs_error"] <= 0.02
        # mean/min/max are f32 in the C result (BenchmarkResult), so allow one rounding step
        assert 0 < r["min_ms"] <= r["mean_ms"] * (1 + 1e-6) and r["mean_ms"] <= r["max_ms"] * (1 + 1e-6)


def test_profile_flash_command(gpu, capsys):
    """runProfileFlash (src/main.zig:81-130): attributes, occupancy limits, then the c3 compare record."""
    assert fh.main(["profile-flash", "--warmup", "1", "--iters", "2"]) == 0
    out = capsys.readouterr().out
    prof = [json.loads(line)["profile"] for line in out.splitlines() if line.startswith('{"profile"')][0]
    sel = nc.select_kernel(nc.options(batch_heads=8, seq_len=1024, head_dim=64, scale=0.125, causal=True))
    assert prof["kernel"] == sel.name.decode()
    assert prof["blocks_per_cu"] >= 1 and prof["waves_per_cu"] == prof["blocks_per_cu"] * sel.threads // 64
    assert prof["static_lds"] == sel.lds_bytes and prof["local"] == 0
    assert prof["cu_count"] >= 1 and prof["device"].startswith("gfx950")
    rec = _records(out)[-1]
    assert rec["shape"] == "batch_heads=8,seq=1024,head=64,causal=true" and rec["correct"]


def test_benchmark_flash_command(gpu, capsys):
    assert fh.main(["benchmark-flash", "--warmup", "1", "--iters", "2"]) == 0
    out = capsys.readouterr().out
    assert out.count("--- Benchmark:") == 5 and out.count("TFLOPs") == 5


def test_baselines_command_in_own_process(gpu):
    """torch SDPA records for the first reference shapes, from a child process (PyTorch brings its
    own HIP runtime); each record carries the reference's fields and a max-abs error."""
    import os
    import subprocess
    import sys

    harness = os.path.join(os.path.dirname(fh.__file__), "flash_harness.py")
    r = subprocess.run([sys.executable, harness, "baselines", "--limit", "3", "--warmup", "1", "--iters", "2"],
                       capture_output=True, text=True, timeout=300)
    print(r.stderr[-2000:])
    assert r.returncode == 0
    recs = _records(r.stdout)
    assert recs and all(tuple(x) == fh.RECORD_KEYS for x in recs)
    assert {x["implementation"] for x in recs} <= set(fh.BASELINE_IMPLS)
    assert any(x["implementation"] == "torch_sdpa_math_f32" and x["correct"] for x in recs)


def test_mfma_ceiling_kernel_closed_form(gpu):
    """The MFMA-ceiling kernel that bench.py times: with every operand 1.0 each 32x32x16 MFMA adds
    16 to every accumulator element, so each thread's sum is 4 accumulators x 16 elements x 2
    MFMAs per iteration x 16 = 2048 per iteration, exactly."""
    import ctypes

    import numpy as np

    fn = gpu.get_function("nc_util_mfma_ceiling")
    ones = np.full(64 * 8, 0x3C00, dtype=np.uint16)  # f16 1.0
    grid, threads, iters = 2, 768, 37
    ops = nc.DeviceBuffer.from_array(ones)
    out = nc.DeviceBuffer(grid * threads * 4)
    try:
        out.memset(0)
        fn.launch((grid,), (threads,), [ctypes.c_void_p(ops.ptr), ctypes.c_uint32(len(ones) // 8),
                                       ctypes.c_void_p(out.ptr), ctypes.c_uint32(iters)])
        nc.synchronize()
        got = out.download(np.float32, grid * threads)
    finally:
        ops.free()
        out.free()
    assert np.all(got == 2048.0 * iters), got[:8]


def test_timeline_command_c3(gpu, capsys):
    """`flash_harness.py timeline` on c3: every query block's waves start, enter and leave their key
    loop and end in that order, the heaviest (last) query blocks end last, and the product kernel
    is the faster of the two copies."""
    assert fh.main(["timeline", "--workload", "c3", "--launches", "20", "--warmup", "20", "--json"]) == 0
    r = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert re.fullmatch(r"nc_flash_fwd_d64_q1s8p2d?_causal", r["kernel"]), r["kernel"]
    assert 1.0 < r["clock_ghz"] < 3.0
    assert r["product_us_per_launch"] < r["stamped_us_per_launch"]
    blocks = {b["query_block"]: b for b in r["blocks"]}
    assert sorted(blocks) == list(range(32)) and all(b["workgroups"] == 8 for b in blocks.values())
    for b in blocks.values():
        assert b["start"][0] <= b["loop_start"][0] <= b["loop_end"][0] <= b["end"][0] <= r["span_us"] + 1e-6
        assert b["key_blocks"] == b["query_block"] // 8 + 1
    assert blocks[31]["end"][1] > blocks[0]["end"][1]
