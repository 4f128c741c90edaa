"""Host-side tests of the flash harness CLI (not-cute-zig_amd/flash_harness.py): its float64
reference against the CPU oracle, the compare-record format of src/main.zig:859-881, the compare
table of modal_run.py:34-69, and runFlashBenchmark's fills (src/main.zig:787-795)."""

import io
import json
import math

import numpy as np
import pytest

import flash_harness as fh
import flashcheck as fc
from flash_workloads import REFERENCE_FILLS, Workload, reference_smoke_cases


@pytest.mark.parametrize("wl", [
    Workload("h_nc", 2, 37, 16, False, 0.25, (("normal", 0.0, 1.0),) * 3, seed=5),
    Workload("h_c", 3, 70, 32, True, 1.0 / math.sqrt(32), (("normal", 0.0, 2.0),) * 3, seed=6),
    Workload("h_pat", 2, 64, 64, True, 0.125, REFERENCE_FILLS),
] + reference_smoke_cases(), ids=lambda w: w.name)
def test_f64_reference_matches_oracle(wl):
    q, k, v = wl.make_inputs()
    ref = fc.oracle(wl, q, k, v, o_init=np.zeros(wl.length("o"), np.float32))
    mine = fh.attention_f64(wl, q, k, v)
    idx = fc.active_index(wl)
    assert np.max(np.abs(mine[idx] - ref[idx])) < 2e-5
    pad = np.setdiff1d(np.arange(wl.length("o")), idx)
    assert np.all(mine[pad] == 0)


def test_f64_reference_row_subset():
    wl = Workload("h_rows", 2, 300, 32, True, 0.2, (("normal", 0.0, 1.0),) * 3, seed=9)
    q, k, v = wl.make_inputs()
    rows = np.array([0, 1, 17, 150, 299])
    full = fh.attention_f64(wl, q, k, v)
    sub = fh.attention_f64(wl, q, k, v, rows)
    idx = fh.active_index(wl, rows)
    assert np.array_equal(full[idx], sub[idx])


def test_shape_name_and_work_follow_the_reference():
    assert fh.shape_name(8, 1024, 64, True) == "batch_heads=8,seq=1024,head=64,causal=true"
    assert fh.shape_name(2, 32, 16, False) == "batch_heads=2,seq=32,head=16,causal=false"
    # src/main.zig:1032-1034: S(S+1)/2 pairs when causal; Q, K, V f16 + O f32
    assert fh.reference_work(8, 1024, 64, True) == (1074790400, 8 * 1024 * 64 * 10)
    assert fh.reference_work(2, 32, 16, False) == (2 * 4 * 32 * 32 * 16, 2 * 32 * 16 * 10)


def test_record_fields_and_formulas():
    rec = fh.make_record("not_cute", "batch_heads=2,seq=32,head=16,causal=false", True, 0.5, 0.4, 0.7,
                         1_000_000, 2_000_000_000, 1e-4)
    assert tuple(rec) == fh.RECORD_KEYS
    assert rec["gbps"] == pytest.approx(1_000_000 / (0.5 * 1e6))         # src/benchmark.zig:83-85
    assert rec["tflops"] == pytest.approx(2_000_000_000 / (0.5 * 1e9))   # src/benchmark.zig:86-88
    buf = io.StringIO()
    fh.emit(rec, buf)
    line = buf.getvalue()
    assert line.startswith('{"kernel":"flash_attention","implementation":"not_cute","shape":')
    assert json.loads(line) == rec


def test_compare_table_and_reader(capsys):
    mine = fh.make_record("not_cute", "s1", True, 0.010, 0.009, 0.012, 1, 1, 0.0)
    base = fh.make_record("torch_sdpa_flash", "s1", True, 0.030, 0.029, 0.031, 1, 1, 0.001)
    bad = fh.make_record("torch_sdpa_mem_efficient", "s1", False, 0.020, 0.02, 0.02, 1, 1, 0.5)
    lines = [json.dumps(mine), "not json", "{broken", json.dumps(base), json.dumps(bad), json.dumps({"x": 1})]
    recs = fh.read_records(lines)
    assert len(recs) == 3
    # Other output passes silently; a broken object and one without the table's fields are reported.
    err = capsys.readouterr().err.splitlines()
    assert len(err) == 2 and "line 3" in err[0] and "line 6" in err[1] and "mean_ms" in err[1]
    table = fh.compare_table(recs).splitlines()
    flash_row = [r for r in table if "torch_sdpa_flash" in r][0]
    assert "3.00x" in flash_row and flash_row.rstrip().endswith("yes")
    assert [r for r in table if "mem_efficient" in r][0].rstrip().endswith("no")


def test_compare_table_cli(tmp_path, capsys):
    p = tmp_path / "recs.jsonl"
    p.write_text(json.dumps(fh.make_record("not_cute", "s", True, 1.0, 1.0, 1.0, 1, 1, 0.0)) + "\n" +
                 json.dumps(fh.make_record("torch_sdpa_math_f32", "s", True, 4.0, 4.0, 4.0, 1, 1, 0.0)) + "\n")
    assert fh.main(["compare-table", str(p)]) == 0
    assert "4.00x" in capsys.readouterr().out


def test_benchmark_fills():
    # src/main.zig:787-795: ((i*mul + add) % mod) * scale
    q = fh.modular_fill(12, 3, 1, 11, 0.125).view(np.float16).astype(np.float32)
    assert q.tolist() == [((3 * i + 1) % 11) * 0.125 for i in range(12)]
    v = fh.modular_fill(20, 7, 3, 17, 0.03125).view(np.float16).astype(np.float32)
    assert v.tolist() == [((7 * i + 3) % 17) * 0.03125 for i in range(20)]


def test_profile_counter_passes_fit_the_hardware():
    """Each rocprofv3 pass of `profile-flash --counters` stays within one pass's counter budget (at
    most 8 SQ, 4 TCC with FETCH_SIZE taking 3 and WRITE_SIZE 2, 2 GRBM) and never combines --pmc
    with a trace option."""
    import flash_harness as fh

    tcc_cost = {"FETCH_SIZE": 3, "WRITE_SIZE": 2, "TCC_HIT_sum": 1, "TCC_MISS_sum": 1}
    for name, args in fh.COUNTER_PASSES:
        if "--pmc" not in args:
            assert args == ["--kernel-trace", "--stats"], name
            continue
        assert not any(a.startswith("-") and a != "--pmc" for a in args), name
        ctrs = [a for a in args if a != "--pmc"]
        assert sum(c.startswith("SQ_") for c in ctrs) <= 8, name
        assert sum(c.startswith("GRBM_") for c in ctrs) <= 2, name
        assert sum(tcc_cost.get(c, 1) for c in ctrs if c.startswith(("TCC_", "FETCH", "WRITE"))) <= 4, name


def _stamps(waves):
    """Timeline words for waves given as (workgroup, wave, query block, key blocks, clock GHz, counter
    offset, realtime offset in 10 ns ticks, (start, loop start, loop end, end) in us)."""
    nwg = 1 + max(w[0] for w in waves)
    nw = 1 + max(w[1] for w in waves)
    st = np.zeros((nwg, nw, fh.TIMELINE_WORDS), dtype=np.uint64)
    for wg, wv, qb, nblk, ghz, c_off, r_off, times in waves:
        cyc = [int(c_off + t * 1000 * ghz) for t in times]  # core counter at each point
        r_end = r_off + times[3] * 100                     # chip clock (100 MHz) at the end
        sleep = int(ghz * 1000)                             # exactly 100 ticks of the chip clock
        st[wg, wv, :] = [cyc[0], cyc[1], cyc[2], cyc[3], cyc[3] + sleep, int(r_end), int(r_end) + 100,
                         0, nblk, qb, 0, wv, 0]
    return st


def test_timeline_summary_reconstructs_times():
    """Waves on different clocks and core counters (as on different XCDs) are placed on one timebase
    through their end readings; times come out relative to the first wave's start."""
    waves = [
        (0, 0, 3, 4, 2.0, 10_000, 50_000, (0.2, 1.0, 4.0, 5.0)),
        (0, 1, 3, 4, 2.0, 10_000, 50_000, (0.3, 1.1, 4.6, 5.2)),
        (1, 0, 0, 1, 2.4, 77_777, 50_000, (0.0, 0.9, 1.2, 2.5)),
        (1, 1, 0, 1, 2.4, 77_777, 50_000, (0.1, 0.8, 1.1, 2.6)),
    ]
    r = fh.summarize_timeline(_stamps(waves))
    assert r["wave_start_us"][0] == 0.0 and r["wave_start_us"][2] == pytest.approx(0.3, abs=2e-3)
    assert r["span_us"] == pytest.approx(5.2, abs=2e-3)
    by = {b["query_block"]: b for b in r["blocks"]}
    assert by[3]["loop_end"] == pytest.approx([4.3, 4.6], abs=2e-3)
    assert by[3]["end"][1] == pytest.approx(5.2, abs=2e-3) and by[3]["key_blocks"] == 4
    assert by[0]["loop_start"] == pytest.approx([0.85, 0.9], abs=2e-3)
    # the heaviest block is the one with the longest key loop; its per-wave cycles at 2.0 GHz
    assert r["heaviest_cycles"]["key_loop"] == pytest.approx((3.0 + 3.5) / 2 * 2000, abs=2)
    assert r["heaviest_cycles"]["prologue"] == pytest.approx(0.8 * 2000, abs=2)


def test_timeline_summary_start_anchor():
    """With the entry reading (word 12) each wave's clock is its average over its life: a wave whose
    clock at the end differs from its average is still placed correctly."""
    st = _stamps([(0, 0, 1, 2, 2.0, 5_000, 90_000, (0.0, 1.0, 9.0, 10.0)),
                  (1, 0, 0, 2, 2.0, 9_000, 90_000, (2.0, 3.0, 6.0, 7.0))])
    for wg, t_start in ((0, 0.0), (1, 2.0)):
        st[wg, 0, 12] = int(90_000 + t_start * 100)
        st[wg, 0, 6] = st[wg, 0, 5] + 80  # the end-of-wave clock reads 2.5 GHz: not used when anchored
    r = fh.summarize_timeline(st)
    assert r["anchor"] == "start" and r["clock_ghz"] == pytest.approx(2.0, abs=1e-3)
    by = {b["query_block"]: b for b in r["blocks"]}
    assert by[0]["start"][0] == pytest.approx(2.0, abs=2e-3) and by[0]["loop_end"][0] == pytest.approx(6.0, abs=2e-3)
    assert by[1]["end"][0] == pytest.approx(10.0, abs=2e-3)
