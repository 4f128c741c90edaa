"""GPU parity of the bf16 kernels (the `_bf16` twin of every variant) through the C ABI against
the oracle run on the same bf16 inputs.

The bf16 path rounds the softmax weights to bf16 (8 significant bits) for the PV product, where the
f16 path keeps 11, so its bar is wider than the f16 one (max-abs 2e-3, max-rel 1e-2):
    max-abs <= 8e-3 (the reference's own flash smoke tolerance, src/main.zig:279)
    max-rel <= 4e-2 (|o - r| / max(|r|, 0.2))
The reference has no bf16 path; these inputs are the f16 cases' seeded draws rounded to bf16.
"""

import math
import re

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import CONFIGS, Workload, sample_rows

pytestmark = pytest.mark.gpu

BF16_MAX_ABS = fc.BF16_MAX_ABS  # 8e-3
BF16_MAX_REL = fc.BF16_MAX_REL  # 4e-2


def bf16(wl: Workload, **kw) -> Workload:
    return Workload(**{**wl.__dict__, "dtype": "bf16", "name": wl.name + "_bf16", **kw})


def _check(gpu, wl: Workload, rows=None, offset=0):
    print(f"[case] {wl.describe()} dtype={wl.dtype} offset={offset}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    out = fc.run_gpu(gpu, wl, q, k, v, o_init, offset=offset)
    idx = fc.active_index(wl, rows)
    ea, er = fc.assert_parity(out, ref, idx, wl.name, max_abs=BF16_MAX_ABS, max_rel=BF16_MAX_REL)
    fc.assert_pads_untouched(out, o_init, wl, wl.name)
    print(f"[ok] {wl.name}: max-abs {ea:.2e} max-rel {er:.2e}", flush=True)
    return ea


@pytest.mark.parametrize("name", ["c1", "c2_causal", "c2_full", "c2_slicepad", "c3"])
def test_configs_bf16(gpu, name):
    _check(gpu, bf16(CONFIGS[name]))


@pytest.mark.parametrize("name", ["c4", "c5"])
def test_large_configs_bf16_row_subset(gpu, name):
    wl = bf16(CONFIGS[name])
    _check(gpu, wl, rows=sample_rows(wl.seq_len, extra=24, seed=wl.seed))


@pytest.mark.parametrize("d", [16, 32, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_ragged_bf16(gpu, d, causal):
    for s in (1, 31, 33, 127, 257, 700):
        wl = Workload(f"bf16_ragged_s{s}_d{d}", 2, s, d, causal, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3,
                      seed=500 + s, dtype="bf16")
        _check(gpu, wl)


@pytest.mark.parametrize("d", [16, 32, 64])
def test_misaligned_base_bf16(gpu, d):
    wl = Workload(f"bf16_misaligned_d{d}", 2, 77, d, True, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3,
                  seed=7, dtype="bf16")
    _check(gpu, wl, offset=1)


def test_large_logits_move_the_running_max_bf16(gpu):
    """sigma-3 Q and K at scale 1: log2-domain scores spread over hundreds, so the bf16 weight limit
    (2^20 per lane and tile) moves the running max many times in every row."""
    wl = Workload("bf16_large_logits", 4, 700, 64, False, 1.0, (("normal", 0.0, 3.0), ("normal", 0.0, 3.0),
                                                                ("uniform", -1.0, 1.0)), seed=11, dtype="bf16")
    _check(gpu, wl)
    wlc = Workload("bf16_large_logits_causal", 2, 1500, 64, True, 1.0, wl.dists, seed=12, dtype="bf16")
    _check(gpu, wlc, rows=sample_rows(1500, extra=32, seed=3))


def test_row_padded_every_tensor_bf16(gpu):
    wl = Workload("bf16_rowpad", 3, 150, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=12, dtype="bf16",
                  q_row=72, k_row=64, v_row=80, o_row=68, q_stride=150 * 72 + 8, o_stride=150 * 68 + 12)
    _check(gpu, wl)


def test_bf16_and_f16_kernels_agree_on_exact_inputs(gpu):
    """Inputs that both types hold exactly (the reference's dyadic pattern fills): the two paths see
    identical Q/K/V and differ only in how the weights are rounded."""
    base = Workload("pattern_both", 4, 300, 64, True, 0.125, (("pattern", 3, 1, 0.125), ("pattern", 5, 2, 0.0625),
                                                              ("pattern", 7, 3, 0.03125)))
    outs = []
    for wl in (base, bf16(base)):
        q, k, v = wl.make_inputs()
        o_init = np.zeros(wl.length("o"), np.float32)
        outs.append(fc.run_gpu(gpu, wl, q, k, v, o_init))
    assert np.max(np.abs(outs[0] - outs[1])) <= BF16_MAX_ABS


def _bf16_variant_names():
    import os

    src = open(os.path.join(os.path.dirname(__file__), "..", "not-cute-zig_amd", "csrc", "flash_fwd.hip")).read()
    return sorted(n + "_bf16" for n in set(re.findall(r"NC_FLASH_(?:PIPE_)?KERNEL(?:_WPE)?\((nc_flash_fwd_\w+),", src)))


@pytest.mark.parametrize("name", _bf16_variant_names())
def test_each_bf16_kernel_variant(gpu, name):
    """Every bf16 code-object variant launched directly on a ragged shape (S = 1100)."""
    d = int(re.search(r"_d(\d+)_", name).group(1))
    causal = "_causal" in name
    m = re.search(r"_q(\d+)s(\d+)(?:p|_)", name)
    bm, threads = (32 * int(m.group(1)), 64 * int(m.group(1)) * int(m.group(2))) if m else (64, 256)
    s = 1100
    wl = Workload(f"variant_{name}", 2, s, d, causal, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3, seed=21,
                  dtype="bf16")
    if "_unaligned" in name:
        wl.q_stride = wl.k_stride = wl.v_stride = s * d + 3
        wl.o_stride = s * d + 5
    print(f"[case] {name} bm={bm} threads={threads}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        sel = nc.KernelSelection()
        sel.block_m = bm
        args = nc.pack_args(wl.options(), sel, *[b.ptr for b in bufs])
        grid = ((wl.seq_len + bm - 1) // bm) * wl.batch_heads
        gpu.get_function(name).launch((grid,), (threads,), [args])
        nc.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
    ea, er = fc.assert_parity(out, ref, fc.active_index(wl), name, max_abs=BF16_MAX_ABS, max_rel=BF16_MAX_REL)
    fc.assert_pads_untouched(out, o_init, wl, name)
    print(f"[ok] {name}: max-abs {ea:.2e} max-rel {er:.2e}", flush=True)


def test_materialized_baseline_bf16(gpu):
    wl = bf16(CONFIGS["c3"])
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    stream = nc.Stream()
    plan = nc.Materialized(stream.handle)
    opts = wl.options()
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    bufs.append(nc.DeviceBuffer(nc.Materialized.workspace_bytes(opts)))
    try:
        plan.run(*bufs[:4], bufs[4], opts)
        stream.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
        plan.destroy()
        stream.destroy()
    ea, er = fc.errors(out, ref, fc.active_index(wl))
    print(f"[ok] materialized bf16 c3: max-abs {ea:.2e} max-rel {er:.2e}", flush=True)
    assert ea <= 0.02
