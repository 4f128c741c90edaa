"""GPU parity where the lazy running max has to move on the tile *sum*, not on an overflowed weight.

Key tile t (32 keys) sits 12.3 * t log2-units above tile 0, so each tile's weights are ~5000x the
previous tile's: each stays far below f16's 65504, but a lane's 16 weights sum past it. In every
third tile only 8 keys take the new level (the rest stay at the previous one), so lane sums stay
under 65504 and weights of ~5000 are carried into f16 unscaled; the tile after that is two levels
up, where single weights overflow f16.
- Kernels that add the f32 weights for the row sum must take a lane sum of 65504 or more as the
  sign to move the max (a weight that rounds to infinity is >= 65520).
- Kernels that add the rounded weights move it only on an infinite sum.
Every path must match the oracle.
"""

import math
import re
import sys

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import Workload

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _bf16_bits(x):
    """f32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).ravel()


def _inputs(bh, s, d, scale, seed, dtype="f16"):
    """Q rows = 16 e0 (+ small noise in the other columns); key j of tile t = j // 32 is
    e0 * 12.3 L / (16 sc) with level L = t, except L = t - 1 for keys 8..31 of every third tile."""
    rng = np.random.default_rng(seed)
    sc = scale * LOG2E
    q = np.zeros((bh, s, d), np.float32)
    q[:, :, 0] = 16.0
    q[:, :, 1:] = rng.normal(0.0, 0.05, (bh, s, d - 1))
    k = np.zeros((bh, s, d), np.float32)
    j = np.arange(s)
    t = j // 32
    level = np.where((t % 3 == 2) & ((j % 32) >= 8), t - 1, t)
    k[:, :, 0] = (12.3 * level / (16.0 * sc))[None, :]
    k[:, :, 1:] = rng.normal(0.0, 0.05, (bh, s, d - 1))
    v = rng.normal(0.0, 1.0, (bh, s, d)).astype(np.float32)
    enc = _bf16_bits if dtype == "bf16" else (lambda x: x.astype(np.float16).view(np.uint16).ravel())
    return enc(q), enc(k), enc(v)


def _workload(name, bh, s, d, causal, dtype="f16"):
    wl = Workload(name, bh, s, d, causal, 0.125, (("normal", 0.0, 1.0),) * 3, seed=0)
    wl.dtype = dtype
    return wl


@pytest.mark.parametrize("causal", [False, True])
def test_tile_sum_moves_the_max_dispatched(gpu, causal):
    wl = _workload("tile_sum", 2, 320, 64, causal)
    q, k, v = _inputs(2, 320, 64, wl.scale, 31)
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    say(f"[case] tile-sum dispatched causal={causal} -> {nc.select_kernel(wl.options()).name.decode()}")
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    out = fc.run_gpu(gpu, wl, q, k, v, o_init)
    ea, er = fc.assert_parity(out, ref, fc.active_index(wl), wl.name)
    say(f"[ok] max-abs {ea:.2e} max-rel {er:.2e}")


def _d64_variants():
    import os
    src = open(os.path.join(os.path.dirname(__file__), "..", "not-cute-zig_amd", "csrc", "flash_fwd.hip")).read()
    names = sorted(set(re.findall(r"NC_FLASH_PIPE_KERNEL(?:_WPE)?\((nc_flash_fwd_d64_\w+),", src)))
    return names + [n + "_bf16" for n in names]


@pytest.mark.parametrize("name", _d64_variants())
def test_tile_sum_moves_the_max_every_d64_variant(gpu, name):
    causal = "_causal" in name
    dtype = "bf16" if name.endswith("_bf16") else "f16"
    m = re.search(r"_q(\d+)s(\d+)p\d+(?:t\d+)?_", name)
    bm, threads = 32 * int(m.group(1)), 64 * int(m.group(1)) * int(m.group(2))
    s = 600
    wl = _workload(f"tile_sum_{name}", 2, s, 64, causal, dtype)
    q, k, v = _inputs(2, s, 64, wl.scale, 32, dtype)
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    say(f"[case] tile-sum {name} bm={bm} threads={threads}")
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        sel = nc.KernelSelection()
        sel.block_m = bm
        args = nc.pack_args(wl.options(), sel, *[b.ptr for b in bufs])
        grid = ((s + bm - 1) // bm) * wl.batch_heads
        gpu.get_function(name).launch((grid,), (threads,), [args])
        nc.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
    bar_abs, bar_rel = fc.parity_bar(dtype)
    ea, er = fc.assert_parity(out, ref, fc.active_index(wl), name, max_abs=bar_abs, max_rel=bar_rel)
    fc.assert_pads_untouched(out, o_init, wl, name)
    say(f"[ok] {name}: max-abs {ea:.2e} max-rel {er:.2e}")
