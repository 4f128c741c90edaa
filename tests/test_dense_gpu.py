"""The dense-layout private-staging kernels (q1s8p1d, q1s8p2d): nc_flash_launch picks them for packed
slices. Each must match the oracle and its strided twin bit for bit (same tiles, same order), for
batch_heads a multiple of 8 (grid (8, BH/8, nqb)) and not (grid (BH, 1, nqb)), both element types;
their one-parameter-per-field form must also launch by name and inside a captured graph.
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

DENSE_RE = re.compile(r"_q1s8p\dd_")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _run_by_name(gpu, name, wl, bufs, grid):
    """Launch kernel `name` on `bufs` with the argument block for `wl` (its own parameter form)."""
    sel = nc.KernelSelection()
    sel.block_m = 32
    args = nc.pack_args(wl.options(), sel, *[b.ptr for b in bufs])
    gpu.get_function(name).launch(grid, (512,), nc.kernel_params(name, args))
    nc.synchronize()
    return bufs[3].download(np.float32, wl.length("o"))


# (d, BH, S, causal): one- and two-stage picks, BH a multiple of 8 and not, S ragged.
CASES = [
    (64, 8, 1024, True), (64, 3, 1100, True), (64, 16, 500, False), (64, 5, 300, True),
    (32, 8, 777, True), (32, 6, 1500, False), (16, 8, 640, False), (16, 1, 32, False), (16, 9, 2000, True),
]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"d{c[0]}_bh{c[1]}_s{c[2]}_{'c' if c[3] else 'n'}")
def test_dense_kernel_matches_oracle_and_strided_twin(gpu, case, dtype):
    d, bh, s, causal = case
    wl = Workload(f"dense_d{d}", bh, s, d, causal, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3,
                  seed=70 + d + bh, dtype=dtype)
    sel = nc.select_kernel(wl.options())
    name = sel.name.decode()
    say(f"[case] {wl.describe()} {dtype} -> {name} grid {tuple(sel.grid)}")
    if not DENSE_RE.search(name):
        pytest.skip(f"{name} is not a dense-layout kernel for this shape")
    nqb = -(-s // 32)
    assert tuple(sel.grid) == ((8, bh // 8, nqb) if bh % 8 == 0 else (bh, 1, nqb))
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    out = fc.run_gpu(gpu, wl, q, k, v, o_init)
    bar_abs, bar_rel = fc.parity_bar(dtype)
    ea, er = fc.assert_parity(out, ref, fc.active_index(wl), name, max_abs=bar_abs, max_rel=bar_rel)
    fc.assert_pads_untouched(out, o_init, wl, name)
    twin = DENSE_RE.sub(lambda m: m.group(0)[:-2] + "_", name)
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        tw = _run_by_name(gpu, twin, wl, bufs, (nqb * bh,))
    finally:
        for b in bufs:
            b.free()
    assert np.array_equal(out.view(np.uint32), tw.view(np.uint32)), f"{name} differs from {twin}"
    say(f"[ok] {name}: max-abs {ea:.2e} max-rel {er:.2e}, bitwise equal to {twin}")


def test_dense_kernel_by_name_and_in_a_graph(gpu):
    """The one-parameter-per-field form launched by name with nc.kernel_params, and captured into a
    graph through nc_flash_launch_async and replayed, against the eager result."""
    wl = Workload("dense_graph", 8, 1024, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=77)
    sel = nc.select_kernel(wl.options())
    name = sel.name.decode()
    assert DENSE_RE.search(name), name
    say(f"[case] {wl.describe()} -> {name}, by name and in a graph")
    q, k, v = wl.make_inputs()
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v)] + [nc.DeviceBuffer(wl.length("o") * 4)]
    stream = nc.Stream()
    graph = None
    try:
        bufs[3].memset(0)
        nc.synchronize()
        nc.flash_launch(gpu, *bufs, wl.options(), stream=stream.handle)
        stream.synchronize()
        ref = bufs[3].download(np.float32, wl.length("o"))
        bufs[3].memset(0)
        nc.synchronize()
        by_name = _run_by_name(gpu, name, wl, bufs, tuple(sel.grid))
        assert np.array_equal(by_name.view(np.uint32), ref.view(np.uint32))
        graph = nc.Graph.capture(stream, lambda: [nc.flash_launch(gpu, *bufs, wl.options(), stream=stream.handle)
                                                  for _ in range(3)])
        for r in range(3):
            bufs[3].memset(0)
            nc.synchronize()
            graph.launch(stream)
            stream.synchronize()
            out = bufs[3].download(np.float32, wl.length("o"))
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), f"replay {r}"
        say("[ok] by name and three graph replays bitwise equal to the eager launch")
    finally:
        if graph is not None:
            graph.destroy()
        stream.destroy()
        for b in bufs:
            b.free()
