"""Wave balancing of the grid's last workgroups (nc_flash_kernel_args.balance_tail).

The non-causal shared-staging kernels order their waves by remaining key blocks in the grid's last
`balance_tail` workgroups. That changes only which wave the SIMD issues next, never what a wave
computes, so the output must be bitwise the same for every tail; and nc_flash_pack_args must set
the tail only where it is meant to (more workgroups than CUs, non-causal, a kernel marked for it).
"""

import math

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import CONFIGS, Workload

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)


# The kernels whose dispatch enables balancing, with their workgroups per CU (flash.cpp kPipeModels).
BALANCED = {
    "nc_flash_fwd_d64_q8s1p2t2_full": 2,
    "nc_flash_fwd_d64_q4s1p2t2_full": 4,
    "nc_flash_fwd_d64_q2s4p2_full": 2,
    "nc_flash_fwd_d32_q2s4p2_full": 2,
}


def _geometry(name: str):
    import re

    m = re.search(r"_q(\d+)s(\d+)p\d+(?:t\d+)?_", name)
    nq, ns = int(m.group(1)), int(m.group(2))
    return 32 * nq, 64 * nq * ns


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("name", sorted(BALANCED))
def test_balanced_output_is_bitwise_the_same(gpu, name, bf16):
    """Tail 0 (no balancing), part of the grid, and all of it: the same bits, and oracle parity."""
    import re
    import dataclasses

    d = int(re.search(r"_d(\d+)_", name).group(1))
    bm, threads = _geometry(name)
    # S = 1100 is ragged for every block size; 5 heads make a grid of 10-45 workgroups.
    wl = Workload(f"balance_{name}", 5, 1100, d, False, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3, seed=31)
    if bf16:
        wl = dataclasses.replace(wl, dtype="bf16")
    kname = name + ("_bf16" if bf16 else "")
    grid = ((wl.seq_len + bm - 1) // bm) * wl.batch_heads
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    rows = np.unique(np.concatenate([np.arange(0, wl.seq_len, 37), [wl.seq_len - 1]]))
    ref = fc.oracle(wl, q, k, v, rows=rows)
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    outs = {}
    try:
        fn = gpu.get_function(kname)
        for tail in (0, grid // 2, grid):
            say(f"[case] {kname} grid={grid} balance_tail={tail}")
            bufs[3].upload(o_init)
            sel = nc.KernelSelection()
            sel.block_m = bm
            args = nc.pack_args(wl.options(), sel, *[b.ptr for b in bufs])
            assert args.balance_tail == 0  # a selection without a table name gets none
            args.balance_tail = tail
            fn.launch((grid,), (threads,), [args])
            nc.synchronize()
            outs[tail] = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
    base = outs[0]
    for tail, out in outs.items():
        assert np.array_equal(out.view(np.uint32), base.view(np.uint32)), (kname, tail)
    ea, er = fc.assert_parity(base, ref, fc.active_index(wl, rows), kname)
    fc.assert_pads_untouched(base, o_init, wl, kname)
    say(f"[ok] {kname}: bitwise equal over tails 0/{grid // 2}/{grid}, max-abs {ea:.2e} max-rel {er:.2e}")


def test_pack_args_sets_the_tail_where_it_applies(gpu):
    """c4 (512 workgroups of the q8s1 kernel) balances its last 2 x CUs; one workgroup per CU, a
    causal grid, and the private-staging c3 kernel get none."""
    cus = nc.device_attributes().sm_count
    assert cus > 0

    def tail_of(opts):
        sel = nc.select_kernel(opts)
        a = nc.pack_args(opts, sel, 0x1000, 0x2000, 0x3000, 0x4000)
        return sel.name.decode(), sel.grid[0], a.balance_tail

    name, grid, tail = tail_of(CONFIGS["c4"].options())
    say(f"[case] c4 -> {name} grid={grid} cus={cus} tail={tail}")
    if name in BALANCED and grid > cus:
        assert tail == min(grid, BALANCED[name] * cus)
    else:
        assert tail == 0
    if name == "nc_flash_fwd_d64_q8s1p2t2_full" and cus == 256:
        assert tail == 512
    for key in ("c3", "c5"):
        n, g, t = tail_of(CONFIGS[key].options())
        say(f"[case] {key} -> {n} grid={g} tail={t}")
        assert t == 0, key
    # as many workgroups as CUs: nothing to balance
    opts = CONFIGS["c4"].options()
    opts.batch_heads = max(1, cus * 256 // 4096)
    n, g, t = tail_of(opts)
    say(f"[case] BH={opts.batch_heads} S=4096 -> {n} grid={g} tail={t}")
    if g <= cus:
        assert t == 0
