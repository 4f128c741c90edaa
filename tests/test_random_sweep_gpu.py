"""Seeded random-shape parity sweeps on the GPU: batch_heads, seq_len, head_dim, causal, scale
(including negative and zero), row pitch and slice padding, and misaligned base pointers, so every
dispatch route (pipelined private/shared staging, generic, element-wise) meets the oracle on shapes
nobody chose by hand; a second sweep takes many heads over short and mid sequences in f16 and bf16,
where the dispatch picks the four- and eight-query-wave kernels. Rows are checked on a
deterministic subset for the longer sequences."""

import math

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import Workload, sample_rows

pytestmark = pytest.mark.gpu

N_CASES = 160


def random_case(i: int):
    rng = np.random.default_rng(1000 + i)
    d = int(rng.choice([16, 32, 64]))
    bucket = int(rng.choice(3, p=[0.35, 0.35, 0.3]))
    s = int([rng.integers(1, 130), rng.integers(130, 900), rng.integers(900, 4200)][bucket])
    # the long bucket has enough workgroups to route to the shared-staging kernels
    bh = int([rng.integers(1, 12), rng.integers(1, 12), rng.integers(6, 34)][bucket])
    causal = bool(rng.integers(0, 2))
    scale = float(rng.choice([1.0 / math.sqrt(d), 0.5, -0.3, 0.0, 2.0], p=[0.6, 0.15, 0.1, 0.05, 0.1]))
    pad = rng.integers(0, 3)
    rows = {}
    if pad == 1:      # row pitch padded by a multiple of 8 elements (16-byte rows stay aligned)
        rows = dict(q_row=d + 8 * int(rng.integers(1, 4)), k_row=d + 8 * int(rng.integers(0, 3)),
                    v_row=d + 8 * int(rng.integers(0, 3)), o_row=d + 4 * int(rng.integers(0, 3)))
    wl = Workload(f"rand{i}_bh{bh}_s{s}_d{d}_{'c' if causal else 'n'}", bh, s, d, causal, scale,
                  (("normal", 0.0, float(rng.choice([0.5, 1.0, 2.5]))),) * 2 + (("uniform", -1.0, 1.0),),
                  seed=2000 + i, **rows)
    if pad == 2:      # slice strides with odd padding (element-wise kernels)
        wl.q_stride = s * wl.row("q") + int(rng.integers(1, 9))
        wl.k_stride = s * wl.row("k") + int(rng.integers(1, 9))
        wl.v_stride = s * wl.row("v") + int(rng.integers(1, 9))
        wl.o_stride = s * wl.row("o") + int(rng.integers(1, 9))
    offset = int(rng.integers(0, 2)) if pad == 0 else 0  # base one element off 16-byte alignment
    return wl, offset


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape(gpu, i):
    wl, offset = random_case(i)
    sel = nc.select_kernel(wl.options())
    rows = None if wl.seq_len * wl.batch_heads <= 4096 else sample_rows(wl.seq_len, extra=24, seed=i)
    print(f"[case] {wl.describe()} rows={'all' if rows is None else len(rows)} offset={offset} -> "
          f"{sel.name.decode()}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    out = fc.run_gpu(gpu, wl, q, k, v, o_init, offset=offset)
    fc.assert_parity(out, ref, fc.active_index(wl, rows), wl.name)
    fc.assert_pads_untouched(out, o_init, wl, wl.name)


def test_sweep_reaches_every_route():
    """The seeded cases cover the private, shared and generic/element-wise kernel families."""
    names, fams = set(), set()
    for i in range(N_CASES):
        wl, offset = random_case(i)
        n = nc.select_kernel(wl.options()).name.decode()
        names.add(n)
        fams.add("unaligned" if offset or n.endswith("unaligned") else "m64" if "_m64_" in n else
                 "private" if "_q1s" in n else "shared")
    assert {"private", "shared", "unaligned"} <= fams, names


N_WIDE = 48


def random_wide_case(i: int):
    """Many heads over short and mid sequences (the grids where the dispatch prices the four- and
    eight-query-wave kernels), f16 and bf16 alternately, dense or row-padded layouts."""
    rng = np.random.default_rng(5000 + i)
    d = int(rng.choice([16, 32, 64]))
    bh = int(rng.integers(64, 513))
    s = int(rng.integers(40, 700))
    causal = bool(rng.integers(0, 2))
    dtype = "bf16" if i % 2 else "f16"
    rows = {}
    if rng.integers(0, 2):
        rows = dict(q_row=d + 8, k_row=d, v_row=d + 16, o_row=d + 4)
    wl = Workload(f"wide{i}_bh{bh}_s{s}_d{d}_{'c' if causal else 'n'}_{dtype}", bh, s, d, causal, 1.0 / math.sqrt(d),
                  (("normal", 0.0, 1.0),) * 3, seed=6000 + i, dtype=dtype, **rows)
    return wl


@pytest.mark.parametrize("i", range(N_WIDE))
def test_random_wide_shape(gpu, i):
    wl = random_wide_case(i)
    sel = nc.select_kernel(wl.options())
    rows = sample_rows(wl.seq_len, extra=8, seed=i)
    print(f"[case] {wl.describe()} rows={len(rows)} -> {sel.name.decode()}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    out = fc.run_gpu(gpu, wl, q, k, v, o_init)
    max_abs, max_rel = fc.parity_bar(wl.dtype)
    fc.assert_parity(out, ref, fc.active_index(wl, rows), wl.name, max_abs=max_abs, max_rel=max_rel)
    fc.assert_pads_untouched(out, o_init, wl, wl.name)
