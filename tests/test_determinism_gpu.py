"""Repeated-run bitwise determinism on the GPU, one shape per kernel family the dispatcher picks.

LDS races (a missing wait or barrier between ring refills, the split merge and the epilogue stores)
have no sanitizer on this GPU; they would show up as run-to-run differences. Each case runs three
times into a fresh sentinel-filled output and must reproduce the same bits.
"""

import math

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import Workload

pytestmark = pytest.mark.gpu

# (batch_heads, seq_len, head_dim, causal, dtype, base offset in elements)
CASES = [
    (8, 1024, 64, True, "f16", 0),    # private staging, 8 key splits (the c3 kernel)
    (32, 2048, 64, False, "f16", 0),  # shared staging, 8 query waves
    (16, 1024, 64, False, "f16", 0),  # 2 query waves x 4 key splits
    (32, 512, 64, True, "f16", 0),    # 2 query waves x 4 key splits, causal
    (128, 512, 64, True, "f16", 0),   # 4 query waves
    (4, 1500, 32, True, "f16", 0),
    (4, 700, 16, False, "f16", 0),
    (2, 333, 64, True, "f16", 1),     # element-wise (unaligned) kernels
    (8, 1024, 64, True, "bf16", 0),
    (16, 1024, 64, False, "bf16", 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"bh{c[0]}_s{c[1]}_d{c[2]}_{'c' if c[3] else 'n'}_{c[4]}_o{c[5]}")
def test_repeated_runs_are_bitwise_identical(gpu, case):
    bh, s, d, causal, dtype, offset = case
    wl = Workload(f"det_{bh}_{s}_{d}", bh, s, d, causal, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3,
                  seed=77 + s, dtype=dtype)
    sel = nc.select_kernel(wl.options())  # for aligned bases; offset 1 takes the element-wise twin
    print(f"[case] {wl.describe()} dtype={dtype} offset={offset} aligned-base kernel={sel.name.decode()}",
          flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    runs = [fc.run_gpu(gpu, wl, q, k, v, o_init, offset=offset) for _ in range(3)]
    for r in runs[1:]:
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32)), wl.name
    fc.assert_pads_untouched(runs[0], o_init, wl, wl.name)
    assert np.all(np.isfinite(runs[0][fc.active_index(wl)]))
