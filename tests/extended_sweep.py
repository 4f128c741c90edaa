"""Extended random-shape parity sweep, run by hand on a GPU (pytest does not collect this file).

Runs cases N0..N1-1 of the committed sweep's generator (`random_case` in
tests/test_random_sweep_gpu.py), odd cases with bf16 inputs. Each case is checked against the CPU
oracle with its element type's parity bar, and the padding must be left untouched. Prints every
failure and, per dispatched kernel, the worst error as a fraction of the bar.

    python tests/extended_sweep.py 160 1760
"""

import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("not-cute-zig_amd", "oracle", "tests"):
    sys.path.insert(0, os.path.join(ROOT, sub))

import numpy as np  # noqa: E402

import flashcheck as fc  # noqa: E402
import notcute_flash as nc  # noqa: E402
from flash_workloads import sample_rows  # noqa: E402
from test_random_sweep_gpu import random_case  # noqa: E402


def main(n0: int, n1: int) -> int:
    nc.load_library()
    nc.init()
    mod = nc.Module.load_embedded()
    worst, fails, t0 = {}, 0, time.time()
    for i in range(n0, n1):
        wl, offset = random_case(i)
        if i % 2:
            wl.dtype = "bf16"
        sel = nc.select_kernel(wl.options()).name.decode()
        rows = None if wl.seq_len * wl.batch_heads <= 4096 else sample_rows(wl.seq_len, extra=24, seed=i)
        q, k, v = wl.make_inputs()
        o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
        ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
        out = fc.run_gpu(mod, wl, q, k, v, o_init, offset=offset)
        idx = fc.active_index(wl, rows)
        ea, er = fc.errors(out, ref, idx)
        bar_abs, bar_rel = fc.parity_bar(wl.dtype)
        mask = np.ones(out.size, bool)
        mask[fc.active_index(wl)] = False
        pads_ok = np.array_equal(out[mask].view(np.uint32), o_init[mask].view(np.uint32))
        ok = bool(np.isfinite(out[idx]).all()) and ea <= bar_abs and er <= bar_rel and pads_ok
        key = sel.replace("nc_flash_fwd_", "")
        w = worst.get(key, (0.0, 0.0, 0))
        worst[key] = (max(w[0], ea / bar_abs), max(w[1], er / bar_rel), w[2] + 1)
        if not ok:
            fails += 1
            print(f"FAIL case {i} {wl.describe()} dtype={wl.dtype} offset={offset} {sel}: max-abs {ea:.3e} "
                  f"max-rel {er:.3e} pads_ok={pads_ok}", flush=True)
        if (i - n0) % 200 == 199:
            print(f"progress: {i - n0 + 1} cases, {fails} failures, {time.time() - t0:.0f} s", flush=True)
    print(f"done: {n1 - n0} cases, {fails} failures")
    for key in sorted(worst):
        a, r, n = worst[key]
        print(f"  {key:34s} cases {n:4d}  worst max-abs {a:.2f} of bar, worst max-rel {r:.2f} of bar")
    mod.unload()
    return 1 if fails else 0


if __name__ == "__main__":
    sys.exit(main(int(sys.argv[1]), int(sys.argv[2])))
