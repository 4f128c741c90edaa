"""The reference's kernel symbols in the gfx950 code object (src/main_device.zig:19-47), launched
the way the reference's own callers launch them (src/main.zig:822-840, 1024-1035): module
getFunction by name, the 12 kernel parameters (88 bytes), grid (ceil(S/16), batch_heads), block =
the reference's thread count (src/flash.zig:84-95). Parity against the oracle, pads untouched."""

import ctypes

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import REFERENCE_FILLS, Workload, reference_compare_cases, reference_smoke_cases

pytestmark = pytest.mark.gpu

# symbol -> threads per block in the reference (4 warps of 32 = 128, flash_warps = 2 -> 64)
REF_KERNELS = {"flash_attention_fwd_v2": 128, "flash_attention_fwd_h64_bn32": 128, "flash_attention_fwd_h64": 64,
               "flash_attention_fwd_opt": 64, "flash_attention_fwd_h64_causal": 64, "flash_attention_fwd": 64}


def launch_reference_way(mod, name, threads, wl, q, k, v, o_init):
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        params = [ctypes.c_void_p(b.ptr) for b in bufs] + [
            ctypes.c_uint64(wl.seq_len), ctypes.c_uint64(wl.head_dim), ctypes.c_uint64(wl.stride("q")),
            ctypes.c_uint64(wl.stride("k")), ctypes.c_uint64(wl.stride("v")), ctypes.c_uint64(wl.stride("o")),
            ctypes.c_float(wl.scale), ctypes.c_uint32(1 if wl.causal else 0)]
        grid = ((wl.seq_len + 15) // 16, wl.batch_heads)
        mod.get_function(name).launch(grid, (threads,), params)
        nc.synchronize()
        return bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()


CASES = reference_smoke_cases() + reference_compare_cases()[::3] + [
    Workload("ra_neg_scale", 2, 45, 32, True, -0.4, (("normal", 0.0, 1.0),) * 3, seed=31),
    Workload("ra_s1", 3, 1, 64, False, 0.125, (("normal", 0.0, 1.0),) * 3, seed=32),
    Workload("ra_long", 2, 700, 64, True, 0.125, (("normal", 0.0, 2.0),) * 3, seed=33, q_stride=700 * 64 + 5),
    Workload("ra_d16", 4, 130, 16, False, 0.25, REFERENCE_FILLS, o_stride=130 * 16 + 3),
]


@pytest.mark.parametrize("name", sorted(REF_KERNELS))
@pytest.mark.parametrize("wl", CASES, ids=lambda w: w.name)
def test_reference_symbol(gpu, name, wl):
    threads = REF_KERNELS[name]
    print(f"[case] {name} threads={threads} {wl.describe()}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    out = launch_reference_way(gpu, name, threads, wl, q, k, v, o_init)
    fc.assert_parity(out, ref, fc.active_index(wl), f"{name}/{wl.name}")
    fc.assert_pads_untouched(out, o_init, wl, f"{name}/{wl.name}")


def test_reference_symbol_other_block_sizes(gpu):
    """256 threads (four waves) gives the same result; an unsupported head_dim writes nothing."""
    wl = Workload("ra_bs", 2, 300, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=34)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    out = launch_reference_way(gpu, "flash_attention_fwd_h64_bn32", 256, wl, q, k, v, o_init)
    fc.assert_parity(out, ref, fc.active_index(wl), "256 threads")
    bad = Workload("ra_d48", 1, 40, 48, False, 0.1, (("normal", 0.0, 1.0),) * 3, seed=35)
    q, k, v = bad.make_inputs()
    o_init = np.full(bad.length("o"), fc.SENTINEL, dtype=np.float32)
    out = launch_reference_way(gpu, "flash_attention_fwd_opt", 64, bad, q, k, v, o_init)
    assert np.array_equal(out.view(np.uint32), o_init.view(np.uint32))
