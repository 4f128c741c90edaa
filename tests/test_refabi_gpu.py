"""The reference's kernel symbols in the gfx950 code object (src/main_device.zig:19-47), launched
the way the reference's own callers launch them (src/main.zig:822-840, 1024-1035): module
getFunction by name, the 12 kernel parameters (88 bytes), grid (ceil(S/16), batch_heads), block =
the reference's thread count (src/flash.zig:84-95).

Each symbol is held to its reference kernel's contract, not to the dispatched path's:
  - flash_attention_fwd_h64_causal ignores its `causal` argument and always masks
    (`_ = causal`, src/flash_h64_causal.zig:34; mask key_row <= q_row, :113-118), so a launch with
    causal = 0 must match the *causal* oracle;
  - flash_attention_fwd_h64, _h64_bn32 and _h64_causal return without writing when head_dim != 64
    (src/flash_h64.zig:35, src/flash_h64_bn32.zig:40, src/flash_h64_causal.zig:35): O stays
    bit-identical to the sentinel it was filled with;
  - flash_attention_fwd_v2, _opt and the legacy flash_attention_fwd accept head_dim 16, 32 and 64
    (src/flash_v2.zig:37, src/flash_opt.zig:31, src/kernels.zig:394) and honour `causal`.
Parity against the oracle, pads untouched."""

import ctypes
import dataclasses

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import REFERENCE_FILLS, Workload, reference_compare_cases, reference_smoke_cases

pytestmark = pytest.mark.gpu

# symbol -> threads per block in the reference (4 warps of 32 = 128, flash_warps = 2 -> 64)
REF_KERNELS = {"flash_attention_fwd_v2": 128, "flash_attention_fwd_h64_bn32": 128, "flash_attention_fwd_h64": 64,
               "flash_attention_fwd_opt": 64, "flash_attention_fwd_h64_causal": 64, "flash_attention_fwd": 64}
D64_ONLY = {"flash_attention_fwd_h64", "flash_attention_fwd_h64_bn32", "flash_attention_fwd_h64_causal"}
ALWAYS_CAUSAL = {"flash_attention_fwd_h64_causal"}


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


def expected(name, wl, q, k, v, o_init):
    """What the reference kernel `name` leaves in O: nothing written (None) outside its head_dim
    domain, else the oracle with the kernel's effective causal flag."""
    if name in D64_ONLY and wl.head_dim != 64:
        return None, wl
    eff = dataclasses.replace(wl, causal=True) if name in ALWAYS_CAUSAL else wl
    return fc.oracle(eff, q, k, v, o_init=o_init), eff


CASES = reference_smoke_cases() + reference_compare_cases()[::3] + [
    Workload("ra_neg_scale", 2, 45, 32, True, -0.4, (("normal", 0.0, 1.0),) * 3, seed=31),
    Workload("ra_s1", 3, 1, 64, False, 0.125, (("normal", 0.0, 1.0),) * 3, seed=32),
    Workload("ra_long", 2, 700, 64, True, 0.125, (("normal", 0.0, 2.0),) * 3, seed=33, q_stride=700 * 64 + 5),
    Workload("ra_long_nc", 2, 300, 64, False, 0.125, (("normal", 0.0, 2.0),) * 3, seed=36),
    Workload("ra_d16", 4, 130, 16, False, 0.25, REFERENCE_FILLS, o_stride=130 * 16 + 3),
    Workload("ra_d32_nc", 2, 96, 32, False, 0.2, (("normal", 0.0, 1.0),) * 3, seed=37),
]


@pytest.mark.parametrize("name", sorted(REF_KERNELS))
@pytest.mark.parametrize("wl", CASES, ids=lambda w: w.name)
def test_reference_symbol(gpu, name, wl):
    threads = REF_KERNELS[name]
    print(f"[case] {name} threads={threads} {wl.describe()}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref, eff = expected(name, wl, q, k, v, o_init)
    out = launch_reference_way(gpu, name, threads, wl, q, k, v, o_init)
    if ref is None:
        assert np.array_equal(out.view(np.uint32), o_init.view(np.uint32)), \
            f"{name}/{wl.name}: head_dim {wl.head_dim} must leave O untouched"
        return
    fc.assert_parity(out, ref, fc.active_index(eff), f"{name}/{wl.name}")
    fc.assert_pads_untouched(out, o_init, eff, f"{name}/{wl.name}")


def test_h64_causal_ignores_causal_flag(gpu):
    """causal = 0 and causal = 1 launches of flash_attention_fwd_h64_causal are bitwise equal, and
    both differ from the non-causal oracle (the mask matters on this input)."""
    wl = Workload("ra_flag", 2, 200, 64, False, 0.125, (("normal", 0.0, 1.0),) * 3, seed=38)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    out0 = launch_reference_way(gpu, "flash_attention_fwd_h64_causal", 64, wl, q, k, v, o_init)
    out1 = launch_reference_way(gpu, "flash_attention_fwd_h64_causal", 64, dataclasses.replace(wl, causal=True),
                                q, k, v, o_init)
    assert np.array_equal(out0.view(np.uint32), out1.view(np.uint32))
    ref_nc = fc.oracle(wl, q, k, v, o_init=o_init)
    ea, _ = fc.errors(out0, ref_nc, fc.active_index(wl))
    assert ea > 0.1, "the causal mask should change this output"


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
    for name in sorted(REF_KERNELS):
        out = launch_reference_way(gpu, name, 64, bad, q, k, v, o_init)
        assert np.array_equal(out.view(np.uint32), o_init.view(np.uint32)), name


# The 128-thread symbols: one workgroup of each pair of 16-row blocks computes both with the
# pipelined body (two key-split waves), and from 16384 workgroups (d=64) one of each group of four
# computes 64 rows (two query waves). S = 8200 and 1040 leave a last pair or group of one block; the
# rotation of the working workgroup covers every one.
COARSE_CASES = [
    Workload("rc_6x4096_c", 6, 4096, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=41),
    Workload("rc_6x4096_n", 6, 4096, 64, False, 0.125, (("normal", 0.0, 1.0),) * 3, seed=42),
    Workload("rc_3x8200_c", 3, 8200, 64, True, 0.125, (("normal", 0.0, 2.0),) * 3, seed=43),
    Workload("rc_24x1040_n", 24, 1040, 64, False, -0.2, (("normal", 0.0, 1.0),) * 3, seed=44),
    Workload("rc_32x8200_c", 32, 8200, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=48),  # 16416: four blocks
    Workload("rc_64x4096_n", 64, 4096, 64, False, 0.125, (("normal", 0.0, 1.0),) * 3, seed=49),  # 16384: four blocks
]


def _sampled(wl, seed):
    from flash_workloads import sample_rows

    return sample_rows(wl.seq_len, extra=24, seed=seed)


@pytest.mark.parametrize("name", ["flash_attention_fwd_h64_bn32", "flash_attention_fwd_v2"])
@pytest.mark.parametrize("wl", COARSE_CASES, ids=lambda w: w.name)
def test_reference_symbol_large_grid(gpu, name, wl):
    grid = (wl.seq_len + 15) // 16 * wl.batch_heads
    print(f"[case] {name} threads=128 {wl.describe()} grid={grid}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    rows = _sampled(wl, 5)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    out = launch_reference_way(gpu, name, 128, wl, q, k, v, o_init)
    fc.assert_parity(out, ref, fc.active_index(wl, rows), f"{name}/{wl.name}")
    fc.assert_pads_untouched(out, o_init, wl, f"{name}/{wl.name}")


def test_reference_symbol_large_grid_fallbacks(gpu):
    """A large grid whose O slices are not float4 aligned takes the 16-row body (same results); one
    narrower than ceil(S/16) blocks writes only the rows its blocks cover, like the reference."""
    wl = Workload("rc_odd_o", 6, 4096, 64, False, 0.125, (("normal", 0.0, 1.0),) * 3, seed=45,
                  o_stride=4096 * 64 + 2)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    rows = _sampled(wl, 6)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    out = launch_reference_way(gpu, "flash_attention_fwd_h64_bn32", 128, wl, q, k, v, o_init)
    fc.assert_parity(out, ref, fc.active_index(wl, rows), wl.name)
    fc.assert_pads_untouched(out, o_init, wl, wl.name)

    wl = Workload("rc_narrow", 7, 4096, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=46)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    gx = (wl.seq_len + 15) // 16 - 3  # 253 x 7 = 1771 workgroups, above the coarse threshold
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        params = [ctypes.c_void_p(b.ptr) for b in bufs] + [
            ctypes.c_uint64(wl.seq_len), ctypes.c_uint64(64), ctypes.c_uint64(wl.stride("q")),
            ctypes.c_uint64(wl.stride("k")), ctypes.c_uint64(wl.stride("v")), ctypes.c_uint64(wl.stride("o")),
            ctypes.c_float(wl.scale), ctypes.c_uint32(1)]
        gpu.get_function("flash_attention_fwd_h64_bn32").launch((gx, wl.batch_heads), (128,), params)
        nc.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
    # blocks 0 .. gx-1 (taken last-first by the causal body) cover rows 0 .. 16*gx-1
    covered = np.arange(0, 16 * gx)
    rows = np.unique(np.concatenate([covered[::97], [16 * gx - 1]]))
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    fc.assert_parity(out, ref, fc.active_index(wl, rows), "narrow grid")
    untouched = fc.active_index(wl, np.arange(16 * gx, wl.seq_len))
    assert np.array_equal(out[untouched].view(np.uint32), o_init[untouched].view(np.uint32))


@pytest.mark.parametrize("name", ["flash_attention_fwd_opt", "flash_attention_fwd_h64", "flash_attention_fwd_h64_causal",
                                  "flash_attention_fwd"])
def test_reference_64_thread_symbols_stage_two_waves(gpu, name):
    """The symbols the reference launches with 64 threads hold LDS for two waves: a 128-thread launch
    (one chunk stream per wave) gives the 64-thread result, and a wider one writes nothing."""
    wl = Workload("ra_w2", 3, 333, 64, name == "flash_attention_fwd_h64_causal", 0.125, (("normal", 0.0, 1.0),) * 3,
                  seed=47)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    for threads in (64, 128):
        print(f"[case] {name} threads={threads}", flush=True)
        out = launch_reference_way(gpu, name, threads, wl, q, k, v, o_init)
        fc.assert_parity(out, ref, fc.active_index(wl), f"{name}/{threads}")
        fc.assert_pads_untouched(out, o_init, wl, f"{name}/{threads}")
    print(f"[case] {name} threads=192", flush=True)
    out = launch_reference_way(gpu, name, 192, wl, q, k, v, o_init)
    assert np.array_equal(out.view(np.uint32), o_init.view(np.uint32)), name


# One-wave launches that take the two-block form (one workgroup of each pair of 16-row blocks runs
# the pipelined body): odd block counts leave a last pair of one block; causal launches take it with
# 8 or more slices or from 512 workgroups.
PAIR_CASES = [
    Workload("rp_d16", 8, 1100, 16, False, 0.25, (("normal", 0.0, 1.0),) * 3, seed=51),
    Workload("rp_d32_c", 8, 1040, 32, True, 1.0 / 32 ** 0.5, (("normal", 0.0, 1.0),) * 3, seed=52),
    Workload("rp_d64", 5, 520, 64, False, -0.125, (("normal", 0.0, 1.0),) * 3, seed=53),
    Workload("rp_d32_c2", 2, 4200, 32, True, 0.2, (("normal", 0.0, 2.0),) * 3, seed=54),
]


@pytest.mark.parametrize("name", ["flash_attention_fwd_opt", "flash_attention_fwd", "flash_attention_fwd_h64",
                                  "flash_attention_fwd_h64_causal"])
@pytest.mark.parametrize("wl", PAIR_CASES, ids=lambda w: w.name)
def test_reference_symbol_two_block_form(gpu, name, wl):
    print(f"[case] {name} threads=64 {wl.describe()}", flush=True)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    if name in D64_ONLY and wl.head_dim != 64:
        out = launch_reference_way(gpu, name, 64, wl, q, k, v, o_init)
        assert np.array_equal(out.view(np.uint32), o_init.view(np.uint32)), name
        return
    eff = dataclasses.replace(wl, causal=True) if name in ALWAYS_CAUSAL else wl
    rows = _sampled(eff, 7)
    ref = fc.oracle(eff, q, k, v, rows=rows, o_init=o_init)
    out = launch_reference_way(gpu, name, 64, wl, q, k, v, o_init)
    fc.assert_parity(out, ref, fc.active_index(eff, rows), f"{name}/{wl.name}")
    fc.assert_pads_untouched(out, o_init, eff, f"{name}/{wl.name}")
