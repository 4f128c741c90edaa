"""GPU parity: the gfx950 kernels through the C ABI (nc_flash_launch) against the CPU oracle.

Cases: the five benchmark configurations (c4/c5 on a deterministic row subset, exact per row), the
reference's own smoke cases (odd slice pads -> element-wise kernels) and compare cases, ragged
sequence lengths around every tile edge, a misaligned base pointer, large logits, determinism and
padding that must stay untouched.
"""

import math
import sys

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import CONFIGS, Workload, reference_compare_cases, reference_smoke_cases, sample_rows

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(gpu, wl: Workload, rows=None, offset=0, o_fill=fc.SENTINEL, **tol):
    say(f"[case] {wl.describe()} offset={offset} rows={'all' if rows is None else len(rows)}")
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), o_fill, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    out = fc.run_gpu(gpu, wl, q, k, v, o_init, offset=offset)
    idx = fc.active_index(wl, rows)
    ea, er = fc.assert_parity(out, ref, idx, wl.name, **tol)
    fc.assert_pads_untouched(out, o_init, wl, wl.name)
    say(f"[ok] {wl.name}: max-abs {ea:.2e} max-rel {er:.2e}")
    return out, ref


@pytest.mark.parametrize("name", ["c1", "c2_causal", "c2_full", "c2_slicepad", "c3"])
def test_config_full_oracle(gpu, name):
    _check(gpu, CONFIGS[name])


@pytest.mark.parametrize("name", ["c4", "c5"])
def test_config_row_subset(gpu, name):
    wl = CONFIGS[name]
    _check(gpu, wl, rows=sample_rows(wl.seq_len, extra=48, seed=wl.seed))


@pytest.mark.parametrize("name", ["c4", "c5"])
def test_config_every_row(gpu, name):
    """The long-sequence configurations against the full oracle: every row of every slice (the
    oracle runs threaded over (slice, row); c5 is ~5.5e11 flops, a few seconds on 16 host cores)."""
    _check(gpu, CONFIGS[name])


@pytest.mark.parametrize("wl", reference_smoke_cases(), ids=lambda w: w.name)
def test_reference_smoke_cases(gpu, wl):
    """src/main.zig:196-287: O zero-initialised, abs tolerance 0.008 on the active region, the pad
    regions never written."""
    sel = nc.select_kernel(wl.options())
    assert sel.aligned == (1 if all(wl.stride(x) % 8 == 0 for x in "qkv") and wl.stride("o") % 4 == 0 else 0)
    out, ref = _check(gpu, wl, o_fill=np.float32(0.0))
    idx = fc.active_index(wl)
    assert np.max(np.abs(out[idx] - ref[idx])) <= 0.008


@pytest.mark.parametrize("wl", reference_compare_cases(), ids=lambda w: w.name)
def test_reference_compare_cases(gpu, wl):
    """src/main.zig:976-1047: max-abs over the whole (contiguous) output <= 0.02, plus the parity bar."""
    out, ref = _check(gpu, wl, o_fill=np.float32(0.0))
    assert float(np.max(np.abs(out - ref))) <= 0.02


RAGGED = [1, 2, 3, 15, 31, 32, 33, 47, 63, 64, 65, 95, 127, 129, 200, 255, 257, 513]


@pytest.mark.parametrize("d", [16, 32, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_ragged_lengths(gpu, d, causal):
    for s in RAGGED:
        bh = 3 if s < 100 else 2
        wl = Workload(f"ragged_s{s}_d{d}_{'c' if causal else 'n'}", bh, s, d, causal, 1.0 / math.sqrt(d),
                      (("normal", 0.0, 1.0),) * 3, seed=100 + s)
        _check(gpu, wl)


@pytest.mark.parametrize("d", [16, 32, 64])
def test_misaligned_base(gpu, d):
    """Base pointers one element off 16-byte alignment select the element-wise kernels."""
    wl = Workload(f"misaligned_d{d}", 2, 77, d, True, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3, seed=7)
    _check(gpu, wl, offset=1)


def test_large_logits_rescale(gpu):
    """Scores with sigma ~ 72: the running max moves by large steps between key tiles."""
    wl = Workload("large_logits", 4, 700, 64, False, 1.0, (("normal", 0.0, 3.0), ("normal", 0.0, 3.0),
                                                           ("uniform", -1.0, 1.0)), seed=11)
    _check(gpu, wl)


def test_row_padded_every_tensor(gpu):
    wl = Workload("rowpad_mixed", 3, 150, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=12,
                  q_row=72, k_row=64, v_row=80, o_row=68, q_stride=150 * 72 + 8, o_stride=150 * 68 + 12)
    _check(gpu, wl)


def test_deterministic(gpu):
    wl = CONFIGS["c3"]
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    a = fc.run_gpu(gpu, wl, q, k, v, o_init)
    b = fc.run_gpu(gpu, wl, q, k, v, o_init)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_every_kernel_variant(gpu):
    """Each code-object symbol the dispatcher can return exists, and its LDS size matches what the
    selection reports."""
    seen = set()
    for d in (16, 32, 64):
        for causal in (False, True):
            for bh, s in ((1, 32), (4, 1024), (64, 4096)):
                o = nc.options(batch_heads=bh, seq_len=s, head_dim=d, causal=causal)
                sel = nc.select_kernel(o)
                fn = gpu.get_function(sel.name.decode())
                attrs = fn.attributes()
                assert attrs.shared_size_bytes == sel.lds_bytes, sel.name
                assert attrs.local_size_bytes == 0, f"{sel.name} spills to scratch"
                seen.add(sel.name)
    assert len(seen) >= 6


def test_no_kernel_uses_scratch(gpu):
    """No kernel symbol of the code object (every variant, f16 and bf16) spills registers or keeps
    an array in private memory: scratch traffic would cost several times the kernel's time."""
    names = _variant_names()
    names += [n + "_bf16" for n in names]
    for name in names:
        attrs = gpu.get_function(name).attributes()
        assert attrs.local_size_bytes == 0, f"{name} uses {attrs.local_size_bytes} bytes of scratch"
    assert len(names) >= 80


def test_memset_done_before_stream_work(gpu):
    """nc_memset returns once the fill is complete: a kernel launched right after it on a
    non-blocking stream (which does not wait for the null stream the fill runs on) writes over the
    filled bytes, and its writes are what stays. 512 MiB make a late fill overwrite them."""
    import ctypes

    big_bytes, n16 = 512 << 20, 64
    src_words = np.arange(n16 * 4, dtype=np.uint32) + 1
    src = nc.DeviceBuffer.from_array(src_words)
    big = nc.DeviceBuffer(big_bytes)
    stream = nc.Stream()
    fn = gpu.get_function("nc_util_copy_b128")
    try:
        for rep in range(3):
            say(f"[case] memset 512 MiB then copy on a non-blocking stream, rep {rep}")
            big.memset(0xFF)
            fn.launch((1,), (256,), [ctypes.c_void_p(src.ptr), ctypes.c_void_p(big.ptr), ctypes.c_uint64(n16)],
                      stream=stream.handle)
            stream.synchronize()
            head = big.download(np.uint32, n16 * 4)
            tail = big.download(np.uint32, 64, big_bytes - 256)
            assert np.array_equal(head, src_words), f"rep {rep}: the fill landed after the copy"
            assert np.all(tail == 0xFFFFFFFF), f"rep {rep}: the fill did not reach the end"
    finally:
        stream.destroy()
        src.free()
        big.free()


def test_upload_done_before_stream_work(gpu):
    """nc_memcpy_htod returns once the bytes are on the device: a kernel launched right after it on
    a non-blocking stream reads the uploaded tail of a 512 MiB pageable-host copy."""
    import ctypes

    n16 = 64
    host = np.empty((512 << 20) // 4, dtype=np.uint32)
    dst = nc.DeviceBuffer(n16 * 16)
    stream = nc.Stream()
    fn = gpu.get_function("nc_util_copy_b128")
    big = nc.DeviceBuffer(host.nbytes)
    try:
        for rep in range(3):
            say(f"[case] upload 512 MiB then copy its tail on a non-blocking stream, rep {rep}")
            host[:] = np.uint32(0x01010101 * (rep + 1))
            big.upload(host)
            fn.launch((1,), (256,), [ctypes.c_void_p(big.ptr + host.nbytes - n16 * 16), ctypes.c_void_p(dst.ptr),
                                     ctypes.c_uint64(n16)], stream=stream.handle)
            stream.synchronize()
            got = dst.download(np.uint32, n16 * 4)
            assert np.all(got == np.uint32(0x01010101 * (rep + 1))), f"rep {rep}: the kernel read before the upload"
    finally:
        stream.destroy()
        dst.free()
        big.free()


def test_launch_rejects_short_buffers(gpu):
    wl = CONFIGS["c1"]
    q, k, v = wl.make_inputs()
    dq, dk, dv = (nc.DeviceBuffer.from_array(x) for x in (q, k, v))
    do = nc.DeviceBuffer(wl.length("o") * 4)
    with pytest.raises(nc.NcError) as ei:
        nc.flash_launch(gpu, dq, dk, dv, do, wl.options(), o_len=wl.length("o") - 1)
    assert ei.value.name == "InvalidValue"
    for b in (dq, dk, dv, do):
        b.free()


def _variant_names():
    import re
    import os
    src = open(os.path.join(os.path.dirname(__file__), "..", "not-cute-zig_amd", "csrc", "flash_fwd.hip")).read()
    return sorted(set(re.findall(r"NC_FLASH_(?:PIPE_)?KERNEL(?:_WPE)?\((nc_flash_fwd_\w+),", src)))


@pytest.mark.parametrize("name", _variant_names())
def test_each_kernel_variant_parity(gpu, name):
    """Every code-object variant, launched directly (not only those the dispatcher picks for the
    standard shapes), on a ragged causal/non-causal shape."""
    import re

    d = int(re.search(r"_d(\d+)_", name).group(1))
    causal = "_causal" in name
    m = re.search(r"_q(\d+)s(\d+)(?:p\d+(?:t\d+)?x?)?_", name)
    bm, threads = (32 * int(m.group(1)), 64 * int(m.group(1)) * int(m.group(2))) if m else (64, 256)
    # S = 1100: every wave of every variant (up to 512 keys per staged block) steps through
    # several blocks, so ring reuse and refills are exercised; S is not a multiple of any tile.
    s = 1100
    wl = Workload(f"variant_{name}", 2, s, d, causal, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3, seed=21)
    if name.endswith("_unaligned"):
        wl.q_stride = wl.k_stride = wl.v_stride = s * d + 3
        wl.o_stride = s * d + 5
    say(f"[case] {name} bm={bm} threads={threads}")
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
    ea, er = fc.assert_parity(out, ref, fc.active_index(wl), name)
    fc.assert_pads_untouched(out, o_init, wl, name)
    say(f"[ok] {name}: max-abs {ea:.2e} max-rel {er:.2e}")
