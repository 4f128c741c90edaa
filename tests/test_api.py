"""Host-side tests of the C ABI (no GPU calls): exported symbols, flash.Options validation
(src/flash.zig:16-28), requireLen (src/flash.zig:98-100), the restated reference dispatch table
(src/flash.zig:78-96), the MI355X dispatch geometry, the work model (src/main.zig:1032-1034), the
benchmark arithmetic (src/benchmark.zig:80-89), error mapping (src/cuda.zig:134-178) and the CLI
guard of bench.py."""

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import notcute_flash as nc
from flash_workloads import CONFIGS

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "notcute_flash.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = nc.load_library()
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_oracle_library_loads():
    import flash_oracle

    assert hasattr(flash_oracle.lib(), "oracle_flash_fwd")


def test_product_does_not_import_oracle():
    pkg = os.path.join(ROOT, "not-cute-zig_amd")
    for fn in os.listdir(pkg):
        if fn.endswith(".py"):
            src = open(os.path.join(pkg, fn)).read()
            assert "flash_oracle" not in src and "oracle/" not in src, fn


def test_status_names_follow_cuda_error_order():
    # CudaError members in declaration order, src/cuda.zig:134-151
    ref = ["OutOfMemory", "Overflow", "SharedObjectInitFailed", "NotFound", "InvalidValue", "InvalidContext",
           "InvalidDevice", "InvalidImage", "ContextIsDestroyed", "LaunchFailed", "LaunchOutOfResources",
           "LaunchTimeout", "IllegalAddress", "NoDevice", "NotInitialized", "UnknownError"]
    lib = nc.load_library()
    assert lib.nc_status_name(0) == b"Success"
    for i, name in enumerate(ref, start=1):
        assert lib.nc_status_name(i).decode() == name
    assert lib.nc_status_name(99) == b"UnknownError"


def test_hip_error_mapping():
    lib = nc.load_library()
    # hipError_t values from hip_runtime_api.h
    table = {0: "Success", 2: "OutOfMemory", 1: "InvalidValue", 100: "NoDevice", 3: "NotInitialized",
             200: "InvalidImage", 303: "SharedObjectInitFailed", 500: "NotFound", 700: "IllegalAddress",
             701: "LaunchOutOfResources", 702: "LaunchTimeout", 709: "ContextIsDestroyed", 719: "LaunchFailed",
             101: "InvalidDevice", 201: "InvalidContext", 999: "UnknownError"}
    for hip, name in table.items():
        assert nc.STATUS_NAMES[lib.nc_status_from_hip(hip)] == name, hip


def test_init_without_gpu_reports_no_device():
    if nc.device_count() != 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(nc.NcError) as ei:
        nc.init()
    assert ei.value.name == "NoDevice"


def _opts(**kw):
    base = dict(batch_heads=2, seq_len=64, head_dim=32)
    base.update(kw)
    return nc.options(**base)


def _status(o):
    return nc.STATUS_NAMES[nc.load_library().nc_flash_validate(ctypes.byref(o))]


def test_options_defaults_match_reference():
    o = nc.FlashOptions()
    nc.load_library().nc_flash_options_init(ctypes.byref(o))
    assert o.batch_heads == 1 and o.causal == 0  # src/flash.zig:6,14
    assert o.q_row_stride == o.k_row_stride == o.v_row_stride == o.o_row_stride == 0


@pytest.mark.parametrize("d", [1, 8, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 96, 128])
def test_validate_head_dim(d):
    want = "Success" if d in (16, 32, 64) else "InvalidValue"
    assert _status(_opts(head_dim=d)) == want


def test_validate_zero_batch_or_seq():
    assert _status(_opts(batch_heads=0)) == "InvalidValue"
    assert _status(_opts(seq_len=0)) == "InvalidValue"


@pytest.mark.parametrize("which", ["q", "k", "v", "o"])
def test_validate_slice_strides(which):
    s, d = 64, 32
    assert _status(_opts(**{f"{which}_stride": s * d})) == "Success"
    assert _status(_opts(**{f"{which}_stride": s * d - 1})) == "InvalidValue"
    assert _status(_opts(**{f"{which}_stride": s * d + 17})) == "Success"


@pytest.mark.parametrize("which", ["q", "k", "v", "o"])
def test_validate_row_strides(which):
    s, d = 64, 32
    # row stride below head_dim
    assert _status(_opts(**{f"{which}_row_stride": d - 1, f"{which}_stride": 10 * s * d})) == "InvalidValue"
    # padded rows need (S-1)*row + d elements per slice
    row = 40
    need = (s - 1) * row + d
    assert _status(_opts(**{f"{which}_row_stride": row, f"{which}_stride": need})) == "Success"
    assert _status(_opts(**{f"{which}_row_stride": row, f"{which}_stride": need - 1})) == "InvalidValue"


def test_validate_overflow():
    o = _opts(batch_heads=1 << 40, q_stride=1 << 30)
    assert _status(o) == "Overflow"


def test_select_grid_within_dispatch_limit():
    """A dispatch packet holds each grid dimension in work-items as 32 bits: the selection refuses a
    grid past 2^32 - 1 threads in x (2^24 one-block slices of workgroups of at least 256 threads) and
    keeps every accepted grid within it."""
    def sel(bh, **kw):
        return nc.options(batch_heads=bh, seq_len=32, head_dim=16, **kw)

    for kw in ({}, dict(q_stride=40 * 32, k_stride=40 * 32, v_stride=40 * 32, o_stride=40 * 32)):
        with pytest.raises(nc.NcError) as e:
            nc.select_kernel(sel(1 << 24, **kw))
        assert e.value.name == "Overflow", kw
        for bh in ((1 << 23) - 8, 1 << 23, (1 << 24) - 8):
            try:
                s = nc.select_kernel(sel(bh, **kw))
            except nc.NcError as err:
                assert err.name == "Overflow" and bh > 1 << 23, (bh, kw)
                continue
            assert s.grid[0] * s.threads <= 0xFFFFFFFF and s.grid[1] <= 65535 and s.grid[2] <= 65535, (bh, kw)


# The reference's selectKernel decisions at every boundary of src/flash.zig:83-95, hand-tabulated.
REFERENCE_DISPATCH = [
    # (d, S, BH, causal) -> reference kernel
    ((16, 256, 8, False), "flash_attention_fwd_v2"),
    ((16, 257, 8, False), "flash_attention_fwd_opt"),
    ((32, 256, 9, True), "flash_attention_fwd_opt"),
    ((32, 255, 8, True), "flash_attention_fwd_v2"),
    ((64, 256, 8, False), "flash_attention_fwd_v2"),
    ((64, 256, 8, True), "flash_attention_fwd_h64"),
    ((64, 257, 8, False), "flash_attention_fwd_h64"),
    ((64, 511, 8, False), "flash_attention_fwd_h64"),
    ((64, 512, 8, False), "flash_attention_fwd_h64_bn32"),
    ((64, 512, 1, True), "flash_attention_fwd_h64_bn32"),
    ((64, 256, 9, False), "flash_attention_fwd_h64"),
    ((64, 1024, 8, True), "flash_attention_fwd_h64_bn32"),
    ((16, 4096, 64, True), "flash_attention_fwd_opt"),
]


@pytest.mark.parametrize("case,want", REFERENCE_DISPATCH)
def test_reference_dispatch_table(case, want):
    d, s, bh, causal = case
    sel = nc.select_kernel(nc.options(batch_heads=bh, seq_len=s, head_dim=d, causal=causal))
    assert sel.reference_name.decode() == want


@pytest.mark.parametrize("d", [16, 32, 64])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("bh,s", [(1, 1), (1, 32), (8, 1024), (32, 4096), (64, 8192), (3, 333)])
def test_dispatch_geometry(d, causal, bh, s):
    sel = nc.select_kernel(nc.options(batch_heads=bh, seq_len=s, head_dim=d, causal=causal))
    name = sel.name.decode()
    assert f"_d{d}_" in name and name.endswith("_causal" if causal else "_full")
    assert sel.threads % 64 == 0 and 64 <= sel.threads <= 1024
    nqb = -(-s // sel.block_m)
    if re.search(r"_q1s8p\dd_", name):  # dense-layout twin: 3-D grid, the same workgroups in linear order
        assert tuple(sel.grid) == ((8, bh // 8, nqb) if bh % 8 == 0 else (bh, 1, nqb))
    else:
        assert sel.grid[0] == nqb * bh and sel.grid[1] == sel.grid[2] == 1
    # 32 or 64 keys per key-split wave per staged block (one or two 32-key sub-tiles)
    assert sel.block_m % 32 == 0 and sel.block_n in (32 * sel.kv_splits, 64 * sel.kv_splits)
    assert sel.threads == 2 * sel.block_m * sel.kv_splits  # (block_m/32) query waves x splits x 64 lanes
    assert 0 < sel.lds_bytes <= 160 * 1024
    assert sel.aligned == 1


def test_dispatch_headline_and_large_configs():
    c3 = nc.select_kernel(CONFIGS["c3"].options())
    assert c3.name == b"nc_flash_fwd_d64_q1s8p2d_causal" and tuple(c3.grid) == (8, 1, 32)
    assert nc.select_kernel(CONFIGS["c4"].options()).name == b"nc_flash_fwd_d64_q8s1p2t2_full"
    assert nc.select_kernel(CONFIGS["c5"].options()).name == b"nc_flash_fwd_d64_q8s1p2t2_causal"


def test_dispatch_alignment_fallbacks():
    # odd slice pad (the reference's smoke strides): element-wise kernel
    sel = nc.select_kernel(nc.options(batch_heads=2, seq_len=32, head_dim=32, q_stride=32 * 32 + 17,
                                      k_stride=32 * 32 + 19, v_stride=32 * 32 + 23, o_stride=32 * 32 + 29,
                                      causal=True))
    assert sel.aligned == 0 and sel.name.decode().endswith("_unaligned")
    # misaligned base pointer
    o = nc.options(batch_heads=2, seq_len=64, head_dim=64)
    assert nc.select_kernel_for(o, 4096 + 2, 4096, 4096, 4096).aligned == 0
    assert nc.select_kernel_for(o, 4096, 4096, 4096, 4096).aligned == 1
    # slices too large for 32-bit buffer offsets: generic 64-bit kernel
    big = nc.options(batch_heads=1, seq_len=1 << 20, head_dim=64, q_row_stride=2048, k_row_stride=2048,
                     v_row_stride=2048, q_stride=(1 << 20) * 2048, k_stride=(1 << 20) * 2048,
                     v_stride=(1 << 20) * 2048)
    sel = nc.select_kernel(big)
    assert sel.aligned == 1 and "_m64_" in sel.name.decode()


def test_pack_args_resolves_row_strides():
    o = nc.options(batch_heads=3, seq_len=100, head_dim=32, q_row_stride=40, q_stride=100 * 40, scale=0.5,
                   causal=True)
    sel = nc.select_kernel(o)
    a = nc.pack_args(o, sel, 0x1000, 0x2000, 0x3000, 0x4000)
    assert (a.q, a.k, a.v, a.o) == (0x1000, 0x2000, 0x3000, 0x4000)
    assert a.seq_len == 100 and a.head_dim == 32 and a.causal == 1 and a.scale == 0.5
    assert a.q_row_stride == 40 and a.k_row_stride == a.v_row_stride == a.o_row_stride == 32
    assert a.num_q_blocks == -(-100 // sel.block_m) and a.batch_heads == 3
    # the first 88 bytes are the reference kernels' parameter list (src/flash.zig:55-68)
    assert nc.KernelArgs.scale.offset == 80 and nc.KernelArgs.causal.offset == 84


def test_pack_args_balance_tail_needs_a_device():
    """The balancing tail comes from the current device's CU count; a causal grid, the private-staging
    kernels and a process without a GPU get 0 (the field only orders waves, never changes results)."""
    from flash_workloads import CONFIGS

    for key in ("c3", "c5"):
        opts = CONFIGS[key].options()
        a = nc.pack_args(opts, nc.select_kernel(opts), 0x1000, 0x2000, 0x3000, 0x4000)
        assert a.balance_tail == 0, key
    if nc.device_count() == 0:
        opts = CONFIGS["c4"].options()
        a = nc.pack_args(opts, nc.select_kernel(opts), 0x1000, 0x2000, 0x3000, 0x4000)
        assert a.balance_tail == 0
    assert nc.KernelArgs.balance_tail.offset == 136 and ctypes.sizeof(nc.KernelArgs) == 144


def test_launch_validates_before_touching_the_module():
    lib = nc.load_library()
    bad = nc.options(batch_heads=1, seq_len=16, head_dim=24)
    st = lib.nc_flash_launch(None, 0x1000, 10 ** 6, 0x1000, 10 ** 6, 0x1000, 10 ** 6, 0x1000, 10 ** 6,
                             ctypes.byref(bad))
    assert nc.STATUS_NAMES[st] == "InvalidValue"
    good = nc.options(batch_heads=2, seq_len=16, head_dim=16)
    # requireLen: one element short on O (src/flash.zig:43); fails before the (null) module is used
    st = lib.nc_flash_launch(ctypes.c_void_p(0x10), 0x1000, 512, 0x1000, 512, 0x1000, 512, 0x1000, 511,
                             ctypes.byref(good))
    assert nc.STATUS_NAMES[st] == "InvalidValue"


class _FakeBuffer:
    """Stands in for a DeviceBuffer: flash_launch only reads .ptr and .nbytes before the C call."""

    def __init__(self, nbytes):
        self.ptr = 0x10000
        self.nbytes = nbytes


@pytest.mark.parametrize("kw", [
    {"q_offset": -1}, {"k_offset": 513}, {"o_offset": 600},          # offsets outside the buffer
    {"v_len": -5}, {"q_len": 513}, {"o_offset": 10, "o_len": 503},   # lengths past what is left
])
def test_python_launch_rejects_bad_offsets_and_lengths(kw):
    """A negative or oversized length would wrap in size_t and defeat requireLen; the binding raises
    ValueError before anything reaches the C ABI (the fake module handle would fail there)."""
    q, k, v = _FakeBuffer(512 * 2), _FakeBuffer(512 * 2), _FakeBuffer(512 * 2)
    o = _FakeBuffer(512 * 4)

    class _Mod:
        handle = None

    with pytest.raises(ValueError):
        nc.flash_launch(_Mod(), q, k, v, o, nc.options(batch_heads=2, seq_len=16, head_dim=16), **kw)


def test_work_model_matches_reference_formulas():
    w = nc.work_model(CONFIGS["c3"].options())
    assert w.flops_reference == 1_074_790_400  # BH*4*S(S+1)/2*d, src/main.zig:1032-1033
    assert w.flops_halfsquare == 1_073_741_824  # 4*BH*S^2*d/2
    assert w.bytes == 5_242_880  # BH*S*d*(3*2+4), src/main.zig:1034
    w4 = nc.work_model(CONFIGS["c4"].options())
    assert w4.flops_reference == w4.flops_halfsquare == 4 * 32 * 4096 * 4096 * 64


def test_benchmark_arithmetic():
    r = nc.benchmark_finish([1.0, 2.0, 3.0], bytes_=6_000_000, flops=4_000_000_000)
    assert (r.mean_ms, r.min_ms, r.max_ms) == (2.0, 1.0, 3.0)
    assert r.has_gbps and abs(r.throughput_gbps - 3.0) < 1e-6      # bytes/(mean_ms*1e6)
    assert r.has_tflops and abs(r.tflops - 2.0) < 1e-6             # flops/(mean_ms*1e9)
    r0 = nc.benchmark_finish([0.5])
    assert not r0.has_gbps and not r0.has_tflops


def test_bench_refuses_multi_gpu():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert p.returncode == 2 and "one GPU" in p.stderr


def test_f16_conversion_matches_numpy():
    lib = nc.load_library()
    h = np.arange(65536, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(f)
    back = np.array([lib.nc_f32_to_f16(float(x)) for x in f[fin][::5]], dtype=np.uint16)
    assert np.array_equal(back, h[fin][::5])
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    special = np.array([65504.0, 65519.99, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26,
                        6.1e-5, 5.96e-8, -0.0, 0.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], dtype=np.float32)
    vals = np.concatenate([vals, special, -special])
    got = np.array([lib.nc_f32_to_f16(float(x)) for x in vals], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert lib.nc_f32_to_f16(float("inf")) == 0x7C00
    assert (lib.nc_f32_to_f16(float("nan")) & 0x7C00) == 0x7C00 and (lib.nc_f32_to_f16(float("nan")) & 0x3FF)
    dec = np.array([lib.nc_f16_to_f32(int(x)) for x in h[fin][::3]], dtype=np.float32)
    assert np.array_equal(dec.view(np.uint32), f[fin][::3].view(np.uint32))


def test_seeded_fills():
    u = nc.fill_uniform(200_000, 1, 0, -1.0, 1.0).view(np.float16).astype(np.float64)
    assert u.min() >= -1.0 and u.max() <= 1.0 and abs(u.mean()) < 0.01 and abs(u.std() - 1 / np.sqrt(3)) < 0.01
    n = nc.fill_normal(200_001, 3, 1, 0.0, 3.0).view(np.float16).astype(np.float64)
    assert abs(n.mean()) < 0.03 and abs(n.std() - 3.0) < 0.03
    # deterministic, keyed by (seed, tensor), counter-based (prefixes agree)
    assert np.array_equal(nc.fill_normal(1000, 3, 1), nc.fill_normal(1000, 3, 1))
    assert np.array_equal(nc.fill_normal(1000, 3, 1), nc.fill_normal(5000, 3, 1)[:1000])
    assert not np.array_equal(nc.fill_normal(1000, 3, 1), nc.fill_normal(1000, 3, 2))
    assert not np.array_equal(nc.fill_uniform(1000, 3, 1), nc.fill_uniform(1000, 4, 1))


def test_code_object_exports_reference_kernel_symbols():
    """The gfx950 code object carries the reference's kernel names (src/main_device.zig:19-47) next to
    its own, so callers that look kernels up by those names keep working."""
    import os
    path = os.path.join(os.path.dirname(__file__), "..", "not-cute-zig_amd", "flash_fwd_gfx950.hsaco")
    blob = open(path, "rb").read()
    for name in ("flash_attention_fwd_v2", "flash_attention_fwd_opt", "flash_attention_fwd_h64",
                 "flash_attention_fwd_h64_bn32", "flash_attention_fwd_h64_causal"):
        assert name.encode() + b"\0" in blob, name
    assert b"\0flash_attention_fwd\0" in blob


# (head_dim, batch_heads, seq_len, causal): the kernel that beat every other pipelined variant in
# interleaved GPU timings of all of them (f16, one MI355X), with its time and the runner-up's ratio.
# Off-grid shapes from the validation sweeps, two per kernel and head size.
MEASURED_WINNERS = [
    ((16, 1, 8687, True), "q1s8p2"),  # 17.2 us, next 1.99x
    ((16, 1, 5753, True), "q1s8p2"),  # 11.9 us, next 1.98x
    ((16, 48, 1536, True), "q2s4p2"),  # 13.8 us, next 1.27x
    ((16, 62, 571, True), "q2s4p2"),  # 6.4 us, next 1.23x
    ((16, 768, 384, True), "q4s1p2t2"),  # 16.1 us, next 1.57x
    ((16, 751, 110, True), "q4s1p2t2"),  # 5.7 us, next 1.46x
    ((32, 1, 6536, True), "q1s8p2"),  # 15.0 us, next 1.99x
    ((32, 1, 4811, False), "q1s8p2"),  # 12.0 us, next 1.94x
    ((32, 29, 1919, True), "q2s4p2"),  # 19.0 us, next 1.25x
    ((32, 48, 768, True), "q2s4p2"),  # 8.1 us, next 1.21x
    ((32, 973, 87, False), "q4s1p3"),  # 6.6 us, next 2.22x
    ((32, 780, 65, False), "q4s1p3"),  # 5.9 us, next 2.09x
    ((64, 1, 5399, False), "q1s8p2"),  # 17.5 us, next 1.78x
    ((64, 4, 2351, True), "q1s8p2"),  # 9.5 us, next 1.63x
    ((64, 6, 2048, True), "q1s8p2"),  # 10.9 us, q2s4 1.27x (one-stage q1s8 ties)
    ((64, 4, 4096, True), "q1s8p2"),  # 19.3 us, q2s4 1.25x (one-stage q1s8 ties)
    ((64, 3, 6000, True), "q1s8p1"),  # 28.4 us, two-stage 1.06x, q2s4 1.23x
    ((64, 2, 12000, True), "q1s8p1"),  # 56.9 us, two-stage 1.09x
    ((64, 48, 384, True), "q2s4p2"),  # 6.3 us, next 1.44x
    ((64, 24, 1536, True), "q2s4p2"),  # 15.8 us, next 1.40x
    ((64, 776, 91, True), "q4s1p2t2"),  # 9.0 us, next 1.68x
    ((64, 926, 80, True), "q4s1p2t2"),  # 9.5 us, next 1.66x
    ((64, 406, 190, False), "q8s1p2t2"),  # 11.8 us, next 1.29x
    ((64, 441, 130, False), "q8s1p2t2"),  # 11.2 us, next 1.12x
]


@pytest.mark.parametrize("case,kernel", MEASURED_WINNERS)
def test_dispatch_picks_measured_winner(case, kernel):
    d, bh, s, causal = case
    for dtype in ("f16", "bf16"):
        name = nc.select_kernel(nc.options(batch_heads=bh, seq_len=s, head_dim=d, causal=causal, dtype=dtype)).name
        assert re.search(rf"_{kernel}d?_", name.decode()), (case, dtype, name)  # d: its dense-layout twin


@pytest.mark.parametrize("d,causal,s_last", [(64, True, 768), (64, False, 512), (32, True, 768), (32, False, 768),
                                             (16, True, 768), (16, False, 768)])
def test_one_stage_private_kernel_boundary(d, causal, s_last):
    """Short sequences on the private-staging route take the one-stage kernel (at most three 32-key
    tiles per wave), longer ones the two-stage kernel; both element types."""
    for dtype in ("f16", "bf16"):
        for s, stages in ((s_last, "p1"), (s_last + 1, "p2")):
            name = nc.select_kernel(nc.options(batch_heads=2, seq_len=s, head_dim=d, causal=causal, dtype=dtype)).name
            assert re.search(rf"_q1s8{stages}d?_", name.decode()), (d, causal, s, dtype, name)


def test_pair_split_dispatch_region():
    """The pair-split kernel replaces the private-staging one for d=64 causal shapes with at least 96
    query blocks whose grid fits one workgroup per CU (measured faster there, slower elsewhere)."""
    from flash_workloads import Workload

    for bh in (1, 2, 3, 4, 8):
        for s in (1024, 2048, 3040, 3041, 3072, 4096, 8192, 8193, 16384):
            for d, causal in ((64, True), (64, False), (32, True)):
                sel = nc.select_kernel(Workload("x", bh, s, d, causal, 0.1, (("normal", 0, 1),) * 3).options())
                nqb = (s + 31) // 32
                q1s8 = "q1s8p2" in sel.name.decode()
                want = d == 64 and causal and nqb >= 96 and nqb * bh <= 256
                assert ("q1s8p2x" in sel.name.decode()) == (want and q1s8), (bh, s, d, causal, sel.name)
                if "q1s8p2x" in sel.name.decode():
                    pairs = bh * (nqb // 2)
                    assert sel.scratch_bytes == 65536 + pairs * 2 * (32 * 64 * 4 + 32 * 8)
                    assert (sel.grid[0], sel.threads, sel.block_m) == (nqb * bh, 512, 32)
                else:
                    assert sel.scratch_bytes == 0


def test_kernel_scratch_bytes_by_name():
    o = CONFIGS["c3"].options()
    assert nc.kernel_scratch_bytes("nc_flash_fwd_d64_q1s8p2x_causal", o) == 65536 + 128 * 2 * 8448
    assert nc.kernel_scratch_bytes("nc_flash_fwd_d64_q1s8p2x_causal_bf16", o) == 65536 + 128 * 2 * 8448
    assert nc.kernel_scratch_bytes("nc_flash_fwd_d64_q1s8p2_causal", o) == 0
    with pytest.raises(nc.NcError) as e:
        nc.kernel_scratch_bytes("flash_attention_fwd_v2", o)
    assert e.value.name == "NotFound"


def test_kernel_scratch_bytes_refuses_more_pairs_than_counters():
    """The counter region holds NC_XS_MAX_PAIRS = 16384 exchange counters: BH=64 S=16384 (64 x 256
    pairs) is the largest BH=64 shape that fits; one more query block per head (S=16448, 64 x 257
    pairs) would put counters inside pair 0's partial slot, so the by-name size query refuses it."""
    from flash_workloads import Workload

    def opts(bh, s):
        return Workload("x", bh, s, 64, True, 0.125, (("normal", 0, 1),) * 3).options()

    fits = nc.kernel_scratch_bytes("nc_flash_fwd_d64_q1s8p2x_causal", opts(64, 16384))
    assert fits == 65536 + 16384 * 2 * 8448
    for name in ("nc_flash_fwd_d64_q1s8p2x_causal", "nc_flash_fwd_d64_q1s8p2x_causal_bf16"):
        with pytest.raises(nc.NcError) as e:
            nc.kernel_scratch_bytes(name, opts(64, 16448))
        assert e.value.name == "InvalidValue"
    # kernels without scratch have no such limit
    assert nc.kernel_scratch_bytes("nc_flash_fwd_d64_q1s8p2_causal", opts(64, 16448)) == 0


# C struct name of each ctypes mirror. A foreign binding (a Zig `@cImport` of the header, ctypes
# here) maps its fields onto exactly these offsets and sizes.
_ABI_STRUCTS = {
    "nc_flash_options": nc.FlashOptions,
    "nc_flash_kernel_selection": nc.KernelSelection,
    "nc_flash_kernel_args": nc.KernelArgs,
    "nc_launch_config": nc.LaunchConfig,
    "nc_function_attributes": nc.FunctionAttributes,
    "nc_device_attributes": nc.DeviceAttributes,
    "nc_flash_work": nc.FlashWork,
    "nc_benchmark_options": nc.BenchmarkOptions,
    "nc_benchmark_result": nc.BenchmarkResult,
}


def test_header_struct_layout_matches_binding(tmp_path):
    """Every struct of include/notcute_flash.h, compiled by gcc, has the field names, offsets and
    sizes (and the total size) of the binding's mirror, so a binding generated from the header
    (Zig's @cImport) and the ctypes one agree on the ABI."""
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "notcute_flash.h"', "int main(void) {"]
    for cname, py in _ABI_STRUCTS.items():
        lines.append(f'printf("{cname} - %zu %zu\\n", sizeof({cname}), _Alignof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname} {fname} %zu %zu\\n", offsetof({cname}, {fname}), '
                         f'sizeof((({cname} *)0)->{fname}));')
    lines.append('printf("macro NC_ELEMENT_F16 %u 0\\n", NC_ELEMENT_F16);')
    lines.append('printf("macro NC_ELEMENT_BF16 %u 0\\n", NC_ELEMENT_BF16);')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    seen = {}
    for line in filter(None, out):
        cname, fname, a, b = line.split()
        seen[(cname, fname)] = (int(a), int(b))
    assert seen[("macro", "NC_ELEMENT_F16")][0] == nc.ELEMENT_TYPES["f16"]
    assert seen[("macro", "NC_ELEMENT_BF16")][0] == nc.ELEMENT_TYPES["bf16"]
    for cname, py in _ABI_STRUCTS.items():
        assert seen[(cname, "-")] == (ctypes.sizeof(py), ctypes.alignment(py)), cname
        for fname, ftype in py._fields_:
            assert seen[(cname, fname)] == (getattr(py, fname).offset, ctypes.sizeof(ftype)), (cname, fname)


def test_options_fields_a_binding_sets():
    """What a binding's toC (a Zig conversion of flash.Options: nc_flash_options_init, then every
    field, causal as @intFromBool) relies on: element_type defaults to f16, causal 1 selects the causal
    kernel and 0 the non-causal one, bf16 selects the _bf16 twin."""
    o = nc.FlashOptions()
    nc.load_library().nc_flash_options_init(ctypes.byref(o))
    assert o.element_type == nc.ELEMENT_TYPES["f16"]
    base = CONFIGS["c3"].options()
    for flag, want in ((1, True), (0, False)):
        base.causal = flag
        name = nc.select_kernel(base).name.decode()
        assert name.endswith("_causal") == want, (flag, name)
    base.element_type = nc.ELEMENT_TYPES["bf16"]
    assert nc.select_kernel(base).name.decode().endswith("_bf16")


def test_noalloc_buffer_holds_every_dispatched_pair_split():
    """nc_flash_launch_noalloc serves pair-split kernels from a static buffer of
    NC_NOALLOC_SCRATCH_BYTES (4 MiB): every shape the dispatcher routes to them (d=64 causal, at least
    96 query blocks, at most 256 workgroups) needs at most 64 KB + 128 pairs x 2 slots, so none is
    refused."""
    from flash_workloads import Workload

    with open(os.path.join(ROOT, "include", "notcute_flash.h")) as f:
        m = re.search(r"#define NC_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", f.read())
    cap = int(m.group(1)) << int(m.group(2))
    worst = 0
    for bh in range(1, 9):
        for s in range(32 * 90, 32 * 260, 32 * 3):
            sel = nc.select_kernel(Workload("x", bh, s, 64, True, 0.1, (("normal", 0, 1),) * 3).options())
            worst = max(worst, sel.scratch_bytes)
    assert 0 < worst <= cap, (worst, cap)


def test_dense_twin_only_for_packed_slices():
    """The private-staging kernels' dense-layout twins (q1s8p1d, q1s8p2d) take over exactly when every
    tensor is a stack of packed slices (slice stride S*d, row stride d); any pad keeps the kernel that
    reads the strides. Their 3-D grid holds the same workgroups: (8, BH/8, nqb) or (BH, 1, nqb)."""
    def sel(**kw):
        return nc.select_kernel(nc.options(**kw))

    base = dict(batch_heads=8, seq_len=1024, head_dim=64, causal=True)
    s = sel(**base)
    assert s.name == b"nc_flash_fwd_d64_q1s8p2d_causal" and tuple(s.grid) == (8, 1, 32)
    s = sel(**dict(base, batch_heads=3))
    assert s.name == b"nc_flash_fwd_d64_q1s8p2d_causal" and tuple(s.grid) == (3, 1, 32)
    s = sel(batch_heads=1, seq_len=32, head_dim=16)  # c1
    assert s.name == b"nc_flash_fwd_d16_q1s8p1d_full" and tuple(s.grid) == (1, 1, 1)
    # a padded slice of any one tensor, or padded rows, keep the strided kernel and a 1-D grid
    for pad in (dict(q_stride=1024 * 64 + 8), dict(k_stride=1024 * 64 + 8), dict(v_stride=1024 * 64 + 8),
                dict(o_stride=1024 * 64 + 4), dict(q_row_stride=72, q_stride=1024 * 72),
                dict(o_row_stride=68, o_stride=1024 * 68)):
        s = sel(**dict(base, **pad))
        assert s.name == b"nc_flash_fwd_d64_q1s8p2_causal" and tuple(s.grid) == (256, 1, 1), pad
    # c2's padded rows (pitch 40): the strided kernel
    assert not re.search(r"q1s8p\dd_", nc.select_kernel(CONFIGS["c2_causal"].options()).name.decode())
    # shared-staging selections have no dense twin
    assert nc.select_kernel(CONFIGS["c4"].options()).name == b"nc_flash_fwd_d64_q8s1p2t2_full"


def test_kernel_params_forms():
    """nc_flash_kernel_params: the argument block as one parameter for most kernels, one parameter per
    field (aliasing the block) for the dense-layout kernels; unknown names are refused."""
    o = CONFIGS["c3"].options()
    sel = nc.select_kernel(o)
    a = nc.pack_args(o, sel, 0x1000, 0x2000, 0x3000, 0x4000)
    p = nc.kernel_params(sel.name.decode(), a)
    assert len(p) == nc.MAX_KERNEL_PARAMS == len(nc.KernelArgs._fields_)
    assert [ctypes.addressof(x) for x in p] == [ctypes.addressof(a) + getattr(nc.KernelArgs, f).offset
                                                 for f, _ in nc.KernelArgs._fields_]
    assert p[0].value == 0x1000 and p[4].value == 1024 and p[6].value == 1024 * 64
    for name in ("nc_flash_fwd_d64_q1s8p2_causal", "nc_flash_fwd_d64_q8s1p2t2_full", "nc_flash_fwd_d64_m64_causal"):
        assert nc.kernel_params(name, a) == [a]
    with pytest.raises(nc.NcError) as e:
        nc.kernel_params("flash_attention_fwd_v2", a)
    assert e.value.name == "NotFound"
