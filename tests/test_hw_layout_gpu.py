"""The gfx950 instruction semantics the flash kernels are built on, pinned on the GPU with one-wave
probes (not-cute-zig_amd/csrc/hw_probe.hip): the MFMA operand/accumulator lane layout, the lane
mapping of ds_read_b64_tr_b16 and the lane-pair exchange of v_permlane32_swap. These pin the
hardware, not the reference; a failure here names the broken assumption directly."""

import os

import numpy as np
import pytest

import notcute_flash as nc

pytestmark = pytest.mark.gpu

PROBE = os.path.join(os.path.dirname(__file__), "..", "not-cute-zig_amd", "hw_probe_gfx950.hsaco")


@pytest.fixture(scope="module")
def probe(gpu):
    if not os.path.exists(PROBE):
        pytest.fail(f"{PROBE} is missing: run __graft_entry__.build()")
    return nc.Module.load_file(PROBE)


def _launch(probe, name, *args):
    probe.get_function(name).launch((1,), (64,), list(args))
    nc.synchronize()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_mfma_32x32x16_lane_layout(probe, dtype):
    """Lane l supplies A[l%32][8(l/32)+j] and B[8(l/32)+j][l%32]; accumulator register r of lane l
    holds D[8(r/4) + 4(l/32) + r%4][l%32] (the layout the kernels' softmax reads scores in)."""
    import ctypes

    rng = np.random.default_rng(5)
    a = rng.integers(-8, 9, size=(32, 16)).astype(np.float32)
    b = rng.integers(-8, 9, size=(16, 32)).astype(np.float32)
    if dtype == "f16":
        a16, b16 = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    else:  # small integers are exact in bf16: the upper half of the f32 pattern
        a16 = (a.view(np.uint32) >> 16).astype(np.uint16)
        b16 = (b.view(np.uint32) >> 16).astype(np.uint16)
    da, db = nc.DeviceBuffer.from_array(a16.ravel()), nc.DeviceBuffer.from_array(b16.ravel())
    dd = nc.DeviceBuffer(64 * 16 * 4)
    try:
        _launch(probe, "nc_probe_mfma32x32x16", ctypes.c_void_p(da.ptr), ctypes.c_void_p(db.ptr),
                ctypes.c_void_p(dd.ptr), ctypes.c_int(1 if dtype == "bf16" else 0))
        got = dd.download(np.float32, 64 * 16).reshape(64, 16)
    finally:
        for buf in (da, db, dd):
            buf.free()
    want = a @ b
    lanes, regs = np.meshgrid(np.arange(64), np.arange(16), indexing="ij")
    rows = 8 * (regs // 4) + 4 * (lanes // 32) + regs % 4
    cols = lanes % 32
    assert np.array_equal(got, want[rows, cols])


def test_ds_read_b64_tr_b16_lane_mapping(probe):
    """Inside a 16-lane group, lane m supplies the address of V[r0 + m/4][d0 + 4(m%4)] and lane i
    receives V[r0 .. r0+3][d0 + i] (V row-major, 16-bit elements)."""
    import ctypes

    out = nc.DeviceBuffer(64 * 4 * 2)
    try:
        _launch(probe, "nc_probe_ds_read_tr", ctypes.c_void_p(out.ptr))
        got = out.download(np.uint16, 64 * 4).reshape(64, 4).astype(np.int64)
    finally:
        out.free()
    lanes = np.arange(64)
    g, i = lanes // 16, lanes % 16
    r0, d0 = 4 * g, 8 * g
    want = np.stack([(r0 + j) * 64 + d0 + i for j in range(4)], axis=1)
    assert np.array_equal(got, want)


def test_permlane32_swap_pairs_lanes(probe):
    """Each lane gets its own value and that of lane l^32 (in either order): the pair the kernels'
    row max and row sum combine."""
    import ctypes

    out = nc.DeviceBuffer(64 * 2 * 4)
    try:
        _launch(probe, "nc_probe_permlane32", ctypes.c_void_p(out.ptr))
        got = out.download(np.uint32, 128).reshape(64, 2)
    finally:
        out.free()
    for lane in range(64):
        assert sorted(got[lane].tolist()) == sorted([1000 + lane, 1000 + (lane ^ 32)]), lane
