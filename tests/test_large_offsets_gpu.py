"""64-bit addressing at large sizes, through nc_flash_launch.

The pipelined kernels address a slice with 64-bit base pointers (head * stride) and 32-bit offsets
inside it; the generic kernels use 64-bit offsets throughout and take every layout whose rows lie
too far apart for 32-bit offsets. Two layouts put the data where a truncated 32-bit product would
land elsewhere:
  * slices 4 GiB + 128 bytes apart (slice strides of 2^31 + 64 f16 elements, 2^30 + 32 f32 for O),
    contiguous rows: the pipelined route, with the second slice past 2^32 bytes;
  * rows 4 MiB apart (row pitch 2^21 elements): the selection falls back to the 64-bit generic
    kernel, whose row offsets pass 2^31 bytes inside one slice.
Only the active rows are uploaded; the output is checked against the oracle on the same data laid
out densely, and the O bytes around every slice keep their fill.
"""

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import Workload

pytestmark = pytest.mark.gpu

FILL = 0xFFFFFFFF  # nc_memset(0xff) pattern of an untouched f32


def _place(buf, rows2d, base, row_stride, esize):
    """Write rows2d[r] at element base + r*row_stride of buf."""
    if row_stride == rows2d.shape[1]:
        buf.upload(np.ascontiguousarray(rows2d), base * esize)
        return
    for r in range(rows2d.shape[0]):
        buf.upload(np.ascontiguousarray(rows2d[r]), (base + r * row_stride) * esize)


def _run(gpu, wl, slice_stride, o_slice_stride, row):
    bh, s, d = wl.batch_heads, wl.seq_len, wl.head_dim
    q, k, v = wl.make_inputs()  # dense layout, the oracle's
    ref = fc.oracle(wl, q, k, v)
    opts = nc.options(batch_heads=bh, seq_len=s, head_dim=d, q_stride=slice_stride, k_stride=slice_stride,
                      v_stride=slice_stride, o_stride=o_slice_stride, scale=wl.scale, causal=wl.causal,
                      q_row_stride=row, k_row_stride=row, v_row_stride=row)
    sel = nc.select_kernel(opts)
    print(f"[case] {wl.describe()} slice stride {slice_stride} row {row} o stride {o_slice_stride} -> "
          f"{sel.name.decode()}", flush=True)
    bufs = []
    try:
        for _ in range(3):
            bufs.append(nc.DeviceBuffer(bh * slice_stride * 2))
        bo = nc.DeviceBuffer(bh * o_slice_stride * 4)
        bufs.append(bo)
        bo.memset(0xFF)
        for buf, x in zip(bufs[:3], (q, k, v)):
            for b in range(bh):
                _place(buf, x[b * s * d:(b + 1) * s * d].reshape(s, d), b * slice_stride, row, 2)
        nc.flash_launch(gpu, *bufs, opts)
        nc.synchronize()
        out = np.concatenate([bo.download(np.float32, s * d, b * o_slice_stride * 4) for b in range(bh)])
        # the padding after each slice's last row, up to 64 floats from either end
        pad = min(64, o_slice_stride - s * d)
        assert pad > 0, "the layouts leave padding between O slices"
        edges = []
        for b in range(bh):
            edges.append(bo.download(np.uint32, pad, (b * o_slice_stride + s * d) * 4))
            edges.append(bo.download(np.uint32, pad, ((b + 1) * o_slice_stride - pad) * 4))
        ea, er = fc.assert_parity(out, ref, fc.active_index(wl), wl.name)
        for e in edges:
            assert np.all(e == FILL), f"{wl.name}: O written outside its rows"
        print(f"[ok] {wl.name} -> {sel.name.decode()}: max-abs {ea:.2e} max-rel {er:.2e}", flush=True)
        return sel.name.decode()
    finally:
        for b in bufs:
            b.free()


@pytest.mark.parametrize("d,causal", [(64, True), (32, False)])
def test_slices_past_4gib(gpu, d, causal):
    wl = Workload(f"far_slices_d{d}", 2, 300, d, causal, 1.0 / np.sqrt(d), (("normal", 0.0, 1.0),) * 3, seed=91)
    name = _run(gpu, wl, (1 << 31) + 64, (1 << 30) + 32, d)
    assert "_m64_" not in name, "contiguous rows stay on the pipelined route"


def test_rows_past_2gib(gpu):
    wl = Workload("far_rows_d64", 2, 200, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=92)
    row = 1 << 21
    name = _run(gpu, wl, 200 * row, 200 * 64 + 36, row)
    assert "_m64_" in name, "4 MiB rows need the 64-bit generic kernel"
