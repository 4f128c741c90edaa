"""Host-side pins of the bf16 extension (no GPU): the f32 -> bf16 rounding and its inverse, the
bf16 seeded fills, the oracle's bf16 input path against an independent float64 softmax, and the
validation and dispatch of element_type."""

import ctypes
import math

import numpy as np
import pytest

import flash_harness as fh
import flash_oracle
import flashcheck as fc
import notcute_flash as nc
from flash_workloads import CONFIGS, Workload


def _bf16_value(h: int) -> float:
    return float(np.array([h << 16], dtype=np.uint32).view(np.float32)[0])


def test_bf16_widening_is_exact_for_every_pattern():
    h = np.arange(0, 65536, 3, dtype=np.uint32)
    want = (h << 16).view(np.float32)
    for conv in (nc.bf16_to_f32, flash_oracle.bf16_to_float):
        got = np.array([conv(int(x)) for x in h], dtype=np.float32)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_bf16_rounds_to_nearest_even():
    """Each result is the bf16 value nearest to x (float64 distances); exact ties go to the even
    pattern; every finite bf16 value maps to itself."""
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-30, 30, 3000),
                         (np.arange(1, 200) * 2 ** -7 + 1.0)]).astype(np.float32)  # exact ties among these
    for x in xs:
        h = nc.f32_to_bf16(float(x))
        got = _bf16_value(h)
        lo_bits = int(np.array([x], np.float32).view(np.uint32)[0]) >> 16
        cands = [_bf16_value(lo_bits), _bf16_value(lo_bits + 1)]
        dist = [abs(c - float(x)) for c in cands]
        if dist[0] == dist[1]:
            assert h % 2 == 0 and got in cands, x
        else:
            assert got == cands[int(np.argmin(dist))], x
    for h in range(0, 0x7f80, 97):
        assert nc.f32_to_bf16(_bf16_value(h)) == h
        assert nc.f32_to_bf16(-_bf16_value(h)) == h | 0x8000
    assert nc.f32_to_bf16(float("inf")) == 0x7f80
    assert nc.f32_to_bf16(3.4e38) == 0x7f80  # rounds past the largest finite bf16
    assert math.isnan(_bf16_value(nc.f32_to_bf16(float("nan"))))


def test_bf16_fills_round_the_same_draws():
    """bf16 and f16 fills of one (seed, tensor) come from the same f32 value: they differ by at most
    half a bf16 ulp plus half an f16 ulp of it."""
    for fill16, fillbf, args in ((nc.fill_normal, nc.fill_normal_bf16, (0.0, 3.0)),
                                 (nc.fill_uniform, nc.fill_uniform_bf16, (-1.0, 1.0))):
        a = fill16(4096, 7, 2, *args).view(np.float16).astype(np.float64)
        b = fh.decode(fillbf(4096, 7, 2, *args), "bf16")
        bound = np.abs(b) * 2.0 ** -8 + np.abs(a) * 2.0 ** -11 + 2.0 ** -25
        assert np.all(np.abs(a - b) <= bound)
        assert np.count_nonzero(a != b) > 100  # bf16 is genuinely coarser


def _bf16_workload(name, bh, s, d, causal, scale, dists, seed, **kw):
    return Workload(name, bh, s, d, causal, scale, dists, seed=seed, dtype="bf16", **kw)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [16, 64])
def test_oracle_bf16_matches_float64(causal, d):
    wl = _bf16_workload(f"bf16_f64_{d}", 2, 45, d, causal, 1.0 / math.sqrt(d), (("normal", 0.0, 1.0),) * 3, 4,
                        q_row=d + 8, o_row=d + 4, q_stride=45 * (d + 8) + 3, o_stride=45 * (d + 4) + 1)
    q, k, v = wl.make_inputs()
    o = fc.oracle(wl, q, k, v)
    ref = fh.attention_f64(wl, q, k, v)
    idx = fc.active_index(wl)
    assert np.max(np.abs(o[idx] - ref[idx])) <= 1e-5
    # the same bits read as f16 give a different answer: the element type really is honoured
    o16 = fc.oracle(Workload(**{**wl.__dict__, "dtype": "f16"}), q, k, v)
    assert np.max(np.abs(o16[idx] - o[idx])) > 1e-2


def test_oracle_bf16_closed_forms():
    wl = _bf16_workload("bf16_const", 1, 33, 32, True, 0.5, (("normal", 0.0, 2.0),) * 3, 9)
    q, k, _ = wl.make_inputs()
    v = np.full_like(q, nc.f32_to_bf16(0.375))
    o = fc.oracle(wl, q, k, v)
    assert np.max(np.abs(o[fc.active_index(wl)] - 0.375)) <= 1e-6  # constant V -> constant O
    o0 = fc.oracle(wl, q, k, q.copy(), rows=[0])  # causal row 0 sees key 0 only: O[0] = V[0]
    assert np.array_equal(o0[:32], fh.decode(q[:32], "bf16").astype(np.float32))


def test_reference_pattern_fill_is_exact_in_bf16():
    wl = Workload("pat", 1, 64, 16, False, 0.25, (("pattern", 3, 1, 0.125), ("pattern", 5, 2, 0.0625),
                                                   ("pattern", 7, 3, 0.03125)), dtype="bf16")
    q16 = nc.fill_flash_input(wl.length("q"), 3, 1, 0.125)
    qb = wl.make_inputs()[0]
    assert np.array_equal(fh.decode(qb, "bf16"), q16.view(np.float16).astype(np.float64))


def test_element_type_validation_and_dispatch():
    bad = nc.options(seq_len=64, head_dim=64)
    bad.element_type = 2
    with pytest.raises(nc.NcError) as ei:
        nc.validate(bad)
    assert ei.value.name == "InvalidValue"
    for wl in (CONFIGS["c1"], CONFIGS["c3"], CONFIGS["c4"], CONFIGS["c5"], CONFIGS["c2_slicepad"]):
        o16 = wl.options()
        obf = Workload(**{**wl.__dict__, "dtype": "bf16"}).options()
        s16, sbf = nc.select_kernel(o16), nc.select_kernel(obf)
        assert sbf.name.decode() == s16.name.decode() + "_bf16"
        assert (tuple(sbf.grid), sbf.threads, sbf.lds_bytes) == (tuple(s16.grid), s16.threads, s16.lds_bytes)
    # misaligned bases pick the element-wise bf16 twin
    o = Workload(**{**CONFIGS["c3"].__dict__, "dtype": "bf16"}).options()
    sel = nc.select_kernel_for(o, 0x1002, 0x2000, 0x3000, 0x4000)
    assert sel.name.decode().endswith("_unaligned_bf16")


def test_options_default_element_type_is_f16():
    o = nc.FlashOptions()
    nc.lib().nc_flash_options_init(ctypes.byref(o))
    assert o.element_type == 0
