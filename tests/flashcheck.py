"""Shared helpers for the parity tests: oracle runs, GPU runs through the C ABI, and the error
metrics of the parity bar.

Parity bar (per active output element, o = GPU, r = oracle):
  max-abs = max |o - r|                      <= 2e-3
  max-rel = max |o - r| / max(|r|, 0.2)      <= 1e-2
The reference's own tolerances are checked on its own cases: 0.008 on the active region of the
smoke cases (src/main.zig:273-284) and 0.02 max-abs over the whole output of the compare cases
(src/main.zig:1038-1042).
"""

from __future__ import annotations

import os
from typing import Optional, Sequence, Tuple

import numpy as np

import flash_oracle
import notcute_flash as nc
from flash_workloads import Workload

MAX_ABS = 2e-3
MAX_REL = 1e-2
REL_FLOOR = 0.2
# bf16 extension: weights rounded to bf16 (8 significant bits) for the PV product.
BF16_MAX_ABS = 8e-3
BF16_MAX_REL = 4e-2


def parity_bar(dtype: str = "f16") -> Tuple[float, float]:
    """(max-abs, max-rel) bar of the element type."""
    return (BF16_MAX_ABS, BF16_MAX_REL) if dtype == "bf16" else (MAX_ABS, MAX_REL)
SENTINEL = np.float32(-7777.0)


def host_threads() -> int:
    """Oracle threads: the GPU box gives a 16-core share; stay within it and within this host."""
    return max(1, min(16, os.cpu_count() or 1))


def active_index(wl: Workload, rows: Optional[Sequence[int]] = None) -> np.ndarray:
    """Flat O indices of the active rows x head_dim region of every slice."""
    r = np.arange(wl.seq_len, dtype=np.int64) if rows is None else np.asarray(rows, dtype=np.int64)
    b = np.arange(wl.batch_heads, dtype=np.int64)
    c = np.arange(wl.head_dim, dtype=np.int64)
    idx = (b[:, None, None] * wl.stride("o") + r[None, :, None] * wl.row("o") + c[None, None, :])
    return idx.reshape(-1)


def oracle(wl: Workload, q, k, v, rows=None, o_init: Optional[np.ndarray] = None,
           threads: Optional[int] = None) -> np.ndarray:
    o = np.full(wl.length("o"), SENTINEL, dtype=np.float32) if o_init is None else o_init.copy()
    flash_oracle.flash_fwd(q, k, v, o, batch_heads=wl.batch_heads, seq_len=wl.seq_len, head_dim=wl.head_dim,
                           q_stride=wl.stride("q"), k_stride=wl.stride("k"), v_stride=wl.stride("v"),
                           o_stride=wl.stride("o"), scale=wl.scale, causal=wl.causal, q_row=wl.row("q"),
                           k_row=wl.row("k"), v_row=wl.row("v"), o_row=wl.row("o"),
                           threads=host_threads() if threads is None else threads, rows=rows, dtype=wl.dtype)
    return o


def run_gpu(mod: nc.Module, wl: Workload, q, k, v, o_init: np.ndarray, offset: int = 0) -> np.ndarray:
    """Upload, launch through nc_flash_launch, download. `offset` shifts every base pointer by that
    many elements (misaligned-base cases)."""
    bufs = []
    try:
        dq = nc.DeviceBuffer((q.size + offset) * 2)
        dk = nc.DeviceBuffer((k.size + offset) * 2)
        dv = nc.DeviceBuffer((v.size + offset) * 2)
        do = nc.DeviceBuffer((o_init.size + offset) * 4)
        bufs = [dq, dk, dv, do]
        dq.upload(q, 2 * offset)
        dk.upload(k, 2 * offset)
        dv.upload(v, 2 * offset)
        do.upload(o_init, 4 * offset)
        nc.flash_launch(mod, dq, dk, dv, do, wl.options(), q_offset=offset, k_offset=offset, v_offset=offset,
                        o_offset=offset)
        nc.synchronize()
        return do.download(np.float32, o_init.size, 4 * offset)
    finally:
        for b in bufs:
            b.free()


def errors(o: np.ndarray, r: np.ndarray, idx: np.ndarray) -> Tuple[float, float]:
    d = np.abs(o[idx].astype(np.float64) - r[idx].astype(np.float64))
    if d.size == 0:
        return 0.0, 0.0
    rel = d / np.maximum(np.abs(r[idx].astype(np.float64)), REL_FLOOR)
    return float(np.nanmax(d)) if not np.isnan(d).any() else float("nan"), float(np.max(rel))


def assert_parity(o: np.ndarray, r: np.ndarray, idx: np.ndarray, what: str, max_abs: float = MAX_ABS,
                  max_rel: float = MAX_REL) -> Tuple[float, float]:
    assert np.all(np.isfinite(o[idx])), f"{what}: non-finite output"
    ea, er = errors(o, r, idx)
    assert ea <= max_abs and er <= max_rel, f"{what}: max-abs {ea:.3e} (<= {max_abs}), max-rel {er:.3e} (<= {max_rel})"
    return ea, er


def assert_pads_untouched(o: np.ndarray, o_init: np.ndarray, wl: Workload, what: str) -> None:
    mask = np.ones(o.size, dtype=bool)
    mask[active_index(wl)] = False
    assert np.array_equal(o[mask].view(np.uint32), o_init[mask].view(np.uint32)), f"{what}: padding was written"
