"""Named flash-attention workloads: the MI355X benchmark configurations and the reference's own
smoke and compare cases, with deterministic host-side inputs (f16 bit patterns).

Inputs come from the library's host fills (``nc_fill_*``): SplitMix64 keyed by (seed, tensor id
Q=0 / K=1 / V=2) for the seeded configurations, and fillFlashInput (src/main.zig:1207-1211) for the
reference's cases, whose fills are (mul, add, scale) = (3, 1, 0.125), (5, 2, 0.0625),
(7, 3, 0.03125) for Q, K, V (src/main.zig:219-221, 991-993).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Tuple

import numpy as np

import notcute_flash as nc

Dist = Tuple  # ("normal", mean, sigma) | ("uniform", lo, hi) | ("pattern", mul, add, scale)

REFERENCE_FILLS = (("pattern", 3, 1, 0.125), ("pattern", 5, 2, 0.0625), ("pattern", 7, 3, 0.03125))


@dataclass
class Workload:
    name: str
    batch_heads: int
    seq_len: int
    head_dim: int
    causal: bool
    scale: float
    dists: Tuple[Dist, Dist, Dist]
    seed: int = 0
    q_stride: int = 0  # 0: dense (S-1)*row + d rounded to S*row
    k_stride: int = 0
    v_stride: int = 0
    o_stride: int = 0
    q_row: int = 0  # 0: head_dim
    k_row: int = 0
    v_row: int = 0
    o_row: int = 0
    note: str = ""
    tags: List[str] = field(default_factory=list)
    dtype: str = "f16"  # element type of Q/K/V: "f16" (the reference's) or "bf16"

    def row(self, which: str) -> int:
        r = getattr(self, f"{which}_row")
        return r if r else self.head_dim

    def stride(self, which: str) -> int:
        s = getattr(self, f"{which}_stride")
        return s if s else self.seq_len * self.row(which)

    def length(self, which: str) -> int:
        return self.batch_heads * self.stride(which)

    def options(self) -> nc.FlashOptions:
        return nc.options(batch_heads=self.batch_heads, seq_len=self.seq_len, head_dim=self.head_dim,
                          q_stride=self.stride("q"), k_stride=self.stride("k"), v_stride=self.stride("v"),
                          o_stride=self.stride("o"), scale=self.scale, causal=self.causal,
                          q_row_stride=self.q_row, k_row_stride=self.k_row, v_row_stride=self.v_row,
                          o_row_stride=self.o_row, dtype=self.dtype)

    def make_inputs(self) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
        """Q, K, V as 16-bit patterns of the workload's element type (the same seeded draws for
        f16 and bf16, each rounded to nearest even)."""
        bf = self.dtype == "bf16"
        out = []
        for tid, which in enumerate("qkv"):
            n = self.length(which)
            d = self.dists[tid]
            if d[0] == "normal":
                out.append((nc.fill_normal_bf16 if bf else nc.fill_normal)(n, self.seed, tid, d[1], d[2]))
            elif d[0] == "uniform":
                out.append((nc.fill_uniform_bf16 if bf else nc.fill_uniform)(n, self.seed, tid, d[1], d[2]))
            elif d[0] == "pattern":
                h = nc.fill_flash_input(n, d[1], d[2], d[3])
                out.append(_f16_to_bf16_exact(h) if bf else h)
            else:
                raise ValueError(d)
        return tuple(out)

    def work(self) -> Dict[str, int]:
        w = nc.work_model(self.options())
        return {"flops_reference": w.flops_reference, "flops": w.flops_halfsquare, "bytes": w.bytes}

    def describe(self) -> str:
        return (f"{self.name}: BH={self.batch_heads} S={self.seq_len} d={self.head_dim} "
                f"causal={self.causal} scale={self.scale:g}")


def _f16_to_bf16_exact(h: np.ndarray) -> np.ndarray:
    """f16 patterns whose values bf16 holds exactly (the reference's small dyadic fills)."""
    bits = h.view(np.float16).astype(np.float32).view(np.uint32)
    if np.any(bits & 0xFFFF):
        raise ValueError("value not representable in bf16")
    return (bits >> 16).astype(np.uint16)


def _normal(s=1.0):
    return ("normal", 0.0, s)


# The five configurations of the MI355X benchmark plan (c1 is the CPU-runnable parity case,
# c3 is the headline: BH=8 S=1024 d=64 causal).
CONFIGS: Dict[str, Workload] = {
    "c1": Workload("c1", 1, 32, 16, False, 0.25, (("uniform", -1.0, 1.0),) * 3, seed=1),
    # Row pitch head_dim+8 = 40 elements, slice stride 128*40 = 5120.
    "c2_causal": Workload("c2_causal", 8, 128, 32, True, 1.0 / math.sqrt(32), (_normal(),) * 3, seed=2,
                          q_row=40, k_row=40, v_row=40, o_row=40),
    "c2_full": Workload("c2_full", 8, 128, 32, False, 1.0 / math.sqrt(32), (_normal(),) * 3, seed=2,
                        q_row=40, k_row=40, v_row=40, o_row=40),
    # The slice-padded reading of config 2 (padding between slices, rows dense), as the reference's
    # own smoke tests pad.
    "c2_slicepad": Workload("c2_slicepad", 8, 128, 32, True, 1.0 / math.sqrt(32), (_normal(),) * 3, seed=2,
                            q_stride=128 * 32 + 8, k_stride=128 * 32 + 8, v_stride=128 * 32 + 8,
                            o_stride=128 * 32 + 8),
    "c3": Workload("c3", 8, 1024, 64, True, 0.125, (_normal(),) * 3, seed=3),
    "c4": Workload("c4", 32, 4096, 64, False, 0.125, (_normal(),) * 3, seed=4),
    "c5": Workload("c5", 64, 8192, 64, True, 0.125, (_normal(3.0), _normal(3.0), ("uniform", -1.0, 1.0)), seed=5),
}

HEADLINE = "c3"


def reference_smoke_cases() -> List[Workload]:
    """runFlashAttention's four cases (src/main.zig:190-193): odd slice pads, S not a multiple of
    16, tolerance 0.008 on the active region (src/main.zig:273-284)."""
    rows = [
        (2, 32, 32, 32 * 32 + 17, 32 * 32 + 19, 32 * 32 + 23, 32 * 32 + 29, True),
        (1, 17, 16, 17 * 16 + 3, 17 * 16 + 5, 17 * 16 + 7, 17 * 16 + 11, False),
        (3, 49, 16, 49 * 16, 49 * 16 + 13, 49 * 16 + 17, 49 * 16 + 19, True),
        (1, 33, 64, 33 * 64 + 3, 33 * 64 + 5, 33 * 64 + 7, 33 * 64 + 11, False),
    ]
    out = []
    for i, (bh, s, d, qs, ks, vs, os_, causal) in enumerate(rows):
        out.append(Workload(f"smoke{i}_bh{bh}_s{s}_d{d}_{'c' if causal else 'n'}", bh, s, d, causal,
                            1.0 / math.sqrt(d), REFERENCE_FILLS, q_stride=qs, k_stride=ks, v_stride=vs,
                            o_stride=os_))
    return out


# runCompareDemo's flash shapes (src/main.zig:141-170): contiguous strides, max-abs <= 0.02
# over the whole output (src/main.zig:1038-1042).
REFERENCE_COMPARE_SHAPES = [
    (2, 32, 16, False), (2, 32, 32, True), (2, 64, 16, False), (2, 64, 32, True), (2, 128, 32, True),
    (8, 128, 16, False), (8, 128, 32, True), (8, 256, 16, False), (8, 256, 32, True), (16, 256, 32, False),
    (16, 512, 32, True), (8, 256, 64, False), (8, 512, 64, True), (16, 512, 64, False), (8, 1024, 64, True),
]


def reference_compare_cases() -> List[Workload]:
    return [Workload(f"compare_bh{bh}_s{s}_d{d}_{'c' if c else 'n'}", bh, s, d, c, 1.0 / math.sqrt(d),
                     REFERENCE_FILLS) for (bh, s, d, c) in REFERENCE_COMPARE_SHAPES]


def sample_rows(seq_len: int, extra: int = 64, seed: int = 0) -> np.ndarray:
    """Deterministic query-row subset for parity on configurations whose full CPU oracle is too slow:
    tile edges 0,1,15,16,17,31,32,63,64,127,128,... up to S-1, plus `extra` seeded rows."""
    rows = {0, 1, seq_len - 1, seq_len - 2}
    p = 16
    while p < seq_len:
        rows.update({p - 1, p, p + 1})
        p *= 2
    rng = np.random.default_rng(seed)
    rows.update(int(x) for x in rng.integers(0, seq_len, size=extra))
    return np.array(sorted(r for r in rows if 0 <= r < seq_len), dtype=np.int64)
