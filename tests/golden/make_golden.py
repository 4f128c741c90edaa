#!/usr/bin/env python3
"""Writes tests/golden/flash_golden.npz: small attention cases with float64 expected outputs.

The expected values come from a textbook float64 computation, softmax(scale * Q K^T, causal mask) V
evaluated with numpy matrix products on the f16 inputs, independent of the C oracle's f32 loop
order. Inputs are drawn with numpy's own generator (not the library's SplitMix64 fills) and
rounded to f16, except case `ref_smoke2`, which uses the reference's fillFlashInput pattern and
strides of its third smoke case (src/main.zig:192, 1207-1211).

Each case stores: q/k/v (uint16 f16 bit patterns, full strided buffers), o_expected (float64, full
O buffer, NaN in padding), and its parameters. Regenerate with:  python tests/golden/make_golden.py
"""

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "flash_golden.npz")


def f64_attention(q, k, v, bh, s, d, strides, rows, scale, causal, o_len):
    qs, ks, vs, os_ = strides
    qr, kr, vr, orr = rows
    out = np.full(o_len, np.nan, dtype=np.float64)
    r = np.arange(s)[:, None]
    c = np.arange(d)[None, :]
    for b in range(bh):
        Q = q[b * qs + r * qr + c].view(np.float16).astype(np.float64)
        K = k[b * ks + r * kr + c].view(np.float16).astype(np.float64)
        V = v[b * vs + r * vr + c].view(np.float16).astype(np.float64)
        sc = (Q @ K.T) * float(np.float32(scale))
        if causal:
            sc = np.where(np.tril(np.ones((s, s), dtype=bool)), sc, -np.inf)
        sc -= sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=1, keepdims=True)
        out[b * os_ + r * orr + c] = p @ V
    return out


def case(name, rng, bh, s, d, causal, scale, dist, strides=None, rows=None):
    rows = rows or (d, d, d, d)
    strides = strides or tuple(s * rw for rw in rows)
    bufs = []
    for t in range(3):
        n = bh * strides[t]
        kind = dist[t] if isinstance(dist, tuple) and isinstance(dist[0], tuple) else dist
        if kind[0] == "normal":
            x = rng.normal(0.0, kind[1], size=n)
        else:
            x = rng.uniform(kind[1], kind[2], size=n)
        bufs.append(x.astype(np.float16).view(np.uint16))
    q, k, v = bufs
    o_len = bh * strides[3]
    o = f64_attention(q, k, v, bh, s, d, strides, rows, scale, causal, o_len)
    return name, dict(q=q, k=k, v=v, o_expected=o,
                      params=np.array([bh, s, d, int(causal), *strides, *rows], dtype=np.int64),
                      scale=np.array([scale], dtype=np.float32))


def ref_fill(n, mul, add, scale):
    i = np.arange(n, dtype=np.int64)
    return (((i * mul + add) % 17).astype(np.float32) * np.float32(scale)).astype(np.float16).view(np.uint16)


def main():
    rng = np.random.default_rng(20240611)
    cases = [
        case("u_s8_d16", rng, 1, 8, 16, False, 0.25, ("uniform", -1.0, 1.0)),
        case("n_s17_d16_causal", rng, 2, 17, 16, True, 0.25, ("normal", 1.0)),
        case("n_s32_d32_causal", rng, 1, 32, 32, True, 1 / np.sqrt(32), ("normal", 1.0)),
        case("n_s33_d64", rng, 2, 33, 64, False, 0.125, ("normal", 2.0)),
        case("rowpad_s40_d64_causal", rng, 1, 40, 64, True, 0.125, ("normal", 1.0),
             strides=(40 * 72 + 8, 40 * 64, 40 * 80 + 3, 40 * 68 + 5), rows=(72, 64, 80, 68)),
        case("peaked_s5_d32", rng, 3, 5, 32, False, 2.0, ("normal", 1.5)),
        case("mixed_s64_d64_causal", rng, 1, 64, 64, True, 0.125,
             (("normal", 3.0), ("normal", 3.0), ("uniform", -1.0, 1.0))),
    ]
    # The reference's third smoke case: fills and odd slice strides of src/main.zig:192.
    bh, s, d = 3, 49, 16
    strides = (49 * 16, 49 * 16 + 13, 49 * 16 + 17, 49 * 16 + 19)
    q = ref_fill(bh * strides[0], 3, 1, 0.125)
    k = ref_fill(bh * strides[1], 5, 2, 0.0625)
    v = ref_fill(bh * strides[2], 7, 3, 0.03125)
    o = f64_attention(q, k, v, bh, s, d, strides, (d, d, d, d), 1 / np.sqrt(d), True, bh * strides[3])
    cases.append(("ref_smoke2", dict(q=q, k=k, v=v, o_expected=o,
                                     params=np.array([bh, s, d, 1, *strides, d, d, d, d], dtype=np.int64),
                                     scale=np.array([1 / np.sqrt(d)], dtype=np.float32))))
    flat = {}
    for name, arrays in cases:
        for key, val in arrays.items():
            flat[f"{name}/{key}"] = val
    flat["names"] = np.array([n for n, _ in cases])
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT}: {len(cases)} cases, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
