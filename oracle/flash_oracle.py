"""ctypes wrapper of the CPU oracle (``oracle/flash_ref.c``).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker. The product path never calls it.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C oracle`")
        _lib = ctypes.CDLL(LIB_PATH)
        u64 = ctypes.c_uint64
        p = ctypes.c_void_p
        _lib.oracle_flash_fwd.restype = ctypes.c_int
        _lib.oracle_flash_fwd.argtypes = [u64, u64, u64, p, u64, u64, p, u64, u64, p, u64, u64, p, u64, u64,
                                          ctypes.c_float, ctypes.c_uint32, ctypes.c_int, p, u64]
        _lib.oracle_flash_fwd_typed.restype = ctypes.c_int
        _lib.oracle_flash_fwd_typed.argtypes = list(_lib.oracle_flash_fwd.argtypes) + [ctypes.c_uint32]
        _lib.oracle_half_to_float.restype = ctypes.c_float
        _lib.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        _lib.oracle_bf16_to_float.restype = ctypes.c_float
        _lib.oracle_bf16_to_float.argtypes = [ctypes.c_uint16]
    return _lib


def flash_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, o: np.ndarray, *, batch_heads: int, seq_len: int,
              head_dim: int, q_stride: int, k_stride: int, v_stride: int, o_stride: int, scale: float,
              causal: bool, q_row: int = 0, k_row: int = 0, v_row: int = 0, o_row: int = 0, threads: int = 1,
              rows: Optional[Sequence[int]] = None, dtype: str = "f16") -> np.ndarray:
    """Run computeFlashReferenceOne (src/main.zig:1271-1307) over every slice, writing into ``o``
    (float32, modified in place and returned). q/k/v are uint16 bit patterns of f16 (the
    reference's type) or, with dtype="bf16", of bfloat16."""
    assert q.dtype == np.uint16 and k.dtype == np.uint16 and v.dtype == np.uint16 and o.dtype == np.float32
    for a in (q, k, v, o):
        assert a.flags.c_contiguous
    rows_arr = None
    nrows = 0
    if rows is not None:
        rows_arr = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
        nrows = rows_arr.size
    rc = lib().oracle_flash_fwd_typed(batch_heads, seq_len, head_dim, q.ctypes.data, q_stride, q_row,
                                      k.ctypes.data, k_stride, k_row, v.ctypes.data, v_stride, v_row, o.ctypes.data,
                                      o_stride, o_row, scale, 1 if causal else 0, threads,
                                      None if rows_arr is None else rows_arr.ctypes.data, nrows,
                                      {"f16": 0, "bf16": 1}[dtype])
    if rc != 0:
        raise RuntimeError("oracle_flash_fwd failed")
    return o


def half_to_float(h: int) -> float:
    return float(lib().oracle_half_to_float(h))


def bf16_to_float(h: int) -> float:
    return float(lib().oracle_bf16_to_float(h))
