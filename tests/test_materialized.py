"""Host-side tests of the materialized-attention baseline library (include/notcute_baselines.h):
exported symbols, workspace size (tools/cuda_baselines.cu:683-686, 757) and argument validation,
all without a GPU call."""

import ctypes
import os
import re

import pytest

import notcute_flash as nc
from flash_workloads import CONFIGS

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "notcute_baselines.h")


def test_baselines_library_exports_every_declared_function():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(nc_[a-z0-9_]+)\s*\(", text)))
    assert len(names) == 5
    lib = nc.baselines_library()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_workspace_is_scores_plus_probabilities():
    # scores_len * (sizeof(float) + sizeof(half)), scores_len = BH*S*S
    assert nc.Materialized.workspace_bytes(CONFIGS["c4"].options()) == 32 * 4096 * 4096 * 6
    assert nc.Materialized.workspace_bytes(CONFIGS["c1"].options()) == 1 * 32 * 32 * 6
    # causal changes nothing: both GEMMs cover the full S x S matrices
    assert nc.Materialized.workspace_bytes(CONFIGS["c3"].options()) == 8 * 1024 * 1024 * 6


def test_workspace_zero_for_invalid_or_overflowing_options():
    assert nc.Materialized.workspace_bytes(nc.options(seq_len=16, head_dim=24)) == 0
    huge = nc.options(batch_heads=1 << 20, seq_len=1 << 22, head_dim=16)
    assert nc.Materialized.workspace_bytes(huge) == 0  # 2^20 * 2^44 * 6 overflows 64 bits


def _attention(opts, plan=None, lens=(10 ** 6,) * 4, ws=10 ** 9):
    lib = nc.baselines_library()
    p = ctypes.c_void_p(0x10)
    return nc.STATUS_NAMES[lib.nc_materialized_attention(
        plan, p, lens[0], p, lens[1], p, lens[2], p, lens[3], p, ws, ctypes.byref(opts))]


def test_validation_before_any_device_work():
    """Every rejection below returns before the (fake) plan or pointers are touched."""
    fake_plan = ctypes.c_void_p(0x20)
    assert _attention(nc.options(seq_len=16, head_dim=24), fake_plan) == "InvalidValue"   # flash.Options rules
    good = nc.options(batch_heads=2, seq_len=16, head_dim=16)
    assert _attention(good, None) == "InvalidValue"                                         # no plan
    assert _attention(good, fake_plan, lens=(512, 512, 512, 511)) == "InvalidValue"         # requireLen on O
    assert _attention(good, fake_plan, ws=2 * 16 * 16 * 6 - 1) == "InvalidValue"            # workspace short
    long = nc.options(seq_len=nc.MATERIALIZED_MAX_SEQ + 1, head_dim=16)
    assert _attention(long, fake_plan, lens=(10 ** 7,) * 4, ws=1 << 40) == "InvalidValue"   # softmax limit


def test_last_error_names_the_failure():
    fake_plan = ctypes.c_void_p(0x20)
    good = nc.options(batch_heads=2, seq_len=16, head_dim=16)
    _attention(good, fake_plan, ws=1)
    assert "workspace" in nc.baselines_library().nc_materialized_last_error().decode()


def test_destroy_null_plan_is_a_no_op():
    assert nc.baselines_library().nc_materialized_destroy(None) == 0


@pytest.mark.parametrize("impl", ["rocblas_materialized"])
def test_compare_table_lists_the_baseline(impl):
    import flash_harness as fh

    recs = [fh.make_record("not_cute", "s", True, 1.0, 1.0, 1.0, 10, 10, 0.0),
            fh.make_record(impl, "s", True, 3.0, 3.0, 3.0, 10, 10, 0.0)]
    table = fh.compare_table(recs)
    assert impl in table and "3.00x" in table
