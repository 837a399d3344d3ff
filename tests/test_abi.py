"""The C ABI without a GPU: libtrmoe.so loads, exports every function that
include/trmoe.h declares, and answers the host-only queries (layout sizes,
workspace sizes, argument validation) that need no device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from complexity_amd import _native, build_native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "trmoe.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^[a-z][\w\s\*]*?\b(trmoe_\w+)\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        build_native.build(verbose=False)
    return _native.load()


def test_header_and_binding_list_the_same_functions():
    assert _declared() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(_native.LIB_PATH))
    for name in _declared():
        assert hasattr(raw, name), name


def test_abi_version(lib):
    assert lib.trmoe_abi_version() == _native.ABI_VERSION


def test_pack_dims_layout_rules(lib):
    rows, cols = ctypes.c_int64(), ctypes.c_int64()
    # gate|up: 32-row groups of gate then up, out rounded to row_align/2 per half
    assert lib.trmoe_pack_dims(_native.PACK_GATE_UP, 3072, 896, 256, ctypes.byref(rows), ctypes.byref(cols)) == 0
    assert (rows.value, cols.value) == (6144, 896)
    assert lib.trmoe_pack_dims(_native.PACK_GATE_UP, 100, 30, 128, ctypes.byref(rows), ctypes.byref(cols)) == 0
    assert (rows.value, cols.value) == (256, 32)
    assert lib.trmoe_pack_dims(_native.PACK_PLAIN, 896, 3072, 256, ctypes.byref(rows), ctypes.byref(cols)) == 0
    assert (rows.value, cols.value) == (1024, 3072)
    assert lib.trmoe_pack_dims(7, 8, 8, 64, ctypes.byref(rows), ctypes.byref(cols)) == _native.ERR_INVALID
    assert b"kind" in lib.trmoe_last_error()


def test_dense_routed_feature_count(lib):
    # shared features padded to 128, each expert block to 64, total to 128
    assert lib.trmoe_dense_routed_features(3072, 4, 64) == 3328
    assert lib.trmoe_dense_routed_features(100, 3, 10) == 384
    assert lib.trmoe_dense_routed_features(0, 16, 256) == 4096


def test_route_sort_workspace_is_sized_without_a_device(lib):
    small = lib.trmoe_route_sort_workspace_bytes(64, 2, 4, _native.ORDER_TOKEN)
    big = lib.trmoe_route_sort_workspace_bytes(1 << 20, 2, 16, _native.ORDER_TOKEN)
    assert 0 <= small <= big


def test_invalid_arguments_fail_before_touching_a_device(lib):
    st = lib.trmoe_shared_gate_up(_native.BF16, _native.BF16, None, 16, 64, 64, None, None, 128, None, 128, None)
    assert st == _native.ERR_INVALID
    assert lib.trmoe_last_error()
    with pytest.raises(ValueError):
        _native.check(st, "trmoe_shared_gate_up")


def test_rmsnorm_workspace_and_validation_without_a_device(lib):
    """One fp32 weight partial per backward workgroup (4 rows each, at most
    1024 of them); unsupported hidden sizes size to 0 and are rejected."""
    bf, f32 = _native.BF16, _native.F32
    assert lib.trmoe_rmsnorm_backward_workspace_bytes(bf, 0, 896) == 896 * 4
    assert lib.trmoe_rmsnorm_backward_workspace_bytes(bf, 5, 896) == 2 * 896 * 4
    assert lib.trmoe_rmsnorm_backward_workspace_bytes(bf, 16384, 896) == 1024 * 896 * 4
    assert lib.trmoe_rmsnorm_backward_workspace_bytes(f32, 4096, 2048) == 1024 * 2048 * 4
    for dt, hidden in ((bf, 100), (bf, 4104), (f32, 2052), (f32, 6)):
        assert lib.trmoe_rmsnorm_backward_workspace_bytes(dt, 64, hidden) == 0
        st = lib.trmoe_rmsnorm_forward(dt, None, 16, hidden, hidden, None, 1e-6, None, hidden, None, None)
        assert st == _native.ERR_INVALID
    st = lib.trmoe_rmsnorm_forward(bf, None, 16, 896, 896, None, 1e-6, None, 896, None, None)
    assert st == _native.ERR_INVALID and b"null" in lib.trmoe_last_error()
    st = lib.trmoe_rmsnorm_backward(bf, None, 16, 896, 896, None, None, None, 896, None, 0, None, 896, None,
                                    None, 0, None)
    assert st == _native.ERR_INVALID
