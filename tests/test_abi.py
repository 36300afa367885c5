"""The C ABI library builds, loads without a GPU and exports every entry
point include/hale_moe.h declares; host-side argument checks work without a
device."""
import ctypes
import os
import re

import pytest

import hale_moe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "hale_moe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hale_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(hale_moe.LIB_PATH)
    names = declared_symbols()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the Python view binds exactly the declared surface
    assert sorted(hale_moe.SIGNATURES) == names


def test_row_bytes_through_the_abi():
    assert hale_moe.row_bytes("q8_0", 64) == 68
    assert hale_moe.row_bytes("q4_0", 64) == 36
    assert hale_moe.row_bytes("f32", 64) == 256
    with pytest.raises(ValueError):
        hale_moe.row_bytes("q4_0", 33)
    assert hale_moe.lib().hale_block_bytes(99) == 0


def test_parse_dtype():
    assert hale_moe.parse_dtype("Q4") == hale_moe.Q4_0
    with pytest.raises(ValueError):
        hale_moe.parse_dtype("int3")


def test_context_creation_reports_status():
    """On a machine without a GPU creation fails with a message; with one it
    succeeds.  Either way nothing crashes and the status is meaningful."""
    h = ctypes.c_void_p()
    rc = hale_moe.lib().hale_ctx_create(0, ctypes.byref(h))
    if rc == hale_moe.OK:
        hale_moe.lib().hale_ctx_destroy(h)
    else:
        assert rc == hale_moe.EHIP
        assert hale_moe.lib().hale_last_error(None)


def test_null_arguments_are_rejected_without_a_device():
    L = hale_moe.lib()
    assert L.hale_ctx_create(0, None) == hale_moe.EINVAL
    assert L.hale_matvec(None, None, None, 0, None, 0) == hale_moe.EINVAL
    assert L.hale_moe_forward(None, 1, None, None, None, None, None) == hale_moe.EINVAL
    assert L.hale_matrix_shape(None, None, None, None) == hale_moe.EINVAL
