"""The C-ABI library without a GPU: it loads, exports every function
``include/mlc_hip.h`` declares with the signature the ctypes layer binds,
and its argument checks fail cleanly with a message (no device call is made
on these paths)."""

from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from mlc.runtime import native

HEADER = native.INCLUDE / "mlc_hip.h"


def _declared():
    text = HEADER.read_text()
    body = text[text.index('extern "C" {'):]
    return sorted(set(re.findall(r"\b(mlc_[a-z_]+)\s*\(", body)))


@pytest.fixture(scope="module")
def lib():
    if not native.LIB_PATH.exists():
        native.build_library()
    return native.load_library()


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 19
    out = subprocess.run(["nm", "-D", "--defined-only", str(native.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (mlc_[a-z_]+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        assert hasattr(lib, n)


def test_ctypes_table_matches_header():
    assert sorted(native.SIGNATURES) == _declared()


def test_version(lib):
    assert lib.mlc_version() >> 16 == 1


def test_argument_errors_return_codes_and_messages(lib):
    out = ctypes.c_void_p()
    assert lib.mlc_ctx_create(0, None) == -10001
    assert b"null out" in lib.mlc_last_error()
    assert lib.mlc_plan_create(None, 3, ctypes.byref(out)) == -10001
    assert lib.mlc_slab_alloc(None, 1024, ctypes.byref(out)) == -10001
    assert lib.mlc_module_load(None, None, 0, ctypes.byref(out)) == -10001
    assert lib.mlc_launch(None, 1, 64, 0, None, 0, None) == -10001
    assert b"geometry" in lib.mlc_last_error()
    assert lib.mlc_graph_replay(None, None) == -10001
    assert lib.mlc_plan_run(None, 0, 0, None) == -10001
    assert lib.mlc_ctx_destroy(None) == 0
    assert lib.mlc_plan_destroy(None) == 0


def test_check_raises_with_the_library_message(lib):
    rc = lib.mlc_plan_set(None, 0, None, 1, 64, 0, None, 0)
    with pytest.raises(native.NativeError, match="mlc_plan_set"):
        native.check(rc, "mlc_plan_set")
