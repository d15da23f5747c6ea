"""The C ABI boundary, checked on the CPU: the library loads, and it exports
exactly the entry points include/mockbird_hip.h declares (no compute calls)."""
import ctypes
import os
import re

import pytest

import mockbird_amd as mb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "mockbird_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(mb_[a-z0-9_]+)\s*\(", src))


def test_header_declares_the_python_export_list():
    assert _declared() == set(mb.EXPORTS)


def test_library_exports_every_declared_symbol():
    if not os.path.exists(mb.LIB_PATH):
        pytest.fail("libmockbird_hip.so is not built (python -m mockbird_amd.build)")
    lib = ctypes.CDLL(mb.LIB_PATH)
    missing = [s for s in sorted(_declared()) if not hasattr(lib, s)]
    assert not missing, missing


def test_abi_version_and_argument_errors():
    lib = mb.load()
    assert lib.mb_abi_version() == 2
    # a bad config is rejected before any device call
    cfg = mb.Config(0, 0, 0, 0, 0, 0, 0, 0)
    h = ctypes.c_void_p()
    assert lib.mb_create(ctypes.byref(cfg), ctypes.byref(h)) == mb.MB_ERR_ARG
    assert not h.value
    assert lib.mb_create(None, None) == mb.MB_ERR_ARG
    assert lib.mb_last_error(None) == b"null context"
