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


# entry points without a context argument, or whose result is not a status
_NO_CTX = {"mb_abi_version", "mb_create", "mb_last_error", "mb_destroy", "mb_get_stream",
           "mb_device_bytes"}


def test_every_entry_point_rejects_a_null_context():
    """Each status-returning entry point called with a null context (and null
    or zero for every other argument) returns MB_ERR_ARG before touching
    anything; the others return their neutral value.  Run under
    AddressSanitizer by test_host_sanitized.py, any dereference on the way
    would be reported."""
    lib = mb.load()
    for name in sorted(mb.EXPORTS):
        fn = getattr(lib, name)
        if name in _NO_CTX or fn.argtypes is None:
            continue
        args = [None if t in (ctypes.c_void_p, ctypes.c_char_p) or hasattr(t, "_type_") and
                not isinstance(t._type_, str) else 0 for t in fn.argtypes]
        assert fn(*args) == mb.MB_ERR_ARG, name
    lib.mb_destroy(None)
    assert lib.mb_get_stream(None) is None
    assert lib.mb_device_bytes(None) in (0, -1)


def test_create_fails_cleanly_or_succeeds():
    """A valid configuration: on a host without a GPU mb_create returns
    MB_ERR_HIP with the runtime's message and no context (its clean-up path
    runs); on a GPU host it creates one, which is destroyed again."""
    lib = mb.load()
    cfg = mb.Config(2, 64, 16, 2, 16, mb.MB_KV_BF16, 1, 0)
    h = ctypes.c_void_p()
    rc = lib.mb_create(ctypes.byref(cfg), ctypes.byref(h))
    if rc == mb.MB_OK:
        assert h.value
        lib.mb_destroy(h)
    else:
        assert rc == mb.MB_ERR_HIP and not h.value
    bad = [mb.Config(1, 64, 16, 2, 16, 7, 1, 0),           # unknown KV type
           mb.Config(1, 64, 0, 2, 16, 0, 1, 0),            # no ring
           mb.Config(1, 64, 16, 0, 16, 0, 1, 0),           # no sequences
           mb.Config(-3, 64, 16, 2, 16, 0, 1, 0),          # negative layers
           mb.Config(1, 64, 16, 2, 16, 0, 1, -1),          # negative device
           mb.Config(1, 64, 1 << 30, 1 << 20, 16, 0, 1, 0)]  # absurd ring
    for c in bad:
        h = ctypes.c_void_p()
        assert lib.mb_create(ctypes.byref(c), ctypes.byref(h)) in (mb.MB_ERR_ARG,
                                                                     mb.MB_ERR_NOMEM), (
            c.n_layers, c.capacity, c.max_seqs, c.kv_dtype, c.device)
        assert not h.value
