"""The C ABI without a GPU: the library loads, exports every function that
include/exn_hip.h declares, the Python binding's table matches the header,
and calls that cannot run return clean status codes (no abort)."""
import ctypes
import os
import re

import pytest

import exn_hip as X

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "exn_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(exn_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_trio_and_ops():
    names = declared()
    for n in ("exn_open", "exn_dit_create", "exn_dit_set", "exn_dit_velocity", "exn_dit_release", "exn_mm",
              "exn_attend", "exn_ln_mod", "exn_qkv_prep", "exn_weight_q8_0"):
        assert n in names
    assert len(names) >= 40


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(X.LIB_PATH)
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    assert sorted(X.SIGNATURES) == declared()


def test_library_is_gfx950_code():
    # the shared object carries a gfx950 code object (hipcc --offload-arch=gfx950)
    data = open(X.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_no_gpu_paths_return_status():
    L = X.lib()
    assert L.exn_version() >= 1
    # null arguments are refused before any device call
    assert L.exn_open(0, None) == X.EINVAL
    assert L.exn_sync(None) == X.EINVAL
    assert L.exn_mm(None, None, None, 0, None, 0, 1) == X.EINVAL
    assert L.exn_dit_check(None) == X.EINVAL
    assert L.exn_dit_release(None) == X.EINVAL
    assert b"null" in L.exn_last_error()
    assert L.exn_dit_trace(None, None, 0) == X.EINVAL
    assert L.exn_close(None) == X.OK and L.exn_dit_destroy(None) == X.OK and L.exn_weight_free(None) == X.OK


def test_open_without_a_gpu_is_enodev():
    n = ctypes.c_int(-1)
    r = X.lib().exn_device_count(ctypes.byref(n))
    if r == X.OK and n.value > 0:
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    assert X.lib().exn_open(0, ctypes.byref(h)) == X.ENODEV
    assert not h.value
    with pytest.raises(X.ExnError) as e:
        X.Context(0)
    assert e.value.code == X.ENODEV
