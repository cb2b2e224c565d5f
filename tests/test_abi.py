"""The C-ABI library loads and exports exactly what include/undertow_hip.h declares.

CPU only: no compute calls (there is no GPU in the build container); the one
call made, ut_ctx_create, must fail with a status code rather than crash when
no device is visible.
"""
import ctypes as C
import re

import pytest

from conftest import ROOT


def header_functions():
    text = (ROOT / "include" / "undertow_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ut_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from undertow_amd import runtime

    assert header_functions() == sorted(runtime.EXPORTED)


def test_library_exports_every_declared_symbol():
    import undertow_amd as U

    assert U.LIB_PATH.exists(), "build the library first (__graft_entry__.build())"
    L = U.lib()
    for name in header_functions():
        assert hasattr(L, name), name


def test_ctx_create_without_device_returns_status():
    import torch
    import undertow_amd as U

    if torch.cuda.is_available():
        pytest.skip("a device is visible; covered by the GPU tests")
    h = C.c_void_p()
    rc = U.lib().ut_ctx_create(0, C.byref(h))
    assert rc == U.runtime.UT_ERR_HIP and not h.value


def test_null_handles_are_rejected():
    import undertow_amd as U

    L = U.lib()
    assert L.ut_qtensor_format(None) == U.runtime.UT_ERR_ARG
    assert L.ut_ctx_synchronize(None) == U.runtime.UT_ERR_ARG
    assert L.ut_last_error(None) == b"null context"
