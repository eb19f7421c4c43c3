"""The C ABI library loads and exports every symbol include/scry_hip.h declares.
CPU only: no compute calls."""
import ctypes

import pytest


def test_library_exports_every_declared_symbol():
    from esolearn_amd import _lib

    L = _lib.load()
    names = _lib.header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding declares exactly the header's functions
    assert set(_lib.SIGNATURES) == set(names)


def test_library_is_gfx950_only():
    from esolearn_amd import _lib

    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    for other in (b"amdgcn-amd-amdhsa--gfx942", b"amdgcn-amd-amdhsa--gfx90a"):
        assert other not in data


def test_calls_before_init_fail_cleanly():
    import esolearn_amd as E
    from esolearn_amd import _lib

    n = ctypes.c_int()
    _lib.call("scry_hip_device_count", ctypes.byref(n))
    if n.value > 0:
        pytest.skip("a GPU is present; the no-device path is not reachable")
    with pytest.raises(E.ScryHipError) as ei:
        E.init(0)
    assert ei.value.code == 4  # SCRY_ERR_NOT_INIT
    with pytest.raises(E.ScryHipError) as ei:
        E.HipBackend.zeros(8)
    assert ei.value.code == 4
    assert "scry_hip_init not called" in str(ei.value)
    assert b"not called" in _lib.load().scry_hip_last_error()
