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


@pytest.mark.parametrize("env,want", [
    ({}, 1),
    ({"SCRY_HIP_NO_GRAPH": "1"}, 0),
    ({"ROCP_TOOL_LIBRARIES": "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so"}, 0),
    ({"ROCP_TOOL_LIBRARIES": ""}, 1),
])
def test_graph_replay_off_under_a_profiler_tool(env, want):
    """Decode steps replay captured graphs unless SCRY_HIP_NO_GRAPH is set or
    a rocprofiler tool is attached (rocprofv3 sets ROCP_TOOL_LIBRARIES): the
    profiler's hipGraphLaunch interception faulted the process, so profiled
    runs take direct launches.  Decided from the environment once per process,
    so each case runs in a fresh interpreter; no device is used."""
    import os
    import subprocess
    import sys

    from esolearn_amd import _lib

    base = {k: v for k, v in os.environ.items() if k not in ("SCRY_HIP_NO_GRAPH", "ROCP_TOOL_LIBRARIES")}
    code = ("import ctypes, sys; L = ctypes.CDLL(sys.argv[1]); "
            "print(L.scry_hip_graph_replay())")
    out = subprocess.run([sys.executable, "-c", code, _lib.LIB_PATH], env={**base, **env},
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert int(out.stdout.strip().splitlines()[-1]) == want
