"""The C-ABI library: builds, loads beside torch, exports what the header declares.

No GPU work here: only host-side argument validation is exercised.
"""
import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (loads torch's HIP runtime first, as the product does)

from usaf_amd import _native as N

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "usaf_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(usaf_hip_\w+)\s*\(", text)))


def test_library_loads():
    lib = N.load()
    assert lib.usaf_hip_abi_version() == int(re.search(r"USAF_HIP_ABI_VERSION\s+(\d+)", open(HEADER).read()).group(1))


def test_every_declared_symbol_is_exported():
    lib = N.load()
    declared = _declared()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in usaf_hip.h but not exported"
    # the binding knows every declared entry point (and nothing undeclared)
    assert sorted(N.exported_symbols()) == declared


def test_single_hip_runtime_in_process():
    N.load()
    maps = open("/proc/self/maps").read()
    paths = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    assert len(paths) == 1, paths


def test_host_validation_errors():
    lib = N.load()
    # null pointers with work to do -> USAF_ERR_INVALID, message set, no GPU touched
    rc = lib.usaf_hip_dequant_q4(None, None, None, 1, 64, 128, 128, None, N.F16, None)
    assert rc == N.USAF_ERR_INVALID and "null" in N.last_error()
    rc = lib.usaf_hip_dequant_q4(None, None, None, 1, 64, 128, 128, None, 7, None)
    assert rc == N.USAF_ERR_INVALID and "out_dtype" in N.last_error()
    rc = lib.usaf_hip_quantize_q4(None, N.F32, 0, 128, None, None, None, None)
    assert rc == N.USAF_ERR_INVALID
    # too few nibbles for the groups: same failure the reference's view() raises
    rc = lib.usaf_hip_dequant_q4(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 2, 10, 128, 256,
                                 ctypes.c_void_p(16), N.F16, None)
    assert rc == N.USAF_ERR_INVALID and "exceed" in N.last_error()
    with pytest.raises(ValueError):
        N.check(rc, "dequant")
    # empty work is a no-op success
    assert lib.usaf_hip_dequant_q4(None, None, None, 0, 64, 128, 0, None, N.F16, None) == N.USAF_OK
