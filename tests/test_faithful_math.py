"""The restated host libm (poorgrad_amd/csrc/faithful_math.h) against the
host glibc on every one of the 2^32 single-precision inputs, and its tables
against their definitions. These are the same source lines the device
kernels compile."""
import ctypes
import os
from pathlib import Path

import pytest

_LIB = Path(__file__).resolve().parent / "native" / "libfaithful_check.so"


@pytest.fixture(scope="module")
def check():
    if not _LIB.exists():
        pytest.fail(f"{_LIB} is not built; run `python -m poorgrad_amd.build`")
    lib = ctypes.CDLL(str(_LIB))
    lib.faithful_check.restype = ctypes.c_int64
    lib.faithful_check.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_uint32)]
    lib.faithful_tables_check.restype = ctypes.c_int
    return lib


def test_tables_follow_their_definitions(check):
    assert check.faithful_tables_check() == 0


@pytest.mark.parametrize("function, name", [(0, "expf"), (1, "logf"), (2, "tanhf"), (3, "sqrtf")])
def test_every_f32_input_matches_host_libm(check, function, name):
    threads = max(1, min(16, os.cpu_count() or 1))
    first = ctypes.c_uint32(0)
    bad = check.faithful_check(function, 0, 1 << 32, threads, ctypes.byref(first))
    assert bad == 0, f"{name}: {bad} inputs differ from the host libm, first 0x{first.value:08x}"
