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
        pytest.fail(f"{_LIB} is not built; run `python poorgrad_amd/build.py`")
    lib = ctypes.CDLL(str(_LIB))
    lib.faithful_check.restype = ctypes.c_int64
    lib.faithful_check.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_uint32)]
    lib.faithful_tables_check.restype = ctypes.c_int
    lib.pow_check.restype = ctypes.c_int64
    lib.pow_check.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int,
                              ctypes.POINTER(ctypes.c_float)]
    return lib


def test_tables_follow_their_definitions(check):
    assert check.faithful_tables_check() == 0


@pytest.mark.parametrize("function, name", [(0, "expf"), (1, "logf"), (2, "tanhf"), (3, "sqrtf")])
def test_every_f32_input_matches_host_libm(check, function, name):
    threads = max(1, min(16, os.cpu_count() or 1))
    first = ctypes.c_uint32(0)
    bad = check.faithful_check(function, 0, 1 << 32, threads, ctypes.byref(first))
    assert bad == 0, f"{name}: {bad} inputs differ from the host libm, first 0x{first.value:08x}"


POW_FAMILIES = ["random bits", "positive bases, moderate exponents", "negative bases, integer exponents",
                "bases near one, large exponents", "overflow and underflow edges", "dyadic exponents"]


@pytest.mark.parametrize("family", range(len(POW_FAMILIES)), ids=POW_FAMILIES)
def test_powf_matches_host_libm_on_dense_samples(check, family):
    """powf has 2^64 input pairs, so it is checked on 2^25 seeded pairs per
    family instead (NaN as a class), chosen to cover its special cases, both
    signs and the exponent range, and the rounding of results near overflow
    and underflow."""
    threads = max(1, min(16, os.cpu_count() or 1))
    bad = (ctypes.c_float * 2)()
    count = check.pow_check(family, 7, 1 << 25, threads, bad)
    assert count == 0, f"{POW_FAMILIES[family]}: {count} pairs differ, first powf({bad[0]!r}, {bad[1]!r})"
