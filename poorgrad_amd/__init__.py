"""poorgrad_amd: the MI355X (gfx950) execution backend for topos compiled plans.

The product is the native library ``libtopos_hip.so`` (HIP kernels and the C
ABI declared in ``include/topos_hip.h``). This package builds it in-tree and
binds it with ctypes for the tests and the benchmark; there is no CPU
fallback anywhere: importing without the built library raises ImportError.
"""
from . import _native  # noqa: F401  (fails loudly when the library is missing)
from ._native import EXACT, FAST, HipError, status, status_reason  # noqa: F401
