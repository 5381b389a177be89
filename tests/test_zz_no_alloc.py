"""The no-allocation product (topos_hip_gemm_f32_device_noalloc) against the
allocating device-face product (topos_hip_gemm_f32_device), both called
through the C ABI on the same operands. Both launch the same kernels with the
same split along k; only the home of the split partials differs (a fixed
device array instead of the library's workspace), so the results must agree
bit for bit, and each must meet the oracle's bar (gemm::multiply,
src/payload/gemm.rs:140-211): bitwise under Exact, within
|c - exact| <= 1e-5 * sum_k |a_ik b_kj| under Fast.

Two calls in a row share the fixed array, the second with a smaller product,
so the second runs over the first's leftover partials."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import banner
from tests.gpu_util import assert_bitwise, to_device

pytestmark = pytest.mark.gpu

# (m, k, n, seed). Under Fast both split k: 16 partials of 512 x 512 (16 MiB)
# then 8 of 256 x 384, each within the 64 MiB array.
CASES = [(512, 4096, 512, 21), (256, 2048, 384, 22)]


def _product(entry, a, a_strides, b, b_strides, m, k, n, numerics):
    from poorgrad_amd import _native as nat

    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    code = getattr(nat.lib, entry)(a.data_ptr(), a_strides[0], a_strides[1], b.data_ptr(), b_strides[0],
                                   b_strides[1], m, k, n, numerics, out.data_ptr(), n,
                                   torch.cuda.current_stream().cuda_stream)
    nat.checked(code, entry)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _operands(m, k, n, seed, transposed):
    g = oracle.Generator(seed)
    a = g.normal(m * k, 1.0).reshape(m, k)
    b = g.normal(k * n, 1.0).reshape(k, n)
    if transposed:  # A^T . G: the left operand stored [k, m], strides [1, m]
        return a, b, to_device(np.ascontiguousarray(a.T)), (1, m), to_device(b), (n, 1)
    return a, b, to_device(a), (k, 1), to_device(b), (n, 1)


@pytest.mark.parametrize("transposed", [False, True], ids=["a_b", "at_b"])
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_noalloc_product_equals_allocating_product(hip, posture, transposed):
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    prepared = [(case, _operands(*case, transposed)) for case in CASES]
    allocating = []
    for (m, k, n, seed), (_, _, da, ast, db, bst) in prepared:
        banner(f"noalloc: allocating product {posture} {m}x{k}x{n} transposed={transposed}")
        allocating.append(_product("topos_hip_gemm_f32_device", da, ast, db, bst, m, k, n, numerics))
    # The no-allocation calls back to back: the second, smaller product runs
    # over the first's partials left in the shared array.
    fixed = []
    for (m, k, n, seed), (_, _, da, ast, db, bst) in prepared:
        banner(f"noalloc: no-allocation product {posture} {m}x{k}x{n} transposed={transposed}")
        fixed.append(_product("topos_hip_gemm_f32_device_noalloc", da, ast, db, bst, m, k, n, numerics))
    for ((m, k, n, seed), (a, b, *_)), want, got in zip(prepared, allocating, fixed):
        assert_bitwise(got, want, f"noalloc vs allocating {posture} {m}x{k}x{n}")
        exact = oracle.gemm(a.ravel(), (k, 1), b.ravel(), (n, 1), m, k, n)
        if numerics == hip.EXACT:
            assert_bitwise(got, exact, f"noalloc vs oracle {m}x{k}x{n}")
        else:
            bound = 1e-5 * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
            assert (np.abs(got.astype(np.float64) - exact) <= bound).all(), f"envelope {m}x{k}x{n}"


def test_noalloc_refuses_partials_beyond_its_array(hip):
    from poorgrad_amd import _native as nat

    # 2048 x 2048 over k = 8192 splits six ways under Fast: 96 MiB of partials.
    m, k, n = 2048, 8192, 2048
    banner(f"noalloc: refusal {m}x{k}x{n}")
    a = torch.randn((m, k), device="cuda", generator=torch.Generator("cuda").manual_seed(5))
    b = torch.randn((k, n), device="cuda", generator=torch.Generator("cuda").manual_seed(6))
    out = torch.zeros((m, n), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    code = nat.lib.topos_hip_gemm_f32_device_noalloc(a.data_ptr(), k, 1, b.data_ptr(), n, 1, m, k, n, nat.FAST,
                                                     out.data_ptr(), n, stream)
    assert code == nat.INVALID_ARGUMENT
    assert b"scratch" in nat.lib.topos_hip_last_refusal()
    assert nat.status() == nat.OK  # a refusal does not poison
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(out)) == 0  # nothing was launched
    # The exact posture needs no scratch at any size: bitwise equal to the
    # allocating entry point.
    banner(f"noalloc: exact at {m}x{k}x{n}")
    want = _product("topos_hip_gemm_f32_device", a, (k, 1), b, (n, 1), m, k, n, nat.EXACT)
    got = _product("topos_hip_gemm_f32_device_noalloc", a, (k, 1), b, (n, 1), m, k, n, nat.EXACT)
    assert_bitwise(got, want, "noalloc exact, large")
