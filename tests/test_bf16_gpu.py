"""bf16 products on the device (topos_hip_gemm_bf16_device) against the
oracle's Bf16::gemm (src/payload/bf16.rs:235-262: widen, f32 product, one
rounding): bit-identical under Exact; under Fast (bf16 matrix cores, f32
accumulation) within |c - exact| <= 1e-5 * sum_k |a_ik b_kj| before the
rounding, so within that plus one bf16 spacing of the rounded exact
result. Shapes and stride forms as the f32 grid (forward, both transposed
operands, a narrowed window, and rows not 16-byte aligned), and products
with few tiles over deep k, which Fast cuts into k ranges (f32 partials
added in range order, one rounding)."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import banner

pytestmark = pytest.mark.gpu

SHAPES = [(2, 3, 4), (5, 8, 13), (16, 16, 16), (63, 64, 65), (100, 127, 3), (129, 257, 131), (256, 384, 512),
          (1024, 1024, 1024), (777, 1000, 515),
          # few tiles over deep k: under Fast, k in 8 ranges and in 4 ragged ones
          (128, 4096, 192), (300, 2600, 260),
          # a single output row or column, and k = 1 (operands of outer extent 1, packs of one k)
          (1, 77, 300), (300, 77, 1), (70, 1, 90)]
FORMS = ["contiguous", "a_transposed", "b_transposed", "narrowed"]


def _operands(m, k, n, form, seed):
    g = oracle.Generator(seed)
    a = oracle.bf16_round(g.normal(m * k, 1.0).reshape(m, k))
    b = oracle.bf16_round(g.normal(k * n, 1.0).reshape(k, n))
    a_buf, a_st, a_off = a.ravel(), (k, 1), 0
    b_buf, b_st = b.ravel(), (n, 1)
    if form == "a_transposed":
        a_buf, a_st = np.ascontiguousarray(a.T).ravel(), (1, m)
    if form == "b_transposed":
        b_buf, b_st = np.ascontiguousarray(b.T).ravel(), (1, k)
    if form == "narrowed":
        wide = np.zeros((m, k + 3), np.uint16)
        wide[:, 1:1 + k] = a
        a_buf, a_st, a_off = wide.ravel(), (k + 3, 1), 1
    return a, b, (a_buf, a_st, a_off), (b_buf, b_st)


def _device(a_view, b_view, m, k, n, numerics):
    from poorgrad_amd import _native as nat

    (a_buf, a_st, a_off), (b_buf, b_st) = a_view, b_view
    da = torch.from_numpy(a_buf.view(np.int16).copy()).cuda()
    db = torch.from_numpy(b_buf.view(np.int16).copy()).cuda()
    out = torch.zeros((m, n), dtype=torch.int16, device="cuda")
    nat.checked(nat.lib.topos_hip_gemm_bf16_device(da.data_ptr() + 2 * a_off, a_st[0], a_st[1], db.data_ptr(), b_st[0],
                                                   b_st[1], m, k, n, numerics, out.data_ptr(), n,
                                                   torch.cuda.current_stream().cuda_stream), "bf16 gemm")
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("m, k, n", SHAPES)
def test_bf16_gemm_exact_and_fast(hip, m, k, n, form):
    banner(f"bf16 gemm {m}x{k}x{n} {form}")
    a, b, a_view, b_view = _operands(m, k, n, form, seed=m + 3 * k + 7 * n)
    want = oracle.gemm_bf16(a, (k, 1), b, (n, 1), m, k, n)
    exact = _device(a_view, b_view, m, k, n, hip.EXACT)
    assert np.array_equal(exact, want), f"exact: {int((exact != want).sum())} differ"
    fast = _device(a_view, b_view, m, k, n, hip.FAST)
    wa, wb = oracle.bf16_widen(a).astype(np.float64), oracle.bf16_widen(b).astype(np.float64)
    bound = 1e-5 * (np.abs(wa) @ np.abs(wb))
    w = oracle.bf16_widen(want).astype(np.float64)
    spacing = np.abs(w) * 2.0**-7 + 1e-38  # one bf16 step at the exact result
    assert (np.abs(oracle.bf16_widen(fast).astype(np.float64) - w) <= bound + spacing).all()
    again = _device(a_view, b_view, m, k, n, hip.FAST)
    assert np.array_equal(again, fast), "fast bf16 products repeat bit for bit"


def test_bf16_product_accumulates_in_f32(hip):
    """src/payload/tests/bf16_tests.rs:117-127 on the device, both postures:
    [256, 1, 1] . [1, 1, 1] = 258, per-op bf16 accumulation would say 256."""
    banner("bf16 gemm 258")
    a = oracle.bf16_round(np.array([[256.0, 1.0, 1.0]] * 2, np.float32))
    b = oracle.bf16_round(np.array([[1.0, 1.0], [1.0, 1.0], [1.0, 1.0]], np.float32))
    for numerics in (hip.EXACT, hip.FAST):
        got = _device((a.ravel(), (3, 1), 0), (b.ravel(), (2, 1)), 2, 3, 2, numerics)
        assert (oracle.bf16_widen(got) == 258.0).all(), got


@pytest.mark.parametrize("a_transposed", [False, True])
def test_bf16_narrow_slices_of_wide_buffers(hip, a_transposed):
    """Column slices of wide buffers (a [512, 48] window of a [512, 30011]
    buffer, a [48, 80] window of a [48, 30011] one): the exact path packs the
    operands densely, so its workspace is the product's size, not the
    views' spans; both postures against the oracle."""
    banner(f"bf16 gemm narrow slices a_transposed={a_transposed}")
    m, k, n, wide, start = 512, 48, 80, 30011, 1000
    g = oracle.Generator(5)
    a = oracle.bf16_round(g.normal(m * k, 1.0).reshape(m, k))
    b = oracle.bf16_round(g.normal(k * n, 1.0).reshape(k, n))
    if a_transposed:
        a_host = np.zeros((k, wide), np.uint16)
        a_host[:, start:start + m] = a.T
        a_view = (a_host.ravel(), (1, wide), start)
    else:
        a_host = np.zeros((m, wide), np.uint16)
        a_host[:, start:start + k] = a
        a_view = (a_host.ravel(), (wide, 1), start)
    b_host = np.zeros((k, wide), np.uint16)
    b_host[:, start:start + n] = b
    b_buf = b_host.ravel()[start:]
    want = oracle.gemm_bf16(a, (k, 1), b, (n, 1), m, k, n)
    exact = _device(a_view, (b_buf, (wide, 1)), m, k, n, hip.EXACT)
    assert np.array_equal(exact, want), f"exact: {int((exact != want).sum())} differ"
    fast = _device(a_view, (b_buf, (wide, 1)), m, k, n, hip.FAST)
    wa, wb = oracle.bf16_widen(a).astype(np.float64), oracle.bf16_widen(b).astype(np.float64)
    w = oracle.bf16_widen(want).astype(np.float64)
    bound = 1e-5 * (np.abs(wa) @ np.abs(wb)) + np.abs(w) * 2.0**-7 + 1e-38
    assert (np.abs(oracle.bf16_widen(fast).astype(np.float64) - w) <= bound).all()


@pytest.mark.parametrize("m, k, n", [(4096, 4096, 4096), (8192, 768, 3072), (3072, 8192, 768)])
@pytest.mark.parametrize("form", ["contiguous", "a_transposed", "b_transposed"])
def test_bf16_fast_full_size_sampled_rows(hip, m, k, n, form):
    """The bench's bf16 products at full size under Fast (256x256 tiles for
    4096^3, 256x128 for [8192, 3072], k ranges for [3072, 768] over 8192),
    each operand form, checked on a sample of output rows against the oracle
    within the envelope plus one bf16 spacing, and repeated bit for bit."""
    banner(f"bf16 fast full size {m}x{k}x{n} {form}")
    a, b, a_view, b_view = _operands(m, k, n, form, seed=11)
    fast = _device(a_view, b_view, m, k, n, hip.FAST)
    assert np.array_equal(_device(a_view, b_view, m, k, n, hip.FAST), fast), "fast bf16 products repeat bit for bit"
    wb = oracle.bf16_widen(b).astype(np.float64)
    for r in sorted({0, 1, m // 3, m // 2 + 1, m - 2, m - 1}):
        want = oracle.gemm_bf16(a[r:r + 1], (k, 1), b, (n, 1), 1, k, n)[0]
        w = oracle.bf16_widen(want).astype(np.float64)
        wa = oracle.bf16_widen(a[r:r + 1]).astype(np.float64)
        bound = 1e-5 * (np.abs(wa) @ np.abs(wb))[0] + np.abs(w) * 2.0**-7 + 1e-38
        assert (np.abs(oracle.bf16_widen(fast[r]).astype(np.float64) - w) <= bound).all(), f"row {r}"
