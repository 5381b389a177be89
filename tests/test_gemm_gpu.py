"""GEMM parity on the GPU against the oracle's gemm::multiply
(src/payload/gemm.rs:140-211): bit-identical in the exact posture, within
|c - exact| <= 1e-5 * sum_k |a_ik b_kj| in the fast (MFMA) posture, across the
reference's shape grid (src/backend/cuda/tests/cuda_tests.rs:153-161) and
stride forms (contiguous, transposed A, transposed B, narrowed window,
stride-0 broadcast)."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import banner
from tests.gpu_util import assert_bitwise, to_device

pytestmark = pytest.mark.gpu

SHAPES = [(2, 3, 4), (5, 8, 13), (16, 16, 16), (63, 64, 65), (100, 127, 3), (128, 100, 64), (2, 64, 128),
          (129, 257, 131), (256, 384, 512), (257, 131, 61)]
FORMS = ["contiguous", "a_transposed", "b_transposed", "both_transposed", "narrowed", "broadcast"]


def operands(m, k, n, form, seed):
    """Flat buffers plus (strides, offset) per operand realising the logical
    m x k and k x n matrices in the given stride form."""
    g = oracle.Generator(seed)
    a_logical = g.normal(m * k, 1.0).reshape(m, k)
    b_logical = g.normal(k * n, 1.0).reshape(k, n)
    if form == "broadcast":
        b_logical = np.repeat(b_logical[:1], k, axis=0)  # every row the same: stride 0
    a_buf, a_st, a_off = a_logical.ravel(), (k, 1), 0
    b_buf, b_st, b_off = b_logical.ravel(), (n, 1), 0
    if form in ("a_transposed", "both_transposed"):
        a_buf, a_st = np.ascontiguousarray(a_logical.T).ravel(), (1, m)
    if form in ("b_transposed", "both_transposed"):
        b_buf, b_st = np.ascontiguousarray(b_logical.T).ravel(), (1, k)
    if form == "narrowed":
        wide = np.full((m, k + 5), np.nan, dtype=np.float32)
        wide[:, 3:3 + k] = a_logical
        a_buf, a_st, a_off = wide.ravel(), (k + 5, 1), 3
    if form == "broadcast":
        b_buf, b_st = b_logical[0].copy(), (0, 1)
    return a_logical, b_logical, (a_buf, a_st, a_off), (b_buf, b_st, b_off)


def run_device(a, b, m, k, n, numerics):
    from poorgrad_amd import _native as nat

    (a_buf, a_st, a_off), (b_buf, b_st, b_off) = a, b
    da, db = to_device(a_buf), to_device(b_buf)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    nat.checked(nat.lib.topos_hip_gemm_f32_device(da.data_ptr() + 4 * a_off, a_st[0], a_st[1],
                                                  db.data_ptr() + 4 * b_off, b_st[0], b_st[1], m, k, n, numerics,
                                                  out.data_ptr(), n, torch.cuda.current_stream().cuda_stream),
                "gemm")
    torch.cuda.synchronize()
    return out.cpu().numpy()


def envelope(a_logical, b_logical):
    return 1e-5 * (np.abs(a_logical.astype(np.float64)) @ np.abs(b_logical.astype(np.float64)))


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("m, k, n", SHAPES)
def test_exact_gemm_is_bit_identical(hip, m, k, n, form):
    banner(f"exact gemm {m}x{k}x{n} {form}")
    a_l, b_l, a, b = operands(m, k, n, form, seed=m + 7 * k + 13 * n)
    expected = oracle.gemm(a_l, (k, 1), b_l, (n, 1), m, k, n)
    got = run_device(a, b, m, k, n, hip.EXACT)
    assert_bitwise(got, expected, f"exact {m}x{k}x{n} {form}")


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("m, k, n", SHAPES)
def test_fast_gemm_within_envelope_and_deterministic(hip, m, k, n, form):
    banner(f"fast gemm {m}x{k}x{n} {form}")
    a_l, b_l, a, b = operands(m, k, n, form, seed=3 * m + k + n)
    exact = oracle.gemm(a_l, (k, 1), b_l, (n, 1), m, k, n)
    got = run_device(a, b, m, k, n, hip.FAST)
    error = np.abs(got.astype(np.float64) - exact.astype(np.float64))
    assert (error <= envelope(a_l, b_l)).all(), f"max error {error.max()}"
    again = run_device(a, b, m, k, n, hip.FAST)
    assert_bitwise(again, got, "fast gemm repeat")


def test_negative_zero_seed_survives_on_device(hip):
    banner("exact gemm -0.0 seed")
    a = (np.array([-0.0, 0.0], np.float32), (2, 1), 0)
    b = (np.array([0.0, -0.0], np.float32), (1, 1), 0)
    got = run_device(a, b, 1, 2, 1, hip.EXACT)
    assert got.view(np.uint32)[0, 0] == np.float32(-0.0).view(np.uint32)


@pytest.mark.parametrize("m, k, n", [(1024, 1024, 4096), (512, 512, 512), (4096, 4096, 4096), (8192, 3072, 768),
                                     (768, 8192, 768), (768, 4096, 20001),
                                     (1025, 1027, 1029), (1000, 512, 1020), (300, 64, 260),
                                     # fast tile choices: 64x128 tiles filling whole rounds (k <= 1024),
                                     # unsplit with a tile per CU, two k ranges
                                     (8192, 768, 768), (8192, 768, 2304), (4096, 2048, 2048),
                                     (2048, 4096, 2048),
                                     # 128x64 tiles (an output 64 or fewer wide), whole and ragged
                                     (1024, 1024, 64), (1000, 300, 62),
                                     # 256x256 tiles (four rounds or more), whole and a ragged vocabulary
                                     (8192, 256, 8192), (2048, 192, 50257)])
@pytest.mark.parametrize("product", ["forward", "a_transposed", "b_transposed"])
def test_sweep_shapes_sampled_rows(hip, m, k, n, product):
    """The GEMM-sweep products at full size (forward A.B, then A^T.G and
    G.B^T as transposed views), checked on a sample of output rows against
    the oracle: exact bitwise, fast within the envelope."""
    banner(f"sweep {product} {m}x{k}x{n}")
    g = oracle.Generator(7)
    a_logical = g.normal(m * k, 1.0).reshape(m, k)
    b_logical = g.normal(k * n, 1.0).reshape(k, n)
    a_buf, a_st = a_logical.ravel(), (k, 1)
    b_buf, b_st = b_logical.ravel(), (n, 1)
    if product == "a_transposed":
        a_buf, a_st = np.ascontiguousarray(a_logical.T).ravel(), (1, m)
    if product == "b_transposed":
        b_buf, b_st = np.ascontiguousarray(b_logical.T).ravel(), (1, k)
    rows = np.array(sorted({0, 1, m // 3, m // 2 + 1, m - 2, m - 1}))
    for numerics in (hip.EXACT, hip.FAST):
        got = run_device((a_buf, a_st, 0), (b_buf, b_st, 0), m, k, n, numerics)
        if numerics == hip.FAST:  # split along k or not: the same bits every run
            assert_bitwise(run_device((a_buf, a_st, 0), (b_buf, b_st, 0), m, k, n, numerics), got, "repeat")
        for r in rows:
            expected = oracle.gemm(a_logical[r:r + 1], (k, 1), b_logical, (n, 1), 1, k, n)[0]
            if numerics == hip.EXACT:
                assert_bitwise(got[r], expected, f"row {r}")
            else:
                bound = envelope(a_logical[r:r + 1], b_logical)[0]
                assert (np.abs(got[r].astype(np.float64) - expected) <= bound).all()
