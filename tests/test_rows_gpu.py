"""Row reductions and fused rules on the GPU against the oracle:
bit-identical in the exact posture (ascending, first-term seeded), within a
stated envelope in the fast posture."""
import numpy as np
import pytest
import torch

import oracle
from poorgrad_amd import device
from tests.conftest import banner
from tests.gpu_util import assert_bitwise, to_device

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 5), (64, 10), (65, 129), (257, 1000), (128, 4096), (63, 4099), (2, 50257)]


def sample(rows, columns, seed):
    return oracle.Generator(seed).normal(rows * columns, 3.0).reshape(rows, columns)


def expected_rows(kind, x):
    from poorgrad_amd import _native as n

    if kind == n.ROWS_SUM:
        return oracle.sum_along(x, 1)
    if kind == n.ROWS_MAX:
        return oracle.max_along(x, 1)
    if kind == n.ROWS_LOG_SOFTMAX:
        return oracle.log_softmax_rows(x)
    if kind == n.ROWS_SOFTMAX:
        return oracle.softmax_rows(x)
    return oracle.log_sum_exp_rows(x)


KINDS = ["sum", "max", "log_softmax", "softmax", "log_sum_exp"]


def kind_code(name):
    from poorgrad_amd import _native as n

    return {"sum": n.ROWS_SUM, "max": n.ROWS_MAX, "log_softmax": n.ROWS_LOG_SOFTMAX,
            "softmax": n.ROWS_SOFTMAX, "log_sum_exp": n.ROWS_LOG_SUM_EXP}[name]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows, columns", SHAPES)
def test_exact_rows_bit_identical(hip, kind, rows, columns):
    banner(f"exact rows {kind} {rows}x{columns}")
    x = sample(rows, columns, rows * 31 + columns)
    got = device.rows(kind_code(kind), to_device(x), hip.EXACT)
    torch.cuda.synchronize()
    assert_bitwise(got, expected_rows(kind_code(kind), x), f"{kind} {rows}x{columns}")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows, columns", SHAPES)
def test_fast_rows_within_envelope(hip, kind, rows, columns):
    banner(f"fast rows {kind} {rows}x{columns}")
    x = sample(rows, columns, rows * 17 + columns)
    got = device.rows(kind_code(kind), to_device(x), hip.FAST).cpu().numpy().astype(np.float64)
    want = expected_rows(kind_code(kind), x).astype(np.float64)
    if kind == "max":
        assert_bitwise(got.astype(np.float32), want.astype(np.float32), "fast max")
        return
    # Reassociated sums: a sum's error is bounded by 2 * columns * eps * sum|x|;
    # a log-sum's by 2 * columns * eps absolutely (the relative error of the
    # sum), and softmax's relatively.
    eps = 2.0**-24
    if kind == "sum":
        bound = 2 * columns * eps * np.abs(x.astype(np.float64)).sum(axis=1)
        assert (np.abs(got - want) <= bound + 1e-30).all()
    elif kind == "softmax":
        assert (np.abs(got - want) <= 4 * columns * eps * np.abs(want) + 1e-37).all()
    else:
        assert (np.abs(got - want) <= 4 * columns * eps * (1 + np.abs(want))).all()


def test_exact_rows_special_values(hip):
    banner("exact rows special values")
    x = np.array([[-0.0, -0.0, -0.0, -0.0],
                  [0.0, -0.0, 0.0, -0.0],
                  [np.nan, 1.0, 2.0, np.nan],
                  [np.inf, 1.0, -np.inf, 0.0],
                  [-np.inf, -np.inf, -np.inf, -np.inf],
                  [1e38, 1e38, 1e38, -1e38]], dtype=np.float32)
    for kind in KINDS:
        got = device.rows(kind_code(kind), to_device(x), hip.EXACT)
        torch.cuda.synchronize()
        assert_bitwise(got, expected_rows(kind_code(kind), x), f"special {kind}")


@pytest.mark.parametrize("columns", [8, 1024])
def test_fast_rows_special_values(hip, columns):
    """The fast posture on rows with NaN, infinities and signed zeros (the
    register-resident kernel at 1024 columns, the streaming one at 8): the
    maximum is bitwise the ordered max_f32 fold, and every other reduction
    puts NaN and infinities where the interpreter does."""
    banner(f"fast rows special values {columns}")
    x = np.full((6, columns), 0.5, dtype=np.float32)
    x[0, :] = -0.0
    x[1, 0], x[1, -1] = np.nan, np.nan
    x[2, 1], x[2, -2] = np.inf, -np.inf
    x[3, :] = -np.inf
    x[4, 3] = 1e38; x[4, 4] = 1e38
    x[5, :] = np.nan
    for kind in KINDS:
        got = device.rows(kind_code(kind), to_device(x), hip.FAST).cpu().numpy()
        want = expected_rows(kind_code(kind), x)
        if kind == "max":
            assert_bitwise(got, want, f"fast special {kind}")
            continue
        assert np.array_equal(np.isnan(got), np.isnan(want)), f"fast special {kind}: NaN positions"
        finite = ~np.isnan(want)
        assert np.array_equal(np.isinf(got[finite]), np.isinf(want[finite])), f"fast special {kind}: infinities"
        inf = np.isinf(want) & finite
        assert np.array_equal(np.sign(got[inf]), np.sign(want[inf])), f"fast special {kind}: infinity signs"


@pytest.mark.parametrize("columns", [1024, 4096])
def test_row_max_signed_zero_ties_and_nan_payloads(hip, columns):
    """The ordered max_f32 fold keeps the earlier of two tied signed zeros
    and, over a row of NaNs only, ends on the last term. Rows wide enough to
    spread over every lane and quad of the register-resident kernel put the
    competing zeros in other lanes and quads than column 0; the NaN rows
    carry a distinct payload per column, compared by raw bits."""
    banner(f"row max ties {columns}")
    from poorgrad_amd import _native as n

    x = np.full((8, columns), -1.0, dtype=np.float32)
    x[0, 0] = -0.0; x[0, [1, 5, 67, columns // 2, columns - 1]] = 0.0    # -0 first, +0 in other lanes
    x[1, 0] = 0.0; x[1, [1, 5, 67, columns // 2, columns - 1]] = -0.0    # +0 first, -0 elsewhere
    x[2, 300] = -0.0; x[2, [4, 260, columns - 3]] = 0.0                   # +0 earlier in another quad
    x[3, 4] = -0.0; x[3, [260, columns - 3]] = 0.0                        # -0 in quad 1, +0 later
    nan_bits = (np.uint32(0x7FC00000) | np.arange(1, columns + 1, dtype=np.uint32))
    x[4] = nan_bits.view(np.float32)                                       # every term a distinct quiet NaN
    x[5] = (nan_bits | np.uint32(0x80000000)).view(np.float32)             # negative NaN payloads
    x[6] = nan_bits.view(np.float32); x[6, columns // 3] = -0.0           # one number among NaNs
    x[7, :] = -0.0; x[7, columns - 1] = 0.0
    want = oracle.max_along(x, 1)
    for numerics in (hip.EXACT, hip.FAST):
        got = device.rows(n.ROWS_MAX, to_device(x), numerics).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (
            f"posture {numerics}: {got.view(np.uint32)} vs {want.view(np.uint32)}")
    # The oracle's own fold fixes the answers these rows are built around.
    assert want.view(np.uint32)[0] == np.float32(-0.0).view(np.uint32)
    assert want.view(np.uint32)[1] == np.float32(0.0).view(np.uint32)
    assert want.view(np.uint32)[4] == nan_bits[-1]
    assert want.view(np.uint32)[6] == np.float32(-0.0).view(np.uint32)


@pytest.mark.parametrize("rows, columns", [(3, 5), (64, 768), (257, 1000), (96, 4096)])
def test_layer_norm_exact_and_fast(hip, rows, columns):
    banner(f"layer norm {rows}x{columns}")
    g = oracle.Generator(rows + columns)
    x = g.normal(rows * columns, 1.0).reshape(rows, columns)
    scale, shift = g.normal(columns, 1.0), g.normal(columns, 1.0)
    want = oracle.layer_norm_rows(x, scale, shift, 1e-5)
    got = device.layer_norm(to_device(x), to_device(scale), to_device(shift), 1e-5, hip.EXACT)
    torch.cuda.synchronize()
    assert_bitwise(got, want, "exact layer norm")
    fast = device.layer_norm(to_device(x), to_device(scale), to_device(shift), 1e-5, hip.FAST).cpu().numpy()
    assert np.allclose(fast, want, rtol=1e-4, atol=1e-4 * np.abs(scale).max())


def test_full_size_row_softmax_sampled(hip):
    """The chain config's [16384, 4096] row softmax: sampled rows against the
    oracle, and every row a probability vector."""
    banner("row softmax 16384x4096 sampled")
    x = torch.randn(16384, 4096, generator=torch.Generator().manual_seed(11)).cuda()
    for numerics in (hip.EXACT, hip.FAST):
        out = device.rows(kind_code("softmax"), x, numerics)
        torch.cuda.synchronize()
        picks = [0, 1, 4095, 8191, 16382, 16383]
        host = x[picks].cpu().numpy()
        want = oracle.softmax_rows(host)
        if numerics == hip.EXACT:
            assert_bitwise(out[picks], want, "row softmax sample")
        else:
            assert np.allclose(out[picks].cpu().numpy(), want, rtol=1e-5, atol=1e-9)
        sums = out.sum(dim=1, dtype=torch.float64)
        assert torch.allclose(sums, torch.ones_like(sums), atol=1e-4)
