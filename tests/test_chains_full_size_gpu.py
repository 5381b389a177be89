"""The chain config at its full size, [16384, 4096],
through the same entry points bench.py times (topos_hip_chain_launch for
SiLU + bias, topos_hip_layer_norm_f32_device, topos_hip_rows_f32_device),
every output element against the oracle:

* SiLU + bias, x / (exp(-x) + 1) + b (examples/llama/model.rs:258 with the
  bias of src/neural/linear.rs:94-105): bitwise (a chain has no posture);
* LayerNorm (src/neural/layer_norm.rs:100-132, epsilon 1e-5), row sum and row
  max (src/payload/tensor.rs:1073-1124), row softmax
  (src/function/log_softmax.rs:51-60 then exp): bitwise under Exact; under
  Fast the maximum stays bitwise and the reassociated sums hold the stated
  envelopes (a sum within 2 * columns * eps * sum|x| of the ordered one)."""
import numpy as np
import pytest

import oracle
from tests.conftest import banner
from tests.gpu_util import assert_bitwise

pytestmark = pytest.mark.gpu

ROWS, COLUMNS = 16384, 4096
EPS = 2.0**-24


@pytest.fixture(scope="module")
def operands(hip):
    import torch

    banner(f"chains full size: operands [{ROWS}, {COLUMNS}]")
    g = oracle.Generator(11)
    x = g.normal(ROWS * COLUMNS, 1.0).reshape(ROWS, COLUMNS)
    b = oracle.Generator(12).normal(COLUMNS, 1.0)
    scale = oracle.Generator(13).normal(COLUMNS, 1.0)
    dx = torch.from_numpy(x).cuda()
    return x, b, scale, dx, torch.from_numpy(b).cuda(), torch.from_numpy(scale).cuda()


def _rows(hip, kind, dx, numerics, full):
    import torch

    out = torch.empty((ROWS, COLUMNS) if full else (ROWS,), device="cuda")
    hip.checked(hip.lib.topos_hip_rows_f32_device(kind, dx.data_ptr(), ROWS, COLUMNS, numerics, out.data_ptr(),
                                                  torch.cuda.current_stream().cuda_stream), "rows")
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_full_size_silu_bias(hip, operands):
    import ctypes

    import torch

    from poorgrad_amd import device

    banner("chains full size: silu + bias")
    x, b, _, dx, db, _ = operands
    n = hip
    one = torch.ones(1, device="cuda")
    y = torch.empty_like(dx)
    chain = device.Chain((ROWS, COLUMNS), [((COLUMNS, 1), 0), ((0, 1), 0), ((0, 0), 0)],
                         [(n.CHAIN_NEG, -1, 0), (n.CHAIN_EXP, 0, 0), (n.CHAIN_ADD, 1, -3), (n.CHAIN_DIV, -1, 2),
                          (n.CHAIN_ADD, 3, -2)], [4])
    ins = (ctypes.c_void_p * 3)(dx.data_ptr(), db.data_ptr(), one.data_ptr())
    outs = (ctypes.c_void_p * 1)(y.data_ptr())
    n.checked(n.lib.topos_hip_chain_launch(chain._handle, ins, outs, torch.cuda.current_stream().cuda_stream),
              "silu chain")
    torch.cuda.synchronize()
    e = oracle.map_(oracle.EXP, oracle.map_(oracle.NEG, x))
    want = (x / (e + np.float32(1))) + b
    assert_bitwise(y.cpu().numpy(), want, "silu + bias [16384, 4096]")


@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_full_size_layer_norm(hip, operands, posture):
    import torch

    banner(f"chains full size: layer norm {posture}")
    x, b, scale, dx, db, dscale = operands
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    y = torch.empty_like(dx)
    hip.checked(hip.lib.topos_hip_layer_norm_f32_device(dx.data_ptr(), ROWS, COLUMNS, dscale.data_ptr(), db.data_ptr(),
                                                        1e-5, numerics, y.data_ptr(),
                                                        torch.cuda.current_stream().cuda_stream), "layer norm")
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = oracle.layer_norm_rows(x, scale, b, 1e-5)
    if posture == "exact":
        assert_bitwise(got, want, "layer norm [16384, 4096]")
    else:
        assert np.allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(scale).max())


@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_full_size_row_sum_and_max(hip, operands, posture):
    banner(f"chains full size: row sum and max {posture}")
    x, _, _, dx, _, _ = operands
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    biggest = _rows(hip, hip.ROWS_MAX, dx, numerics, False)
    assert_bitwise(biggest, oracle.max_along(x, 1), f"row max {posture}")
    total = _rows(hip, hip.ROWS_SUM, dx, numerics, False)
    want = oracle.sum_along(x, 1)
    if posture == "exact":
        assert_bitwise(total, want, "row sum exact")
    else:
        bound = 2 * COLUMNS * EPS * np.abs(x.astype(np.float64)).sum(axis=1)
        assert (np.abs(total.astype(np.float64) - want) <= bound).all()


@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_full_size_row_softmax_every_row(hip, operands, posture):
    banner(f"chains full size: row softmax {posture}")
    x, _, _, dx, _, _ = operands
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    got = _rows(hip, hip.ROWS_SOFTMAX, dx, numerics, True)
    want = oracle.softmax_rows(x)
    if posture == "exact":
        assert_bitwise(got, want, "row softmax [16384, 4096]")
    else:
        assert (np.abs(got.astype(np.float64) - want) <= 4 * COLUMNS * EPS * np.abs(want) + 1e-37).all()
