"""The composed formulas' dedicated device forms against the oracle
interpreter, over shapes beyond the reference's bench:

* WindowProduct (src/engine/pattern/window.rs:58-150,
  src/payload/tensor.rs:1475-1544): conv2d's im2col chain is never
  materialised; the forward product and the kernel gradient gather the patch
  matrix from the source (strides 1-3, padding 0-2, square and oblong
  kernels, a permuted source view);
* ReduceWindow (src/engine/pattern/reduce_window.rs): max_pool's lanes read
  the source through window views (one launch, the recorded lane order);
* BatchNormTraining (src/engine/pattern/batch_norm.rs): the statistics, the
  normalisation and the affine map as one column program.

Exact: every readable value bitwise. Fast: the forward window product and
every fold stay exact; the input gradient (a matrix-core product) and a
kernel gradient cut into ranges of whole images (each range an exact chain,
the partials added in range order) are held to the envelope
|c - exact| <= 1e-5 * sum |a| |b|, the bound computed by the oracle over the
operands' magnitudes."""
import numpy as np
import pytest

from poorgrad_amd import topos as t
from tests.conftest import banner
from tests.gpu_util import assert_bitwise
from tests.program_util import run_device, run_oracle

pytestmark = pytest.mark.gpu

# (batch, channels, height, width, filters, kernel_h, kernel_w, stride, padding, permuted source)
CONVS = [
    (2, 3, 9, 11, 4, 3, 3, 2, 0, False),
    (3, 2, 8, 8, 5, 3, 2, 1, 2, False),
    (2, 4, 7, 10, 3, 1, 1, 1, 0, True),
    (1, 3, 12, 12, 6, 5, 5, 3, 1, True),
    (4, 16, 14, 14, 32, 3, 3, 1, 1, False),
    # kernel gradients with few outputs over deep patch rows (the MNIST
    # stages at batch 16 and 8): under Fast, 16 and 2 ranges of images
    (16, 1, 28, 28, 8, 3, 3, 1, 1, False),
    (8, 8, 14, 14, 16, 3, 3, 1, 1, True),
]
# Ranges the Fast kernel gradient is cut into (window_splits), by case index.
FAST_RANGES = {5: 16, 6: 2}


def _conv_step(batch, channels, height, width, filters, kh, kw, stride, padding, permuted):
    tape = t.Tape()
    if permuted:  # the source is a transposed view of the input
        x = tape.input((batch, channels, width, height))
        source = x.permute([0, 1, 3, 2])
    else:
        x = tape.input((batch, channels, height, width))
        source = x
    w = tape.parameter((filters, channels, kh, kw))
    b = tape.parameter((filters,))
    y = t.conv2d(source, w, b, stride, padding)
    r = tape.input(y.shape)
    loss = (y * r).sum()
    gx, gw, gb = tape.differentiate(loss, [x, w, b])
    rng = np.random.default_rng(batch * 100 + channels * 10 + kh)
    params = [rng.standard_normal(w.shape).astype(np.float32), rng.standard_normal(b.shape).astype(np.float32)]
    dense = {x.node.slot: rng.standard_normal(x.shape).astype(np.float32),
             r.node.slot: rng.standard_normal(r.shape).astype(np.float32)}
    return tape, [y, loss, gx, gw, gb], params, dense


@pytest.mark.parametrize("index", range(len(CONVS)),
                         ids=lambda i: "x".join(map(str, CONVS[i][:9])) + ("p" if CONVS[i][9] else ""))
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_window_product_conv_step(hip, index, posture):
    case = CONVS[index]
    banner(f"window product conv {case} {posture}")
    tape, roots, params, dense = _conv_step(*case)
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    want = run_oracle(tape, roots, params, dense)
    got, program = run_device(tape, roots, params, dense, numerics=numerics)
    assert "gemm window patches " in program.describe and "gemm window patches^T" in program.describe
    assert "pad [" not in program.describe
    ranges = FAST_RANGES.get(index, 1) if numerics == hip.FAST else 1
    assert (f" in {ranges} ranges" in program.describe) == (ranges > 1), program.describe
    y, loss, gx, gw, gb = roots
    for r in (y, gb) if ranges > 1 else (y, gw, gb):
        assert_bitwise(got[r.id], want[r.id], f"{posture} node {r.id} {r.shape}")
    if numerics == hip.EXACT:
        assert_bitwise(got[loss.id], want[loss.id], "loss")
        assert_bitwise(got[gx.id], want[gx.id], "input gradient")
        return
    # The envelope of each product: the oracle's gradients over |x| and |r|
    # are sum |a| |b| for the kernel gradient (patches^T . |r|) and the input
    # gradient (|r| . |kernel|^T folded back, a sum of the same magnitudes).
    magnitude = {slot: np.abs(a) for slot, a in dense.items()}
    bound = run_oracle(tape, roots, [np.abs(params[0]), params[1]], magnitude)
    for r in (gx, gw) if ranges > 1 else (gx,):
        error = np.abs(got[r.id].astype(np.float64) - want[r.id].astype(np.float64))
        limit = 1e-5 * bound[r.id].astype(np.float64)
        assert (error <= limit).all(), f"{posture} node {r.id}: max error {error.max()} over limit"
    if ranges > 1:  # deterministic: the ranges are added in a fixed order
        again, _ = run_device(tape, roots, params, dense, numerics=numerics)
        assert_bitwise(again[gw.id], got[gw.id], "repeat of the ranged kernel gradient")


@pytest.mark.parametrize("size, stride", [(2, 2), (3, 2), (3, 1), (2, 3)])
def test_reduce_window_reads_the_source(hip, size, stride):
    """max_pool with overlapping (stride < size) and gapped (stride > size)
    windows, ties and signed zeros included, with its gradient: bitwise, and
    no lane copy."""
    banner(f"reduce window size {size} stride {stride}")
    tape = t.Tape()
    x = tape.input((3, 4, 11, 13))
    pooled = t.max_pool(x, size, stride)
    r = tape.input(pooled.shape)
    loss = (pooled * r).sum()
    (gx,) = tape.differentiate(loss, [x])
    rng = np.random.default_rng(size * 10 + stride)
    values = rng.integers(-3, 4, x.shape).astype(np.float32)  # many ties
    values[0, 0, :2, :] = -0.0
    dense = {x.node.slot: values, r.node.slot: rng.standard_normal(r.shape).astype(np.float32)}
    want = run_oracle(tape, [pooled, gx], [], dense)
    got, program = run_device(tape, [pooled, gx], [], dense)
    assert "copy [" not in program.describe
    for v in (pooled, gx):
        assert_bitwise(got[v.id], want[v.id], f"node {v.id} {v.shape}")


@pytest.mark.parametrize("rows, features", [(256, 512), (64, 100), (7, 33), (1024, 48)])
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_batch_norm_is_one_column_program(hip, rows, features, posture):
    """BatchNorm's statistics and output (src/neural/batch_norm.rs:149-176)
    in one launch, and its training gradients, bitwise in both postures
    (no product is involved)."""
    banner(f"batch norm column program {rows}x{features} {posture}")
    tape = t.Tape()
    x = tape.input((rows, features))
    scale, shift = tape.parameter((features,)), tape.parameter((features,))
    epsilon = tape.leaf(t.Constant((), 1e-5))
    out, mean, variance = t.batch_norm(x, scale, shift, epsilon)
    r = tape.input(out.shape)
    loss = (out * r).sum()
    gx, gs, gb = tape.differentiate(loss, [x, scale, shift])
    rng = np.random.default_rng(rows + features)
    params = [rng.standard_normal(features).astype(np.float32), rng.standard_normal(features).astype(np.float32)]
    dense = {x.node.slot: (3 * rng.standard_normal((rows, features)) + 1).astype(np.float32),
             r.node.slot: rng.standard_normal((rows, features)).astype(np.float32)}
    roots = [out, mean, variance, gx, gs, gb]
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    want = run_oracle(tape, roots, params, dense)
    got, program = run_device(tape, roots, params, dense, numerics=numerics)
    assert program.describe.count("columns [") >= 1
    for v in roots:
        assert_bitwise(got[v.id], want[v.id], f"{posture} node {v.id} {v.shape}")
