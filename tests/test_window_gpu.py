"""Window programs on the device: Unfold as a strided view and Fold as one
kernel (src/function/{unfold,fold}.rs, src/payload/tensor.rs:1392-1462), and
the facades composed from them — conv2d (src/neural/convolution.rs:24-118),
max_pool (src/neural/pooling.rs:10-41) and BatchNorm by the batch's own
statistics (src/neural/batch_norm.rs:104-176) — the composed paths of the
WindowProduct, ReduceWindow and BatchNormTraining formulas
(src/backend/formula.rs:30-37). Under Exact every readable value equals the
oracle interpreter's bit for bit (src/engine/tests/plan_tests.rs:9-22); under
Fast the products meet the envelope."""
import numpy as np
import pytest

from poorgrad_amd import topos as t
from poorgrad_amd import workloads
from tests.conftest import banner
from tests.gpu_util import assert_bitwise
from tests.program_util import run_device, run_oracle

pytestmark = pytest.mark.gpu


def check(tape, roots, parameters, dense, numerics, selections=None):
    want = run_oracle(tape, roots, parameters, dense, selections)
    got, _ = run_device(tape, roots, parameters, dense, selections, numerics)
    return want, got


def pattern_values(count, multiplier, modulus, shift, scale):
    """The reference bench's deterministic fills (benches/pattern.rs:22-90):
    ((index * multiplier % modulus) - shift) / scale."""
    index = np.arange(count, dtype=np.int64)
    return (((index * multiplier) % modulus).astype(np.float32) - np.float32(shift)) / np.float32(scale)


@pytest.mark.parametrize("shape, axis, size, step, dilation", [
    ((37,), 0, 3, 2, 1),          # overlapping windows
    ((37,), 0, 2, 1, 3),          # dilated windows
    ((5, 29, 3), 1, 4, 5, 1),     # gaps between windows (step > size)
    ((4, 9, 6), 1, 9, 3, 1),      # a single window
    ((3, 20, 7), 1, 1, 2, 1),     # one-element windows
    ((2, 3, 11, 13), 3, 3, 2, 2), # dilation and step on the last axis
])
def test_unfold_then_fold_exact(hip, shape, axis, size, step, dilation):
    """A chain over the unfolded view, the fold of a function of it, and the
    fold of a permuted (non-contiguous) operand, all bitwise."""
    banner(f"window unfold/fold {shape} axis={axis} size={size} step={step} dilation={dilation}")
    tape = t.Tape()
    x = tape.input(shape)
    windows = x.unfold(axis, size, step, dilation)
    y = (windows * windows).exp() - windows
    folded = y.fold(axis, size, step, dilation, shape[axis])
    rank = len(windows.shape)
    order = list(range(rank))
    order[0], order[-1] = order[-1], order[0]
    # fold of a permuted view: permute back so the window pair sits at `axis`
    swapped = (y.permute(order) * y.permute(order)).permute(order)
    folded_view = swapped.fold(axis, size, step, dilation, shape[axis])
    values = np.random.default_rng(5).standard_normal(shape).astype(np.float32)
    want, got = check(tape, [y, folded, folded_view], [], {x.node.slot: values}, hip.EXACT)
    for r in (y, folded, folded_view):
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


def test_fold_keeps_signed_zeros_and_order(hip):
    banner("window fold signed zeros and order")
    tape = t.Tape()
    pair = tape.input((2, 2))
    terms = tape.input((3, 3))
    f = pair.fold(0, 2, 1, 1, 3)
    g = terms.fold(0, 3, 1, 1, 5)
    tv = np.zeros((3, 3), np.float32)
    tv[2, 0], tv[1, 1], tv[0, 2] = 1e8, -1e8, 1.0
    pv = np.array([[-0.0, -0.0], [-0.0, 5.0]], np.float32)
    want, got = check(tape, [f, g], [], {pair.node.slot: pv, terms.node.slot: tv}, hip.EXACT)
    assert_bitwise(got[f.id], want[f.id], "signed zeros")
    assert_bitwise(got[g.id], want[g.id], "ascending window-element order")
    assert got[g.id][2] == 1.0 and not np.signbit(got[f.id]).any()


@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_reference_bench_patterns(hip, posture):
    """The three composed patterns of the reference's pattern bench at their
    sizes: max_pool over [64,32,28,28], conv2d [64,16,14,14] x [32,16,3,3]
    padding 1, BatchNorm over [256,512]."""
    banner(f"window bench patterns {posture}")
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    tape = t.Tape()
    pool_in = tape.input((64, 32, 28, 28))
    pooled = t.max_pool(pool_in, 2, 2)
    conv_in = tape.input((64, 16, 14, 14))
    weights = tape.input((32, 16, 3, 3))
    bias = tape.leaf(t.Constant((32,), 0.01))
    features = t.conv2d(conv_in, weights, bias, 1, 1)
    norm_in = tape.input((256, 512))
    scale = tape.leaf(t.Constant((512,), 1.0))
    shift = tape.leaf(t.Constant((512,), 0.0))
    epsilon = tape.leaf(t.Constant((1,), 1e-5))
    normalized, mean, variance = t.batch_norm(norm_in, scale, shift, epsilon)
    dense = {
        pool_in.node.slot: pattern_values(64 * 32 * 28 * 28, 5, 13, 6.0, 4.0).reshape(64, 32, 28, 28),
        conv_in.node.slot: pattern_values(64 * 16 * 14 * 14, 7, 23, 11.0, 8.0).reshape(64, 16, 14, 14),
        weights.node.slot: pattern_values(32 * 16 * 9, 3, 17, 8.0, 16.0).reshape(32, 16, 3, 3),
        norm_in.node.slot: pattern_values(256 * 512, 11, 29, 14.0, 8.0).reshape(256, 512),
    }
    roots = [pooled, features, normalized, mean, variance]
    want, got = check(tape, roots, [], dense, numerics)
    for r in roots:
        if numerics == hip.EXACT or r is not features:
            assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")
        else:
            # the product's envelope, per output: 1e-5 * sum |a * b| over
            # the 144 terms of each filter's window
            e = want[r.id].astype(np.float64)
            assert np.abs(got[r.id].astype(np.float64) - e).max() <= 1e-5 * 144 * 1.375 * 0.5 + 1e-6


@pytest.mark.parametrize("model", ["cnn", "batch_norm_mlp"])
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_train_steps(hip, model, posture):
    """The MNIST convolutional step (examples/mnist/main.rs:59-99, batch 64)
    and the makemore BatchNorm step (examples/makemore/mlp_batchnorm.rs):
    loss and every gradient bitwise under Exact; within the envelope under
    Fast."""
    banner(f"window train step {model} {posture}")
    w = workloads.cnn() if model == "cnn" else workloads.batch_norm_mlp()
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    want, got = check(w.tape, w.roots, w.initial, w.dense_inputs, numerics, w.selection_inputs)
    if numerics == hip.EXACT:
        for r in w.roots:
            assert_bitwise(got[r.id], want[r.id], f"{model} node {r.id} {r.shape}")
        return
    loss_exact, loss_fast = want[w.loss.id].item(), got[w.loss.id].item()
    assert abs(loss_fast - loss_exact) <= 1e-4 * max(abs(loss_exact), 1.0)
    for r in w.gradients:
        g, e = got[r.id].astype(np.float64), want[r.id].astype(np.float64)
        scale = max(np.abs(e).max(), 1e-3)
        assert np.abs(g - e).max() <= 1e-3 * scale, f"{model} gradient {r.id} {r.shape}"


def test_cifar_shaped_step_exact(hip):
    """The CIFAR-10 example's three stages (examples/cifar10/main.rs:
    3 channels, 32x32, filters 16/32/64) at batch 8."""
    banner("window train step cifar-shaped exact")
    w = workloads.cnn(batch=8, channels=3, side=32, filters=(16, 32, 64))
    want, got = check(w.tape, w.roots, w.initial, w.dense_inputs, hip.EXACT, w.selection_inputs)
    for r in w.roots:
        assert_bitwise(got[r.id], want[r.id], f"cifar node {r.id} {r.shape}")
