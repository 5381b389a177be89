"""The host recorder (poorgrad_amd/topos.py) on the CPU: its recorded
gradients evaluated by the oracle interpreter against closed forms and
central finite differences (the reference's own gradient checks,
src/engine/tests/run_tests.rs:15-225), and the loss special cases of
src/neural/tests/loss_tests.rs."""
import math

import numpy as np
import pytest

from poorgrad_amd import topos as t
from poorgrad_amd import workloads
from tests.program_util import run_oracle


def evaluate(tape, roots, params, dense=None, selections=None):
    out = run_oracle(tape, roots, params, dense or {}, selections or {})
    return [out[r.id] for r in roots]


def test_gradient_of_a_product_sum_is_the_other_factor():
    # d/dw sum(w * x) = 0 + 1 * x: x itself, with -0 mapped to +0 by the zero seed.
    tape = t.Tape()
    w = tape.parameter((5,))
    x = tape.input((5,))
    loss = (w * x).sum()
    (grad,) = tape.differentiate(loss, [w])
    xs = np.array([1.5, -0.0, 0.0, -2.25, 3.0], np.float32)
    (g,) = evaluate(tape, [grad], [np.ones(5, np.float32)], {x.node.slot: xs})
    assert np.array_equal(g.view(np.uint32), (np.float32(0.0) + xs).view(np.uint32))
    assert g.view(np.uint32)[1] == 0  # +0


def test_non_ancestor_gradient_is_a_recorded_zero():
    tape = t.Tape()
    a = tape.parameter((2, 3))
    b = tape.parameter((4,))
    loss = a.sum()
    grad_a, grad_b = tape.differentiate(loss, [a, b])
    assert tape.nodes[grad_b.id].op == t.LEAF and tape.nodes[grad_b.id].payload.value == 0.0
    ga, gb = evaluate(tape, [grad_a, grad_b], [np.ones((2, 3), np.float32), np.ones(4, np.float32)])
    assert np.array_equal(ga, np.ones((2, 3), np.float32)) and np.array_equal(gb, np.zeros(4, np.float32))


def test_cross_entropy_of_uniform_logits_is_ln_classes():
    # src/neural/tests/loss_tests.rs:6-18
    tape = t.Tape()
    logits = tape.input((2, 3))
    targets = tape.selection_input(2, 3)
    loss = t.cross_entropy(logits, targets)
    (value,) = evaluate(tape, [loss], [], {logits.node.slot: np.zeros((2, 3), np.float32)},
                        {targets.node.slot: (np.array([0, 2], np.int32), 1.0)})
    assert abs(float(value.reshape(())) - math.log(3.0)) < 1e-6


def test_cross_entropy_of_a_certain_prediction_is_exactly_zero():
    # src/neural/tests/loss_tests.rs:100-132: the winner's log-probability is 0.
    tape = t.Tape()
    logits = tape.input((1, 3))
    targets = tape.selection_input(1, 3)
    loss = t.cross_entropy(logits, targets)
    (value,) = evaluate(tape, [loss], [], {logits.node.slot: np.array([[1000.0, 0.0, -1000.0]], np.float32)},
                        {targets.node.slot: (np.array([0], np.int32), 1.0)})
    assert float(value.reshape(())) == 0.0


def finite_difference_check(build, shapes, seed=0, eps=1e-2, tolerance=2e-2, positive=False):
    """Recorded gradients against central differences of the interpreter's
    loss, parameter by parameter, element by element (f32 arithmetic, so a
    loose tolerance; a wrong sign, term or transposed operand fails it)."""
    rng = np.random.default_rng(seed)
    params = [rng.uniform(0.5, 1.5, s).astype(np.float32) if positive else
              rng.standard_normal(s).astype(np.float32) for s in shapes]
    tape = t.Tape()
    values = [tape.parameter(s) for s in shapes]
    loss = build(tape, values)
    grads = tape.differentiate(loss, values)
    analytic = evaluate(tape, grads, params)
    for p_index, p in enumerate(params):
        for index in np.ndindex(*p.shape):
            bumped = [q.copy() for q in params]
            bumped[p_index][index] += np.float32(eps)
            (up,) = evaluate(tape, [loss], bumped)
            bumped[p_index][index] -= np.float32(2 * eps)
            (down,) = evaluate(tape, [loss], bumped)
            numeric = (float(np.ravel(up)[0]) - float(np.ravel(down)[0])) / (2 * eps)
            a = float(analytic[p_index][index])
            assert abs(a - numeric) <= tolerance * max(1.0, abs(numeric)), (p_index, index, a, numeric)


def test_elementwise_rules_match_finite_differences():
    # Parameters in [0.5, 1.5]: every kink of maximum/relu/abs stays more than
    # two steps away, while both sides of each are taken (central differences
    # straddling a kink average the two slopes).
    def build(tape, v):
        a, b = v
        one = a.one_like()
        y = (a * b).tanh() + (a / (b * b + one)).exp() - (a.abs() + one).ln()
        low = (a * tape.leaf(t.Constant(a.shape, 0.5))).maximum(b + one)     # right side wins
        high = (b + one).maximum(a - tape.leaf(t.Constant(a.shape, 2.0)))    # left side wins
        live = (a - b * tape.leaf(t.Constant(a.shape, 0.3))).relu()          # positive: slope 1
        dead = (b * tape.leaf(t.Constant(a.shape, 0.3)) - a - one).relu()     # negative: slope 0
        return (y.sqrt() * low * b - live * high + dead).sum()
    finite_difference_check(build, [(2, 3), (2, 3)], positive=True)


def test_matmul_and_log_softmax_rules_match_finite_differences():
    def build(tape, v):
        a, b, c = v
        logits = a.matmul(b.transpose()) + c.broadcast_along(0, a.matmul(b.transpose()))
        return (logits.log_softmax(1) * logits).sum() + logits.logsumexp(0).sum()
    finite_difference_check(build, [(3, 4), (5, 4), (5,)])


def test_layer_norm_and_cross_entropy_rules_match_finite_differences():
    def build(tape, v):
        x, scale, shift = v
        eps = tape.leaf(t.Constant((), 1e-5))
        h = t.layer_norm(x, scale, shift, eps)
        targets = tape.leaf(t.Selection(np.array([1, 0, 3], np.int32), 4))
        return t.cross_entropy(h, targets)
    finite_difference_check(build, [(3, 4), (4,), (4,)], tolerance=3e-2)


def test_view_and_index_rules_match_finite_differences():
    def build(tape, v):
        a, table = v
        sel = tape.leaf(t.Selection(np.array([2, 0, 2], np.int32), 3))
        rows = table.gather(sel)                                    # [3, 4]
        cat = t.concat([a.narrow(1, 0, 2), rows.narrow(1, 1, 2)], 1)  # [3, 4]
        batched = cat.reshape((3, 2, 2)).permute((1, 0, 2))         # [2, 3, 2]
        prod = batched.matmul(batched.permute((0, 2, 1)))           # [2, 3, 3]
        return (prod * prod).sum() + cat.sum().broadcast_like(a).sum_along(1).sum()
    finite_difference_check(build, [(3, 4), (3, 4)])


def test_window_rules_match_finite_differences():
    """Unfold's rule folds and Fold's rule unfolds (src/function/unfold.rs,
    src/function/fold.rs): checked through conv2d (padding, stride 2), a
    dilated unfold, a fold of a permuted view, and max_pool over distinct
    values (every window's maximum is strict)."""
    def build(tape, v):
        x, w, b, y = v
        conv = t.conv2d(x, w, b, 2, 1)                                        # [1, 2, 3, 3]
        dilated = y.unfold(1, 2, 1, 2)                                        # [2, 3, 2]
        folded = (dilated * dilated).permute((0, 2, 1)).permute((0, 2, 1)).fold(1, 2, 1, 2, 5)
        pooled = t.max_pool(x, 2, 2)                                           # [1, 1, 2, 2]
        return (conv * conv).sum() + (folded * y).sum() + (pooled * pooled).sum()
    finite_difference_check(build, [(1, 1, 5, 5), (2, 1, 3, 3), (2,), (2, 5)], eps=1e-3)


def test_log_softmax_backward_is_the_seed_minus_scaled_probabilities():
    """src/function/tests/log_softmax_tests.rs:44-66: with a one-hot seed the
    cotangent is onehot - softmax (f32 against the f64 closed form)."""
    tape = t.Tape()
    x = tape.parameter((2, 5))
    picked = tape.leaf(t.Dense(np.eye(5, dtype=np.float32)[[1, 3]]))
    loss = (x.log_softmax(1) * picked).sum()
    (g,) = tape.differentiate(loss, [x])
    values = np.array([[0.3, -1.2, 2.0, 0.0, 0.7], [-0.5, 0.25, 1.5, -2.0, 0.9]], np.float32)
    (got,) = evaluate(tape, [g], [values])
    e = np.exp(values.astype(np.float64) - values.max(1, keepdims=True))
    want = np.eye(5)[[1, 3]] - e / e.sum(1, keepdims=True)
    assert np.abs(got - want).max() < 1e-6


def test_cross_entropy_zero_target_lanes_contribute_exact_zero():
    """src/neural/tests/loss_tests.rs:136-147: a dense soft target with a zero
    lane against an extreme logit: exactly 0, never NaN."""
    tape = t.Tape()
    logits = tape.input((1, 2))
    targets = tape.input((1, 2))
    loss = t.cross_entropy(logits, targets)
    (value,) = evaluate(tape, [loss], [], {logits.node.slot: np.array([[-3.0e38, 3.0e38]], np.float32),
                                           targets.node.slot: np.array([[0.0, 1.0]], np.float32)})
    assert float(np.ravel(value)[0]) == 0.0 and not np.signbit(np.ravel(value)[0])


def test_adamw_decays_weights_and_spares_biases():
    """src/neural/tests/adam_tests.rs:79-143: the rank-1 bias is spared (AdamW
    equals Adam bit for bit there); a rank-2 weight differs from Adam by the
    decoupled term original * decay * rate (f32 rounding); decay 0 is Adam."""
    from tests.program_util import adamw_reference, adamw_state

    weights = np.array([[1.0, -0.5], [0.25, 2.0]], np.float32)
    bias = np.array([0.5, -1.0], np.float32)
    x = np.array([[1.0, -1.0]], np.float32)
    shifted = x @ weights + bias
    grads = [(x.T @ (2 * shifted)).astype(np.float32), (2 * shifted).sum(0).astype(np.float32)]
    plain = adamw_reference([weights, bias], grads, adamw_state([weights, bias]), rate=0.05, decay=0.0)
    decoupled = adamw_reference([weights, bias], grads, adamw_state([weights, bias]), rate=0.05, decay=0.1)
    assert plain[1].tobytes() == decoupled[1].tobytes()
    term = weights.astype(np.float64) * 0.1 * 0.05
    assert np.abs(plain[0].astype(np.float64) - decoupled[0] - term).max() < 1e-6
    assert np.abs(plain[0].astype(np.float64) - decoupled[0]).min() > 1e-4   # the decay is applied


def test_mlp_workload_loss_and_gradient_shapes():
    w = workloads.mlp()
    assert [g.shape for g in w.gradients] == [(784, 128), (128,), (128, 10), (10,)]
    out = run_oracle(w.tape, w.roots, w.initial, w.dense_inputs, w.selection_inputs)
    assert 1.5 < out[w.loss.id].item() < 3.5
    assert np.isfinite(out[w.gradients[0].id]).all()


def test_gpt2_workload_records_the_configured_graph():
    w = workloads.gpt2(batch=2, context=8, vocab=11, width=16, heads=2, layers=1, positions=8)
    ops = [n.op for n in w.tape.nodes]
    assert ops.count(t.GATHER) == 2 and ops.count(t.LOG_SOFTMAX) == 1 and ops.count(t.SCATTER) == 2
    assert len(w.gradients) == len(w.parameters) == 2 + 12 * 1 + 2
    out = run_oracle(w.tape, w.roots, w.initial, {}, w.selection_inputs)
    assert abs(out[w.loss.id].item() - math.log(11)) < 0.5


def test_synthetic_uniform_is_the_reference_stream():
    # init::uniform draws unit() through splitmix64 (src/neural/init.rs:88-91);
    # the oracle's generator is pinned to the reference's golden bits.
    import oracle

    got = workloads.uniform(7, 0.25, (1000,))
    want = oracle.Generator(7).uniform(1000, 0.25)
    assert np.array_equal(got, want)


def test_synthetic_normal_follows_the_reference_stream():
    # Box-Muller over consecutive draw pairs (init.rs:62-66, 93-102); numpy's
    # f64 log/cos may round differently in the last bit, so compare closely.
    import oracle

    got = workloads.normal(7, 0.02, (2000,))
    want = oracle.Generator(7).normal(2000, 0.02)
    assert np.mean(got == want) > 0.99
    assert np.allclose(got, want, rtol=1e-6, atol=1e-9)


def test_adamw_restatement_follows_the_paper_trace():
    """The f32 AdamW restatement the GPU tests hold the device kernel to,
    against the reference's two-step f64 paper trace
    (src/neural/tests/adam_tests.rs:15-53), with no decay as for its
    scalar-shaped parameter: within f32 rounding (1e-6 relative, about a
    dozen ulps of the result; the restatement lands 3.8e-7 away at step 2)
    at each step. A dropped bias correction moves step 1 by 24%, and swapped
    betas move step 2 by 7e-4."""
    from tests.program_util import adamw_reference, adamw_state, paper_adam_trace

    params = [np.ones((), np.float32)]
    state = adamw_state(params)
    trace = paper_adam_trace(2)
    for step in range(2):
        gradient = (np.float32(2) * params[0]).astype(np.float32)
        params = adamw_reference(params, [gradient], state, rate=0.1, decay=0.0)
        assert abs(float(params[0]) - trace[step]) <= 1e-6 * abs(trace[step]), (step, float(params[0]), trace[step])
    # The trace itself: after one step Adam moves w by the rate exactly
    # (m / c1 = g and sqrt(v / c2) = |g|), up to epsilon.
    assert abs(trace[0] - (1.0 - 0.1 * 2.0 / (2.0 + 1e-8))) < 1e-15
