"""Device programs against the topos interpreter (oracle/interpreter.py) on
the same recorded graphs and inputs: every readable value bit-identical in
the exact posture (src/engine/tests/plan_tests.rs:9-22, :83-131 — plan equals
interpreter bitwise), and within the stated envelope in the fast posture
(plan_tests.rs:542-592)."""
import math

import numpy as np
import oracle
import pytest

from poorgrad_amd import topos as t
from poorgrad_amd import workloads
from tests.conftest import banner
from tests.gpu_util import assert_bitwise
from tests.program_util import adamw_reference, adamw_state, paper_adam_trace, run_device, run_oracle

pytestmark = pytest.mark.gpu


def check_workload(w, numerics, hip):
    want = run_oracle(w.tape, w.roots, w.initial, w.dense_inputs, w.selection_inputs)
    got, program = run_device(w.tape, w.roots, w.initial, w.dense_inputs, w.selection_inputs, numerics)
    return want, got, program


def test_mlp_train_step_exact_is_bit_identical(hip):
    """BASELINE configs[0] at its full size: loss and all four gradients."""
    banner("program mlp exact")
    w = workloads.mlp()
    want, got, program = check_workload(w, hip.EXACT, hip)
    for r in w.roots:
        assert_bitwise(got[r.id], want[r.id], f"mlp node {r.id}")
    assert abs(want[w.loss.id].item() - math.log(10)) < 0.5


def test_mlp_train_step_fast_within_envelope(hip):
    banner("program mlp fast")
    w = workloads.mlp()
    want, got, _ = check_workload(w, hip.FAST, hip)
    # plan_tests.rs:583-590: |fast - exact| <= 1e-4 * max(|exact|, 1)
    for r in w.roots:
        g, e = got[r.id].astype(np.float64), want[r.id].astype(np.float64)
        assert (np.abs(g - e) <= 1e-4 * np.maximum(np.abs(e), 1.0)).all(), f"node {r.id}"


@pytest.mark.parametrize("layers, heads", [(1, 2), (2, 4)])
def test_small_gpt2_train_step_exact_is_bit_identical(hip, layers, heads):
    """The GPT-2 graph (batched causal attention, LayerNorm, GELU, tied
    embeddings, cross-entropy, recorded gradients) at a small size."""
    banner(f"program gpt2 small layers={layers}")
    w = workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=heads, layers=layers, positions=24)
    want, got, _ = check_workload(w, hip.EXACT, hip)
    for r in w.roots:
        assert_bitwise(got[r.id], want[r.id], f"gpt2 node {r.id} {r.shape}")


@pytest.mark.parametrize("shape", [(2, 3, 64, 128), (1, 2, 128, 64), (3, 1, 64, 192)])
def test_transposed_view_copied_in_tiles_is_exact(hip, shape):
    """A reshape of a permuted view whose innermost axis steps through the
    input while another axis is contiguous (the key gradient of attention
    read through the head permutation) is copied in 64 x 64 LDS tiles: the
    same bits as the transposition itself, in both postures."""
    B, H, D, T = shape
    banner(f"program tiled transposing copy {shape}")
    rng = np.random.default_rng(61)
    tape = t.Tape()
    x = tape.input((B, H, D, T))
    y = x.permute((0, 3, 1, 2)).reshape((B * T, H * D))
    dense = {x.node.slot: rng.standard_normal((B, H, D, T)).astype(np.float32)}
    want = np.ascontiguousarray(dense[x.node.slot].transpose(0, 3, 1, 2)).reshape(B * T, H * D)
    for posture in (hip.EXACT, hip.FAST):
        got, program = run_device(tape, [y], [], dense, numerics=posture)
        assert "copy (tiles)" in program.describe, program.describe
        assert_bitwise(got[y.id], want, f"copy {shape}")


def test_gpt2_with_tiled_head_copies_fast_within_envelope(hip):
    """Context and head width multiples of 64: under Fast the key gradient,
    read through the head permutation, is copied in 64 x 64 LDS tiles (the
    plan names it `copy (tiles)`). Loss and gradients within the envelope."""
    banner("program gpt2 tiled head copies fast")
    w = workloads.gpt2(batch=2, context=64, vocab=61, width=128, heads=2, layers=1, positions=64)
    want, got, program = check_workload(w, hip.FAST, hip)
    assert "copy (tiles)" in program.describe
    loss_exact, loss_fast = want[w.loss.id].item(), got[w.loss.id].item()
    assert abs(loss_fast - loss_exact) <= 1e-4 * max(abs(loss_exact), 1.0)
    for r in w.gradients:
        g, e = got[r.id].astype(np.float64), want[r.id].astype(np.float64)
        scale = max(np.abs(e).max(), 1e-3)
        assert np.abs(g - e).max() <= 1e-3 * scale, f"gradient {r.id} {r.shape}"


def test_small_gpt2_fast_within_envelope(hip):
    banner("program gpt2 small fast")
    w = workloads.gpt2(batch=2, context=32, vocab=61, width=64, heads=4, layers=2, positions=32)
    want, got, _ = check_workload(w, hip.FAST, hip)
    loss_exact, loss_fast = want[w.loss.id].item(), got[w.loss.id].item()
    assert abs(loss_fast - loss_exact) <= 1e-4 * max(abs(loss_exact), 1.0)
    for r in w.gradients:
        g, e = got[r.id].astype(np.float64), want[r.id].astype(np.float64)
        scale = max(np.abs(e).max(), 1e-3)
        assert np.abs(g - e).max() <= 1e-3 * scale, f"gradient {r.id} {r.shape}"


@pytest.mark.parametrize("layers, heads", [(1, 2), (2, 4)])
def test_small_llama_exact_is_bit_identical(hip, layers, heads):
    """The Llama-style decoder (RMSNorm, rotary embeddings rotated by
    narrow/neg/concat, causal attention, SwiGLU, untied head) at a small size:
    the loss and every gradient bit-identical."""
    banner(f"program llama small layers={layers}")
    w = workloads.llama(batch=2, context=16, vocab=37, width=32, heads=heads, hidden=48, layers=layers)
    want, got, _ = check_workload(w, hip.EXACT, hip)
    for r in w.roots:
        assert_bitwise(got[r.id], want[r.id], f"llama node {r.id} {r.shape}")


def test_small_llama_fast_within_envelope(hip):
    banner("program llama small fast")
    w = workloads.llama(batch=2, context=32, vocab=61, width=64, heads=4, hidden=96, layers=2)
    want, got, _ = check_workload(w, hip.FAST, hip)
    loss_exact, loss_fast = want[w.loss.id].item(), got[w.loss.id].item()
    assert abs(loss_fast - loss_exact) <= 1e-4 * max(abs(loss_exact), 1.0)
    for r in w.gradients:
        g, e = got[r.id].astype(np.float64), want[r.id].astype(np.float64)
        scale = max(np.abs(e).max(), 1e-3)
        assert np.abs(g - e).max() <= 1e-3 * scale, f"gradient {r.id} {r.shape}"


@pytest.mark.parametrize("numerics", ["exact", "fast"])
def test_graph_replay_matches_eager_runs(hip, numerics):
    """A run replayed from a captured HIP graph (main and side streams) equals
    the eager run bitwise: three replays with eager runs, torch work and
    synchronizations between them; then a rebind to new parameter values,
    which recaptures."""
    import torch

    from poorgrad_amd.program import DeviceProgram

    banner(f"program graph replay {numerics}")
    posture = hip.EXACT if numerics == "exact" else hip.FAST
    w = workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24)
    program = DeviceProgram(w.tape, w.roots, numerics=posture)
    params = [torch.from_numpy(a).cuda() for a in w.initial]
    for slot, t_ in enumerate(params):
        program.bind_parameter(slot, t_)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    program.run()
    torch.cuda.synchronize()
    want = {r.id: program.read(r) for r in w.roots}
    for replay in range(3):
        program.replay()
        torch.cuda.synchronize()
        for r in w.roots:
            assert_bitwise(program.read(r), want[r.id], f"replay {replay} node {r.id}")
        program.run()
        noise = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
    moved = [p_ * 1.5 for p_ in params]
    for slot, t_ in enumerate(moved):
        program.bind_parameter(slot, t_)
    program.run()
    torch.cuda.synchronize()
    want = {r.id: program.read(r) for r in w.roots}
    for replay in range(2):
        program.replay()
        torch.cuda.synchronize()
        for r in w.roots:
            assert_bitwise(program.read(r), want[r.id], f"rebound replay {replay} node {r.id}")


def coverage_graph():
    """One graph touching every served variant and storage kind."""
    rng = np.random.default_rng(5)
    tape = t.Tape()
    a = tape.parameter((6, 8))
    b = tape.parameter((8, 5))
    c = tape.parameter((4, 6, 8))
    table = tape.parameter((9, 8))
    x = tape.input((6, 8))
    sel = tape.selection_input(6, 9)
    leaf = tape.leaf(t.Dense(rng.standard_normal((6, 5)).astype(np.float32)))
    two = tape.leaf(t.Constant((), 2.0))
    roots = []
    y = (a * x + x.exp()).tanh() - (a / (x.abs() + two.broadcast_like(x))).sqrt()
    roots.append(y)
    p = y.matmul(b) + leaf
    roots.append(p.log_softmax(0))
    roots.append(p.log_softmax(1))
    roots.append(p.logsumexp(0))
    roots.append(p.logsumexp(1))
    roots.append(p.sum())
    roots.append(p.sum_along(0))
    roots.append(p.transpose())  # a readable view
    cat = t.concat([a.narrow(1, 0, 3), x.narrow(1, 3, 5)], 1)
    roots.append(cat.maximum(y).relu() + cat.step(y))
    roots.append(c.permute((1, 0, 2)).reshape((6, 32)))  # a reshape that copies
    roots.append(c.reshape((24, 8)).sum_along(0))  # a reshape that views
    roots.append(c.matmul(c.permute((0, 2, 1))))  # batched, transposed right operand
    roots.append(c.log_softmax(1).sum_along(2))
    g = table.gather(sel)
    roots.append(g)
    roots.append((g * x).scatter(sel, 9))
    onehot_sum = (tape.value(sel.id) * g.matmul(table.transpose())).sum()
    roots.append(onehot_sum)
    roots.append(tape.value(sel.id).sum_along(1))
    roots.append(two * two + two)  # a host-known constant, readable
    roots.append(p.sum().broadcast_like(p) * p)
    loss = (p * p).sum() + onehot_sum
    grads = tape.differentiate(loss, [a, b, c, table])
    roots += grads
    params = [rng.standard_normal(s).astype(np.float32) for s in tape.parameter_shapes]
    dense = {x.node.slot: rng.standard_normal((6, 8)).astype(np.float32)}
    selections = {sel.node.slot: (np.array([3, 0, 3, 8, 1, 3], np.int32), 1.0)}
    return tape, roots, params, dense, selections


def test_every_served_variant_exact(hip):
    banner("program coverage graph exact")
    tape, roots, params, dense, selections = coverage_graph()
    want = run_oracle(tape, roots, params, dense, selections)
    got, program = run_device(tape, roots, params, dense, selections, hip.EXACT)
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} ({t.NAMES[r.node.op]} {r.shape})")


def test_signed_zero_seeding_survives(hip):
    """Gradient accumulation starts from a Constant zero: 0 + c maps -0 to +0
    (src/engine/run.rs:265,313; src/graph/tape.rs:389-393)."""
    banner("program signed zeros")
    tape = t.Tape()
    w = tape.parameter((4,))
    z = tape.input((4,))
    loss = (w * z).sum()
    (grad,) = tape.differentiate(loss, [w])
    params = [np.array([1.0, -1.0, 2.0, -2.0], np.float32)]
    dense = {z.node.slot: np.array([-0.0, 0.0, -0.0, 3.0], np.float32)}
    want = run_oracle(tape, [loss, grad], params, dense)
    got, _ = run_device(tape, [loss, grad], params, dense)
    assert_bitwise(got[grad.id], want[grad.id], "grad")
    assert_bitwise(got[loss.id], want[loss.id], "loss")
    assert (got[grad.id].view(np.uint32)[:3] == 0).all()  # +0, not -0


def test_large_sparse_sum_is_exact(hip):
    """The cross-entropy alignment term (targets * logits).sum() over a wide
    vocabulary: the ordered sum over the gathered nonzero terms equals the
    interpreter's 1.6M-term left fold."""
    banner("program sparse sum")
    rng = np.random.default_rng(9)
    rows, vocab = 64, 25013
    tape = t.Tape()
    logits = tape.input((rows, vocab))
    targets = tape.selection_input(rows, vocab)
    total = (targets * logits).sum()
    count = targets.sum()
    dense = {logits.node.slot: rng.standard_normal((rows, vocab)).astype(np.float32)}
    selections = {targets.node.slot: (rng.integers(0, vocab, rows).astype(np.int32), 1.0)}
    want = run_oracle(tape, [total, count], [], dense, selections)
    got, _ = run_device(tape, [total, count], [], dense, selections)
    assert_bitwise(got[total.id], want[total.id], "sparse sum")
    assert_bitwise(got[count.id], want[count.id], "selection sum")


def test_sgd_step_matches_the_rule(hip):
    """Sgd::step p - g * lr⇑ (src/neural/optimizer.rs:40-51; the hand rule of
    src/neural/tests/optimizer_tests.rs:16-37)."""
    import torch

    from poorgrad_amd.program import sgd_step

    banner("sgd step")
    rng = np.random.default_rng(2)
    p = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    dp, dg = torch.from_numpy(p.copy()).cuda(), torch.from_numpy(g).cuda()
    sgd_step(dp, dg.data_ptr(), 0.01)
    want = p - g * np.float32(0.01)
    assert_bitwise(dp, want, "sgd")


def test_adamw_steps_match_the_rule(hip):
    """AdamW (src/neural/adam.rs:62-171) over three steps, restated in numpy
    f32 operation by operation."""
    import torch

    from poorgrad_amd.program import AdamW

    banner("adamw steps")
    rng = np.random.default_rng(3)
    shapes = [(7, 5), (5,)]
    params = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    device = [torch.from_numpy(p.copy()).cuda() for p in params]
    opt = AdamW(device, beta1=0.9, beta2=0.999, epsilon=1e-8, decay=0.01)
    f = np.float32
    b1, b2, eps, decay, lr = f(0.9), f(0.999), f(1e-8), f(0.01), f(3e-4)
    m = [np.zeros_like(p) for p in params]
    v = [np.zeros_like(p) for p in params]
    p1, p2 = f(1), f(1)
    for step in range(3):
        grads = [rng.standard_normal(s).astype(np.float32) for s in shapes]
        dgrads = [torch.from_numpy(g).cuda() for g in grads]
        opt.step(device, [g.data_ptr() for g in dgrads], float(lr))
        p1, p2 = f(p1 * b1), f(p2 * b2)
        c1, c2 = f(1) - p1, f(1) - p2
        for i, g in enumerate(grads):
            m[i] = m[i] * b1 + g * (f(1) - b1)
            v[i] = v[i] * b2 + (g * g) * (f(1) - b2)
            direction = (m[i] / c1) / (np.sqrt(v[i] / c2) + eps)
            stepped = params[i] - direction * lr
            params[i] = stepped - (params[i] * decay) * lr if params[i].ndim >= 2 else stepped
        torch.cuda.synchronize()
        for i in range(2):
            assert_bitwise(device[i], params[i], f"adamw step {step} param {i}")


def test_split_product_with_odd_width_and_fused_bias(hip):
    """A Linear layer whose product has enough tiles to fill the chip but
    fills its last round poorly, so it splits along k, with a width of 20001
    (rows that are not whole quads: the partials are reduced in quads of the
    flat output) and the bias added by that reduction: within the envelope
    |c - exact| <= 1e-5 * sum_k |x_ik w_kj| + 1 ulp for the bias addition."""
    banner("program split product, odd width, fused bias")
    tape = t.Tape()
    x = tape.input((640, 1024))
    w = tape.parameter((1024, 20001))
    b = tape.parameter((20001,))
    y = t.linear(x, w, b)
    g = oracle.Generator(23)
    xs = g.normal(640 * 1024, 1.0).reshape(640, 1024)
    ws = g.normal(1024 * 20001, 1.0).reshape(1024, 20001)
    bs = g.normal(20001, 1.0)
    want = run_oracle(tape, [y], [ws, bs], {x.node.slot: xs})[y.id].astype(np.float64)
    got, program = run_device(tape, [y], [ws, bs], {x.node.slot: xs}, numerics=hip.FAST)
    assert "+bias" in program.describe
    bound = 1e-5 * (np.abs(xs.astype(np.float64)) @ np.abs(ws.astype(np.float64)))
    bound += np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert (np.abs(got[y.id].astype(np.float64) - want) <= bound).all()


@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_powf_of_tensors_forward_and_backward(hip, posture):
    """f32::powf of two recorded tensors (src/payload/elementary.rs:133-135)
    and its rule (src/function/powf.rs:48-54: g * exponent * base^(exponent - 1)
    and g * output * ln(base)), in a chain and inside a row program (a
    softmax over powf values): bit-identical to the interpreter in both
    postures (no product in the graph)."""
    banner(f"program powf {posture}")
    rng = np.random.default_rng(41)
    tape = t.Tape()
    base = tape.parameter((24, 40))
    exponent = tape.parameter((24, 40))
    powered = base.powf(exponent)
    loss = (powered.log_softmax(1) * powered).sum()
    (gb, ge) = tape.differentiate(loss, [base, exponent])
    base0 = np.abs(rng.standard_normal((24, 40))).astype(np.float32) * np.float32(2) + np.float32(0.05)
    exponent0 = rng.standard_normal((24, 40)).astype(np.float32) * np.float32(1.5)
    params = [base0, exponent0]
    want = run_oracle(tape, [loss, gb, ge], params)
    got, program = run_device(tape, [loss, gb, ge], params, numerics=hip.EXACT if posture == "exact" else hip.FAST)
    assert "Powf" in program.describe
    for r in (loss, gb, ge):
        assert_bitwise(got[r.id], want[r.id], f"powf node {r.id}")


def test_device_adamw_follows_the_paper_trace(hip):
    """The reference's two-step Adam trace (src/neural/tests/adam_tests.rs:15-53:
    loss = w * w from w = 1, rate 0.1, betas 0.9 / 0.999, epsilon 1e-8, traced
    in f64 from the paper's rule) through the device kernel, with the gradient
    2w formed in f32 each step: within f32 rounding of the f64 trace, and
    bitwise equal to the numpy restatement."""
    import torch

    from poorgrad_amd.program import AdamW

    banner("adamw paper trace")
    w = torch.ones(1, device="cuda")
    opt = AdamW([w], decay=0.0)
    host = [np.ones(1, np.float32)]
    state = adamw_state(host)
    trace = paper_adam_trace(2)
    for step in range(2):
        gradient = (np.float32(2) * w.cpu().numpy()).astype(np.float32)
        g = torch.from_numpy(gradient).cuda()
        opt.step([w], [g.data_ptr()], 0.1)
        torch.cuda.synchronize()
        host = adamw_reference(host, [gradient], state, rate=0.1, decay=0.0)
        assert_bitwise(w, host[0], f"paper trace step {step}: device vs restatement")
        assert abs(float(w.cpu()[0]) - trace[step]) <= 1e-6 * abs(trace[step]), (step, float(w.cpu()[0]), trace[step])


def test_small_gpt2_adamw_steps_exact(hip):
    """Three train steps through the device program and the device AdamW,
    against the interpreter and the AdamW rule: every parameter bit-identical
    after every step. Exercises the side stream (parameter-gradient branches)
    across runs, where a scheduling race would change bits."""
    import torch

    from poorgrad_amd.program import AdamW, DeviceProgram

    banner("program gpt2 small three adamw steps")
    w = workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24)
    program = DeviceProgram(w.tape, w.roots, numerics=hip.EXACT)
    assert "[side]" in program.describe
    device = [torch.from_numpy(a.copy()).cuda() for a in w.initial]
    for slot, t_ in enumerate(device):
        program.bind_parameter(slot, t_)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    optimizer = AdamW(device)
    host = [a.copy() for a in w.initial]
    state = adamw_state(host)
    pointers = None
    for step in range(3):
        want = run_oracle(w.tape, w.roots, host, {}, w.selection_inputs)
        program.run()
        if pointers is None:
            pointers = [program.pointer(g) for g in w.gradients]
        optimizer.step(device, pointers, 3e-4)
        torch.cuda.synchronize()
        host = adamw_reference(host, [want[g.id] for g in w.gradients], state)
        for i, (d, h) in enumerate(zip(device, host)):
            assert_bitwise(d, h, f"step {step} parameter {i}")


def test_long_column_folds_exact(hip):
    """Column folds over many steps (several LDS tiles, a partial last tile),
    over an outer and a middle axis, with fused elementwise operands, a
    broadcast operand and a max fold: bit-identical to the interpreter's
    ascending first-term-seeded fold."""
    banner("program long column folds")
    rng = np.random.default_rng(21)
    tape = t.Tape()
    x = tape.input((1300, 52))
    y = tape.input((1300, 52))
    z = tape.input((3, 1100, 20))
    bias = tape.parameter((52,))
    roots = [
        x.sum_along(0),
        (x * y + bias.broadcast_along(0, x)).sum_along(0),
        (x.exp() - y).maximum(x).sum_along(0),
        z.sum_along(1),
        (z * z).sum_along(0),
        x.log_softmax(0).sum_along(0),
    ]
    params = [rng.standard_normal(52).astype(np.float32)]
    dense = {x.node.slot: rng.standard_normal((1300, 52)).astype(np.float32),
             y.node.slot: rng.standard_normal((1300, 52)).astype(np.float32),
             z.node.slot: rng.standard_normal((3, 1100, 20)).astype(np.float32)}
    want = run_oracle(tape, roots, params, dense)
    got, _ = run_device(tape, roots, params, dense, numerics=hip.EXACT)
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


@pytest.mark.parametrize("steps, columns", [(5000, 24), (8192, 768), (2048, 12), (600, 4096), (4099, 8), (300, 16384)])
def test_column_fold_shapes_exact(hip, steps, columns):
    """Column folds over several whole and partial tiles (an odd and an even
    count), at 16 and 64 outputs a workgroup, the bias-gradient shape
    [8192, 768], an all -0 column, a zero-seeded accumulation of the fold, a
    fused operand, and a per-row operand broadcast along the columns (the
    LayerNorm gain gradient's form): bit-identical to the ordered fold."""
    banner(f"program column fold widths {steps}x{columns}")
    rng = np.random.default_rng(steps + columns)
    tape = t.Tape()
    x = tape.input((steps, columns))
    y = tape.input((steps, columns))
    r = tape.input((steps,))
    folded = (x * y - x).sum_along(0)
    roots = [x.sum_along(0), folded + folded.zero_like(), (x * x).maximum(y).sum_along(0),
             (x * y * r.broadcast_along(1, x)).sum_along(0)]
    dense = {x.node.slot: rng.standard_normal((steps, columns)).astype(np.float32),
             y.node.slot: rng.standard_normal((steps, columns)).astype(np.float32),
             r.node.slot: rng.standard_normal(steps).astype(np.float32)}
    dense[x.node.slot][:, 0] = -0.0   # an all -0 column: -0 from the fold, +0 after the seed
    want = run_oracle(tape, roots, [], dense)
    got, _ = run_device(tape, roots, [], dense, numerics=hip.EXACT)
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


@pytest.mark.parametrize("rows, columns", [(37, 1100), (24, 1028), (130, 40), (9, 3), (5, 9001), (70, 3000)])
def test_row_groups_exact(hip, rows, columns):
    """Row programs (groups of row-local nodes with last-axis reductions):
    register-resident rows and streamed wide rows (several column slabs),
    a partial last row block, quads and single columns, row operands broadcast back along the row, LogSumExp and
    LogSoftmax with fused operands and consumers, a ReLU member, and a row
    input: bit-identical to the interpreter."""
    banner(f"program row groups {rows}x{columns}")
    rng = np.random.default_rng(rows * 7 + columns)
    tape = t.Tape()
    x = tape.input((rows, columns))
    y = tape.input((rows, columns))
    v = tape.input((rows,))
    eps = tape.leaf(t.Constant((), 1e-5))
    mean = x.sum_along(1) / t.counted((rows,), columns)
    c = x - mean.broadcast_along(1, x)
    var = (c * c).sum_along(1) / t.counted((rows,), columns) + v.abs()
    n = c / (var + eps.broadcast_like(var)).sqrt().broadcast_along(1, x)
    soft = (n * y).relu().log_softmax(1)
    roots = [n, var, soft, soft.exp() * y, (x * y).logsumexp(1), (y - x).logsumexp(1).exp()]
    dense = {x.node.slot: (3 * rng.standard_normal((rows, columns))).astype(np.float32),
             y.node.slot: rng.standard_normal((rows, columns)).astype(np.float32),
             v.node.slot: rng.standard_normal(rows).astype(np.float32)}
    want = run_oracle(tape, roots, [], dense)
    got, program = run_device(tape, roots, [], dense, numerics=hip.EXACT)
    assert ": rows [" in program.describe
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


def test_row_groups_rank3_and_selection(hip):
    banner("program row groups rank 3 and selection")
    rng = np.random.default_rng(31)
    tape = t.Tape()
    z = tape.input((5, 6, 16))
    logits = tape.input((12, 7))
    targets = tape.selection_input(12, 7)
    roots = [z.log_softmax(2).exp(), (z * z).sum_along(2), t.cross_entropy(logits, targets),
             tape.value(targets.id).sum_along(1)]
    dense = {z.node.slot: rng.standard_normal((5, 6, 16)).astype(np.float32),
             logits.node.slot: rng.standard_normal((12, 7)).astype(np.float32)}
    selections = {targets.node.slot: (rng.integers(0, 7, 12).astype(np.int32), 1.0)}
    want = run_oracle(tape, roots, [], dense, selections)
    got, _ = run_device(tape, roots, [], dense, selections, hip.EXACT)
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


@pytest.mark.parametrize("one", [1.0, -0.0, 0.0, 2.5, -3.0e38, float("inf")])
@pytest.mark.parametrize("vocab", [1, 7])
def test_selection_sums_exact(hip, one, vocab):
    """Sums of a selection (a one-hot [rows, vocab] with `one` at each row's
    index and +0 elsewhere) along its rows and over everything: planned as
    constants, bit-identical to the interpreter's ordered folds, signed zeros
    and overflow included."""
    banner(f"program selection sums one={one} vocab={vocab}")
    rng = np.random.default_rng(vocab)
    rows = 300
    tape = t.Tape()
    sel = tape.selection_input(rows, vocab, one)
    v = tape.value(sel.id)
    roots = [v.sum_along(1), v.sum(), (v.sum_along(1) * v.sum_along(1)).sum()]
    selections = {sel.node.slot: (rng.integers(0, vocab, rows).astype(np.int32), one)}
    want = run_oracle(tape, roots, [], {}, selections)
    got, _ = run_device(tape, roots, [], {}, selections, hip.EXACT)
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


def test_fast_zero_seeded_product_is_the_product(hip):
    """Under Fast, +0 + p of a matrix-core product is planned as p itself:
    the addition only maps -0 to +0, and the matrix-core accumulators start
    at +0, so a product whose terms are all -0 (or cancel) is +0 already."""
    banner("program fast zero-seeded product")
    tape = t.Tape()
    a = tape.input((64, 32))
    b = tape.input((32, 48))
    zero = tape.leaf(t.Constant((64, 48), 0.0))
    p = a.matmul(b)
    roots = [zero + p]
    av = np.full((64, 32), -0.0, np.float32)
    av[1] = 1.0
    av[2, :2] = [1.0, -1.0]
    bv = np.abs(np.random.default_rng(3).standard_normal((32, 48))).astype(np.float32)
    bv[:2] = 1.0
    got, program = run_device(tape, roots, [], {a.node.slot: av, b.node.slot: bv}, numerics=hip.FAST)
    assert "chain" not in program.describe, program.describe
    out = got[roots[0].id]
    assert (out[0].view(np.uint32) == 0).all() and (out[2].view(np.uint32) == 0).all()  # +0, never -0
    want = run_oracle(tape, roots, [], {a.node.slot: av, b.node.slot: bv})[roots[0].id]
    assert np.allclose(out, want, rtol=1e-5, atol=0)


def test_strided_reshape_views_exact(hip):
    """Reshapes that split strided axes are views; reshapes that merge
    strided axes copy: both read the interpreter's elements in logical
    order."""
    banner("program strided reshape views")
    rng = np.random.default_rng(17)
    tape = t.Tape()
    fused = tape.input((48, 36))
    q = fused.narrow(1, 12, 12).reshape((2, 24, 3, 4))          # split a strided row axis: a view
    heads = q.permute((0, 2, 1, 3)).reshape((6, 24, 4))         # merge strided axes: copied
    back = heads.reshape((2, 3, 24, 4)).permute((0, 2, 1, 3)).reshape((48, 12))
    roots = [q * q, heads.matmul(heads.permute((0, 2, 1))), back + fused.narrow(1, 0, 12),
             fused.transpose().narrow(0, 3, 8).reshape((2, 4, 48)).sum_along(1)]
    dense = {fused.node.slot: rng.standard_normal((48, 36)).astype(np.float32)}
    want = run_oracle(tape, roots, [], dense)
    got, _ = run_device(tape, roots, [], dense, numerics=hip.EXACT)
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


@pytest.mark.parametrize("m, n, k, bias_first", [(64, 48, 32, False), (256, 256, 8192, False),
                                                 (256, 256, 8192, True), (100, 70, 50, True)])
def test_fast_linear_bias_is_added_by_the_product(hip, m, n, k, bias_first):
    """Under Fast, product + bias (Linear::express, src/neural/linear.rs:94-105)
    is written by the matrix-core kernel, with the split-k reduction adding
    the bias when the product is split: bit-identical to the same product
    read back and added in f32 on the host, in the recorded operand order."""
    banner(f"program fast fused bias {m}x{n}x{k} first={bias_first}")
    rng = np.random.default_rng(m + n + k)
    tape = t.Tape()
    a = tape.input((m, k))
    b = tape.input((k, n))
    c = tape.input((n,))
    p = a.matmul(b)
    bias = c.broadcast_along(0, p)
    y = bias + p if bias_first else p + bias
    dense = {a.node.slot: rng.standard_normal((m, k)).astype(np.float32),
             b.node.slot: rng.standard_normal((k, n)).astype(np.float32),
             c.node.slot: rng.standard_normal(n).astype(np.float32)}
    dense[c.node.slot][:3] = [np.inf, -0.0, np.nan]
    got, program = run_device(tape, [y], [], dense, numerics=hip.FAST)
    assert "bias" in program.describe and "chain" not in program.describe, program.describe
    product, _ = run_device(tape, [p], [], dense, numerics=hip.FAST)
    p_host, c_host = product[p.id], dense[c.node.slot][None, :]
    want = (c_host + p_host) if bias_first else (p_host + c_host)
    assert_bitwise(got[y.id], want, "fused bias")


def test_fast_bias_computed_after_the_product_is_not_fused(hip):
    """A bias whose own launch comes after the product's stays a separate
    addition; the result is the interpreter's within the Fast envelope."""
    banner("program fast late bias")
    rng = np.random.default_rng(5)
    tape = t.Tape()
    a = tape.input((96, 40))
    b = tape.input((40, 56))
    c = tape.input((56,))
    p = a.matmul(b)
    late = c * c + c
    y = p + late.broadcast_along(0, p)
    dense = {a.node.slot: rng.standard_normal((96, 40)).astype(np.float32),
             b.node.slot: rng.standard_normal((40, 56)).astype(np.float32),
             c.node.slot: rng.standard_normal(56).astype(np.float32)}
    got, program = run_device(tape, [y], [], dense, numerics=hip.FAST)
    assert "bias" not in program.describe, program.describe
    want = run_oracle(tape, [y], [], dense)[y.id]
    assert (np.abs(got[y.id] - want) <= 1e-4 * np.maximum(np.abs(want), 1.0)).all()


@pytest.mark.parametrize("case", ["dense", "zeros", "nonfinite", "passes"])
def test_whole_sums_exact(hip, case):
    """Whole-tensor sums (tensor.rs:1055-1063) through the gathered ordered
    fold: dense operands whose terms overflow the fold's LDS stage, all-zero
    operands (-0 only when every term is -0), infinities and NaN among the
    terms, and a sparse operand spanning several passes of chunks."""
    banner(f"program whole sum {case}")
    rng = np.random.default_rng(31)
    tape = t.Tape()
    dense, selections = {}, {}
    if case == "dense":
        x = tape.input((1500, 2000))
        dense[x.node.slot] = rng.standard_normal((1500, 2000)).astype(np.float32)
        roots = [x.sum(), (x * x).sum()]
    elif case == "zeros":
        x = tape.input((64, 1000))
        neg = np.full((64, 1000), -0.0, np.float32)
        mixed = neg.copy()
        mixed[40, 999] = 0.0
        y = tape.input((64, 1000))
        dense[x.node.slot], dense[y.node.slot] = neg, mixed
        roots = [x.sum(), y.sum(), (x + x).sum()]
    elif case == "nonfinite":
        x = tape.input((300, 700))
        v = np.zeros((300, 700), np.float32)
        v[3, 5], v[100, 2], v[250, 600] = 2.5, np.inf, -1.0
        w = v.copy()
        w[299, 699] = -np.inf
        u = np.where(rng.random((300, 700)) < 0.001, np.float32(np.nan), np.float32(0.0)).astype(np.float32)
        u[0, 0] = 1.0
        y, z = tape.input((300, 700)), tape.input((300, 700))
        dense[x.node.slot], dense[y.node.slot], dense[z.node.slot] = v, w, u
        roots = [x.sum(), y.sum(), z.sum()]
    else:
        logits = tape.input((2048, 9000))
        targets = tape.selection_input(2048, 9000)
        dense[logits.node.slot] = rng.standard_normal((2048, 9000)).astype(np.float32)
        selections[targets.node.slot] = (rng.integers(0, 9000, 2048).astype(np.int32), 1.0)
        roots = [(targets * logits).sum()]
    want = run_oracle(tape, roots, [], dense, selections)
    got, program = run_device(tape, roots, [], dense, selections)
    assert "sum (ordered, gathered)" in program.describe, program.describe
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"{case} sum node {r.id}")


def test_joined_chains_exact(hip):
    """Consecutive chains over one shape run as one multi-output kernel (a
    member reading an earlier member's output takes it from registers); a
    chain reading that output transposed runs after it. Bit-identical to the
    interpreter either way, including outputs only the joined members read."""
    banner("program joined chains")
    rng = np.random.default_rng(23)
    tape = t.Tape()
    x = tape.input((48, 48))
    y = tape.input((48, 48))
    a = x * x + y
    b = a * x
    c = (b + a).exp()
    d = a.transpose() * y
    g = (c * b).tanh() + b
    roots = [c, d, g]
    dense = {x.node.slot: rng.standard_normal((48, 48)).astype(np.float32),
             y.node.slot: rng.standard_normal((48, 48)).astype(np.float32)}
    want = run_oracle(tape, roots, [], dense)
    got, program = run_device(tape, roots, [], dense)
    assert "outputs" in program.describe, program.describe
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id}")


@pytest.mark.parametrize("columns", [1024, 768])
def test_row_sums_with_zero_tails_exact(hip, columns):
    """Row sums over resident four-row blocks whose rows end in zeros: +0,
    -0 and mixed zero tails, all -0 rows (the sum is -0), a -0 run meeting a
    +0 (+0), cancellations to +0, NaN and infinities before a zero tail, and
    a causal softmax (exp of masked terms is +0): bit-identical to the
    interpreter's ordered folds."""
    banner(f"program row sums zero tails {columns}")
    rng = np.random.default_rng(53)
    rows = 48
    x = rng.standard_normal((rows, columns)).astype(np.float32)
    pz, nz = np.float32(0.0), np.float32(-0.0)
    x[0, 5:] = pz
    x[1, 5:] = nz
    x[2, :] = nz
    x[3, :] = nz; x[3, -1] = pz
    x[4, :] = nz; x[4, 700 % columns] = pz
    x[5, :] = pz
    x[6, :2] = [1.0, -1.0]; x[6, 2:] = nz
    x[7, :2] = [-1.0, 1.0]; x[7, 2:] = nz; x[7, 40] = pz
    x[8, :] = nz; x[8, 33] = 2.5; x[8, 34:] = pz
    x[9, 10] = np.nan; x[9, 11:] = pz
    x[10, 3] = np.inf; x[10, 4:] = nz
    x[11, 31] = 1e-30; x[11, 32:] = nz; x[11, 63] = pz
    for r in range(12, rows):
        tail = int(rng.integers(0, columns))
        x[r, tail:] = np.where(rng.random(columns - tail) < 0.5, pz, nz)
    causal = np.where(np.arange(columns)[None, :] <= (np.arange(rows) * (columns // rows))[:, None], 0.0,
                      -np.inf).astype(np.float32)
    tape = t.Tape()
    xi = tape.input((rows, columns))
    mask = tape.leaf(t.Dense(causal))
    roots = [xi.sum_along(1), (xi + mask).softmax(1), (xi * xi + mask).logsumexp(1)]
    dense = {xi.node.slot: x}
    want = run_oracle(tape, roots, [], dense)
    got, program = run_device(tape, roots, [], dense)
    assert ": rows [" in program.describe
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")


@pytest.mark.parametrize("form", ["plain", "left_transposed", "right_transposed"])
def test_fast_batched_products_with_edges(hip, form):
    """Batched fast products whose tiles overhang m and n (the LDS-DMA
    kernel clamps those loads), in each operand orientation: within the
    envelope of the interpreter's exact product."""
    banner(f"program fast batched edges {form}")
    rng = np.random.default_rng(41)
    B, M, K, N = 3, 300, 96, 260
    tape = t.Tape()
    if form == "left_transposed":
        a = tape.input((B, K, M)); av = a.permute((0, 2, 1))
    else:
        a = tape.input((B, M, K)); av = a
    if form == "right_transposed":
        b = tape.input((B, N, K)); bv = b.permute((0, 2, 1))
    else:
        b = tape.input((B, K, N)); bv = b
    y = av.matmul(bv)
    dense = {a.node.slot: rng.standard_normal(tape.input_shapes[0]).astype(np.float32),
             b.node.slot: rng.standard_normal(tape.input_shapes[1]).astype(np.float32)}
    want = run_oracle(tape, [y], [], dense)[y.id].astype(np.float64)
    got, _ = run_device(tape, [y], [], dense, numerics=hip.FAST)
    la = dense[a.node.slot] if form != "left_transposed" else dense[a.node.slot].transpose(0, 2, 1)
    lb = dense[b.node.slot] if form != "right_transposed" else dense[b.node.slot].transpose(0, 2, 1)
    bound = 1e-5 * np.einsum("bmk,bkn->bmn", np.abs(la.astype(np.float64)), np.abs(lb.astype(np.float64)))
    assert (np.abs(got[y.id].astype(np.float64) - want) <= bound).all()


@pytest.mark.parametrize("form", ["plain", "left_transposed", "right_transposed"])
@pytest.mark.parametrize("shape", [(256, 257, 72, 130), (200, 61, 40, 998), (64, 520, 64, 700), (130, 300, 24, 257)])
def test_fast_many_short_products(hip, form, shape):
    """Many short batched products (k at most 128, over a thousand output
    tiles, like the attention scores): 256x128 tiles with a k tail and
    row/column overhang (k of 72, 64 and 24), and 64x128 tiles with a ragged
    outer-contiguous edge, in each operand orientation. Within the envelope
    of the interpreter's exact product."""
    B, M, K, N = shape
    banner(f"program fast many short products {form} {shape}")
    rng = np.random.default_rng(47)
    tape = t.Tape()
    if form == "left_transposed":
        a = tape.input((B, K, M)); av = a.permute((0, 2, 1))
    else:
        a = tape.input((B, M, K)); av = a
    if form == "right_transposed":
        b = tape.input((B, N, K)); bv = b.permute((0, 2, 1))
    else:
        b = tape.input((B, K, N)); bv = b
    y = av.matmul(bv)
    dense = {a.node.slot: rng.standard_normal(tape.input_shapes[0]).astype(np.float32),
             b.node.slot: rng.standard_normal(tape.input_shapes[1]).astype(np.float32)}
    want = run_oracle(tape, [y], [], dense)[y.id].astype(np.float64)
    got, _ = run_device(tape, [y], [], dense, numerics=hip.FAST)
    la = dense[a.node.slot] if form != "left_transposed" else dense[a.node.slot].transpose(0, 2, 1)
    lb = dense[b.node.slot] if form != "right_transposed" else dense[b.node.slot].transpose(0, 2, 1)
    bound = 1e-5 * np.matmul(np.abs(la.astype(np.float64)), np.abs(lb.astype(np.float64)))
    assert (np.abs(got[y.id].astype(np.float64) - want) <= bound).all()


def test_fast_head_merging_views_within_envelope(hip):
    """Attention heads split from a fused projection and merged back
    (examples/gpt2/model.rs split_heads): the products read the heads through
    two-level batch strides and the head-merging reshape after the last
    product is written by the product itself; gradients flow through both.
    Within the envelope of the interpreter."""
    banner("program fast head views")
    rng = np.random.default_rng(43)
    batch, context, heads, head = 2, 24, 3, 8
    width = heads * head
    tape = t.Tape()
    fused = tape.parameter((batch * context, 3 * width))

    def split(part):
        x = fused.narrow(1, part * width, width).reshape((batch, context, heads, head))
        return x.permute((0, 2, 1, 3)).reshape((batch * heads, context, head))

    q, k, v = split(0), split(1), split(2)
    weights = q.matmul(k.permute((0, 2, 1))).softmax(2)
    attended = weights.matmul(v).reshape((batch, heads, context, head)).permute((0, 2, 1, 3))
    merged = attended.reshape((batch * context, width))
    loss = (merged * merged).sum()
    (grad,) = tape.differentiate(loss, [fused])
    params = [rng.standard_normal((batch * context, 3 * width)).astype(np.float32)]
    want = run_oracle(tape, [loss, merged, grad], params)
    got, program = run_device(tape, [loss, merged, grad], params, numerics=hip.FAST)
    for r in (loss, merged, grad):
        g, e = got[r.id].astype(np.float64), want[r.id].astype(np.float64)
        assert (np.abs(g - e) <= 1e-4 * np.maximum(np.abs(e), 1.0)).all(), f"node {r.id}"


@pytest.mark.parametrize("columns", [1024, 768])
def test_row_softmax_underflow_skip_is_exact(hip, columns):
    """A row program's exponentials of a point are skipped when every point
    of the wave lies at or below -104 after the max shift (each e^x then
    rounds to +0). Rows whose tail columns hold -inf, -1e30, -200, -104 and
    values just above it (-103.99, -103.97, -103.9: e^x is 0 or the smallest
    subnormals) beside a normal head: bitwise against the interpreter, in the
    softmax and log-softmax and in the gradient (src/function/log_softmax.rs:51-72)."""
    banner(f"program softmax underflow skip {columns}")
    rng = np.random.default_rng(53)
    tails = [-np.inf, -1e30, -200.0, -104.0, -103.99, -103.97, -103.9, -50.0]
    rows = 64
    x = (-rng.random((rows, columns))).astype(np.float32)  # head values in (-1, 0]
    for r in range(rows):
        start = 64 + 64 * (r % 4)
        x[r, start:] = np.float32(tails[r % len(tails)])
        x[r, 0] = np.float32(0.0)  # the maximum: a tail's shifted value is the tail itself
    tape = t.Tape()
    a = tape.parameter((rows, columns))
    soft = a.softmax(1)
    logsoft = a.log_softmax(1)
    loss = (soft * soft).sum() + logsoft.sum()
    grads = tape.differentiate(loss, [a])
    roots = [soft, logsoft, loss] + grads
    want = run_oracle(tape, roots, [x])
    got, _ = run_device(tape, roots, [x], numerics=hip.EXACT)
    for r in roots:
        assert_bitwise(got[r.id], want[r.id], f"node {r.id} {r.shape}")
