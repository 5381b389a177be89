"""The engine-backward route on the device: a forward-only table, the
library's own reverse scan (Run::backward, src/engine/run.rs:229-318), one
program. Its gradients equal the recorded route's (Tape::differentiate,
src/graph/tape.rs:335-411, the invariant of
src/graph/tests/differentiate_tests.rs:19-25) and the oracle interpreter's
bit for bit under Exact, and the recorded route's device program bit for bit
under Fast (the two routes plan the same launches)."""
import numpy as np
import pytest

from poorgrad_amd import topos as t
from poorgrad_amd import workloads
from tests.conftest import banner
from tests.gpu_util import assert_bitwise
from tests.program_util import run_oracle

pytestmark = pytest.mark.gpu

CASES = {
    "mlp": lambda g: workloads.mlp(record_gradients=g),
    "gpt2": lambda g: workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24,
                                     record_gradients=g),
    "llama": lambda g: workloads.llama(batch=2, context=16, vocab=37, width=32, heads=4, hidden=48, layers=2,
                                       record_gradients=g),
    "cnn": lambda g: workloads.cnn(batch=4, record_gradients=g),
    "batch_norm_mlp": lambda g: workloads.batch_norm_mlp(batch=8, record_gradients=g),
}


def _bind(program, w):
    import torch

    held = []
    for slot, array in enumerate(w.initial):
        tensor = torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).cuda()
        held.append(tensor)
        program.bind_parameter(slot, tensor)
    for slot, array in w.dense_inputs.items():
        tensor = torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).cuda()
        held.append(tensor)
        program.bind_input(slot, tensor)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    return held


@pytest.mark.parametrize("model", list(CASES))
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_engine_backward_equals_recorded_gradients(hip, model, posture):
    import torch

    from poorgrad_amd.program import DeviceProgram

    numerics = hip.EXACT if posture == "exact" else hip.FAST
    recorded, forward = CASES[model](True), CASES[model](False)
    banner(f"engine backward {model} {posture}: recorded route")
    a = DeviceProgram(recorded.tape, recorded.roots, numerics=numerics)
    held_a = _bind(a, recorded)
    a.run()
    banner(f"engine backward {model} {posture}: engine route")
    b = DeviceProgram.engine_backward(forward.tape, forward.loss, forward.parameters, numerics=numerics)
    held_b = _bind(b, forward)
    b.run()
    torch.cuda.synchronize()
    assert_bitwise(b.read(forward.loss), a.read(recorded.loss), f"{model} loss")
    for i, (p, g) in enumerate(zip(forward.parameters, recorded.gradients)):
        assert_bitwise(b.read_gradient(p), a.read(g), f"{model} gradient {i}")
    if numerics == hip.EXACT:
        want = run_oracle(recorded.tape, recorded.roots, recorded.initial, recorded.dense_inputs,
                          recorded.selection_inputs)
        for i, (p, g) in enumerate(zip(forward.parameters, recorded.gradients)):
            assert_bitwise(b.read_gradient(p), want[g.id], f"{model} gradient {i} vs oracle")
    del held_a, held_b


def test_engine_backward_skips_disconnected_and_data_edges(hip):
    """Only ancestors run their rules (run.rs:266-281): a singular expression
    the target does not depend on, or reaches only through a broadcast's
    reference, leaves the genuine gradient finite; a value after the target
    or outside its ancestry has the zero gradient; the target's own gradient
    is one."""
    import torch

    from poorgrad_amd.program import DeviceProgram

    banner("engine backward: disconnected and data edges")
    tape = t.Tape()
    w = tape.parameter((3, 4))
    zero = w - w
    singular = zero / zero                      # NaN everywhere, never an ancestor
    c = tape.leaf(t.Constant((), 2.0))
    scaled = w * c.broadcast_like(singular)     # `singular` only as a shape reference
    loss = (scaled * w).sum()
    after = loss.exp()                          # recorded after the target
    program = DeviceProgram.engine_backward(tape, loss, [w, singular, after, loss], numerics=hip.EXACT)
    values = np.arange(12, dtype=np.float32).reshape(3, 4) / np.float32(4) - np.float32(1)
    param = torch.from_numpy(values).cuda()
    program.bind_parameter(0, param)
    program.run()
    torch.cuda.synchronize()
    # d/dw sum(2 w * w) recorded by the rules: 2w * 1 (from scaled's Mul) and
    # the product rule's other term, each zero-seeded; compare with the oracle.
    tape2 = t.Tape()
    w2 = tape2.parameter((3, 4))
    zero2 = w2 - w2
    singular2 = zero2 / zero2
    c2 = tape2.leaf(t.Constant((), 2.0))
    loss2 = ((w2 * c2.broadcast_like(singular2)) * w2).sum()
    (g2,) = tape2.differentiate(loss2, [w2])
    want = run_oracle(tape2, [loss2, g2], [values])
    got = program.read_gradient(w)
    assert np.isfinite(got).all()
    assert_bitwise(got, want[g2.id], "gradient through a data edge")
    assert_bitwise(program.read_gradient(singular), np.zeros((3, 4), np.float32), "disconnected value")
    assert_bitwise(program.read_gradient(after), np.zeros((), np.float32), "value after the target")
    assert_bitwise(program.read_gradient(loss), np.ones((), np.float32), "the target's own gradient")
