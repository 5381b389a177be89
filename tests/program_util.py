"""Shared helpers: run a recorded graph through the oracle interpreter and
through the device program, on the same inputs."""
import numpy as np

from oracle import interpreter


def oracle_inputs(tape, dense: dict, selections: dict) -> list:
    inputs = [None] * len(tape.input_shapes)
    for slot, array in dense.items():
        inputs[slot] = np.ascontiguousarray(array, dtype=np.float32)
    for slot, (indices, one) in selections.items():
        inputs[slot] = interpreter.Sel(indices, tape.input_shapes[slot][1], one)
    return inputs


def run_oracle(tape, roots, parameters, dense=None, selections=None) -> dict:
    with np.errstate(all="ignore"):
        return interpreter.run(tape, roots, [np.asarray(p, np.float32) for p in parameters],
                               oracle_inputs(tape, dense or {}, selections or {}))


def run_device(tape, roots, parameters, dense=None, selections=None, numerics=None, observe=()):
    import torch

    from poorgrad_amd import _native as n
    from poorgrad_amd.program import DeviceProgram

    numerics = n.EXACT if numerics is None else numerics
    program = DeviceProgram(tape, roots, observe, numerics=numerics)
    held = []
    for slot, array in enumerate(parameters):
        t = torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).cuda()
        held.append(t)
        program.bind_parameter(slot, t)
    for slot, array in (dense or {}).items():
        t = torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).cuda()
        held.append(t)
        program.bind_input(slot, t)
    for slot, (indices, one) in (selections or {}).items():
        program.bind_selection(slot, indices, one)
    program.run()
    torch.cuda.synchronize()
    out = {r.id: program.read(r) for r in list(roots) + list(observe)}
    return out, program


def adamw_state(parameters) -> dict:
    """Zero moments and unit bias-correction powers for adamw_reference."""
    return {"p1": np.float32(1), "p2": np.float32(1), "m": [np.zeros_like(a) for a in parameters],
            "v": [np.zeros_like(a) for a in parameters]}


def adamw_reference(params, grads, state, rate=3e-4, beta1=0.9, beta2=0.999, epsilon=1e-8, decay=0.01,
                    f=np.float32):
    """AdamW::step (src/neural/adam.rs:62-171) restated in numpy f32, operation
    by operation: the moments, the bias corrections 1 - beta^t, the direction
    (m / c1) / (sqrt(v / c2) + epsilon), the step p - direction * rate, and the
    decoupled decay (p * decay) * rate for parameters of rank >= 2."""
    b1, b2, eps, dec, lr = f(beta1), f(beta2), f(epsilon), f(decay), f(rate)
    state["p1"], state["p2"] = f(state["p1"] * b1), f(state["p2"] * b2)
    c1, c2 = f(1) - state["p1"], f(1) - state["p2"]
    out = []
    for i, (p, g) in enumerate(zip(params, grads)):
        m = state["m"][i] * b1 + g * (f(1) - b1)
        v = state["v"][i] * b2 + (g * g) * (f(1) - b2)
        state["m"][i], state["v"][i] = m, v
        direction = (m / c1) / (np.sqrt(v / c2) + eps)
        stepped = p - direction * lr
        out.append(stepped - (p * dec) * lr if p.ndim >= 2 else stepped)
    return out


def paper_adam_trace(steps: int, w: float = 1.0, rate: float = 0.1) -> list:
    """The hand trace of src/neural/tests/adam_tests.rs:15-53 in f64: loss = w * w,
    gradient 2w, the paper's update rule with betas 0.9 / 0.999 and epsilon 1e-8."""
    m = v = 0.0
    p1 = p2 = 1.0
    out = []
    for _ in range(steps):
        gradient = 2.0 * w
        m = m * 0.9 + gradient * (1.0 - 0.9)
        v = v * 0.999 + gradient * gradient * (1.0 - 0.999)
        p1 *= 0.9
        p2 *= 0.999
        w -= rate * (m / (1.0 - p1)) / (np.sqrt(v / (1.0 - p2)) + 1e-8)
        out.append(w)
    return out
