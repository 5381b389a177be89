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
