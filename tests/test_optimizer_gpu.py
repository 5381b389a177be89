"""The many-parameter AdamW entry (topos_hip_adamw_step_multi_f32) against the
single-parameter one, which the program tests hold to the oracle's
restatement of AdamW::step (src/neural/adam.rs:62-171): the same bits for
every parameter and moment, over three steps, with empty, one-element and
large tensors, decayed and spared ones, and more tensors than one launch
takes (48)."""
import ctypes

import numpy as np
import pytest

from tests.conftest import banner
from tests.gpu_util import assert_bitwise

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("offset", [0, 1, 2])
def test_multi_tensor_adamw_equals_single_tensor_steps(hip, offset):
    """offset 0: 16-byte aligned buffers (whole quads move in 16-byte loads
    and stores); 1 and 2: every buffer, or only the gradients, start one
    float into an allocation (the element-by-element path)."""
    import torch

    banner(f"adamw multi-tensor vs single-tensor offset={offset}")
    rng = np.random.default_rng(3)
    sizes = [0, 1, 5, 768, 1000, 100003, 2304 * 768] + [int(s) for s in rng.integers(1, 5000, 60)]
    make = lambda s: torch.from_numpy(rng.standard_normal(s).astype(np.float32)).cuda()

    def placed(t, shift):
        if not shift:
            return t
        buffer = torch.empty(t.numel() + 1, device="cuda")
        view = buffer[1:]
        view.copy_(t)
        return view

    params = [make(s) for s in sizes]
    grads = [placed(make(s), offset > 0) for s in sizes]
    decayed = [i % 3 != 0 for i in range(len(sizes))]
    single = [(p.clone(), torch.zeros_like(p), torch.zeros_like(p)) for p in params]
    multi = [tuple(placed(x, offset == 1) for x in (p.clone(), torch.zeros_like(p), torch.zeros_like(p)))
             for p in params]
    f = np.float32
    beta1, beta2, eps, decay, rate = f(0.9), f(0.999), f(1e-8), f(0.01), 3e-4
    p1 = p2 = f(1)
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        p1, p2 = f(p1 * beta1), f(p2 * beta2)
        c1, c2 = f(1) - p1, f(1) - p2
        scalars = (float(beta1), float(beta2), float(f(1) - beta1), float(f(1) - beta2), float(c1), float(c2),
                   float(eps), rate, float(decay))
        for (p, m, v), g, d in zip(single, grads, decayed):
            hip.checked(hip.lib.topos_hip_adamw_step_f32(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
                                                         p.numel(), *scalars[:-1], scalars[-1], int(d), stream),
                        "adamw single")
        table = (hip.AdamwTensor * len(sizes))()
        for j, ((p, m, v), g, d) in enumerate(zip(multi, grads, decayed)):
            table[j] = hip.AdamwTensor(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), p.numel(), int(d))
        hip.checked(hip.lib.topos_hip_adamw_step_multi_f32(table, len(sizes), *scalars, stream), "adamw multi")
    torch.cuda.synchronize()
    for j, (a, b) in enumerate(zip(single, multi)):
        for name, x, y in zip(("parameter", "first", "second"), a, b):
            assert_bitwise(y.cpu().numpy(), x.cpu().numpy(), f"tensor {j} ({sizes[j]}) {name}")


def test_multi_tensor_adamw_refuses_bad_tables(hip):
    table = (hip.AdamwTensor * 1)()
    table[0] = hip.AdamwTensor(0, 0, 0, 0, 4, 1)
    assert hip.lib.topos_hip_adamw_step_multi_f32(table, 1, 0.9, 0.999, 0.1, 0.001, 0.1, 0.001, 1e-8, 1e-3, 0.01,
                                                  None) == hip.INVALID_ARGUMENT
    assert hip.lib.topos_hip_adamw_step_multi_f32(None, 0, 0.9, 0.999, 0.1, 0.001, 0.1, 0.001, 1e-8, 1e-3, 0.01,
                                                  None) == hip.OK


def test_multi_tensor_adamw_with_overlapping_entries(hip):
    """A table whose entries share memory (a tied parameter listed twice with
    its own moments, and a gradient that is another entry's parameter): the
    library splits the launch before each overlap, so the result equals the
    one-tensor entry applied in table order."""
    import torch

    banner("adamw multi-tensor, overlapping entries")
    rng = np.random.default_rng(4)
    make = lambda s: torch.from_numpy(rng.standard_normal(s).astype(np.float32)).cuda()
    tied, other = make(4096), make(1000)
    gradients = [make(4096), make(4096), None]
    f = np.float32
    scalars = (0.9, 0.999, float(f(1) - f(0.9)), float(f(1) - f(0.999)), float(f(1) - f(0.9)),
               float(f(1) - f(0.999)), 1e-8, 3e-4, 0.01)
    stream = torch.cuda.current_stream().cuda_stream

    def entries(state):
        tied_p, other_p, moments = state
        # tied twice (each listing with its own moments), then `other`, whose
        # gradient is a window of the tied parameter the first entries write.
        return [(tied_p, gradients[0], moments[0], moments[1], 1), (tied_p, gradients[1], moments[2], moments[3], 1),
                (other_p, tied_p[:1000], moments[4], moments[5], 0)]

    def fresh():
        return (tied.clone(), other.clone(),
                [torch.zeros(4096, device="cuda") for _ in range(4)] + [torch.zeros(1000, device="cuda")
                                                                        for _ in range(2)])

    single, multi = fresh(), fresh()
    for p, g, m, v, d in entries(single):
        hip.checked(hip.lib.topos_hip_adamw_step_f32(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
                                                     p.numel(), *scalars[:-1], scalars[-1], d, stream), "single")
    listed = entries(multi)
    table = (hip.AdamwTensor * len(listed))()
    for j, (p, g, m, v, d) in enumerate(listed):
        table[j] = hip.AdamwTensor(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), p.numel(), d)
    hip.checked(hip.lib.topos_hip_adamw_step_multi_f32(table, len(listed), *scalars, stream), "multi")
    torch.cuda.synchronize()
    assert_bitwise(multi[0].cpu().numpy(), single[0].cpu().numpy(), "tied parameter")
    assert_bitwise(multi[1].cpu().numpy(), single[1].cpu().numpy(), "parameter with an aliased gradient")
    for j, (x, y) in enumerate(zip(single[2], multi[2])):
        assert_bitwise(y.cpu().numpy(), x.cpu().numpy(), f"moment {j}")
