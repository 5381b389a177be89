"""Several host threads on one library: a Plan is Send + Sync and several
threads may forward it (src/engine/plan.rs:20); the CUDA rung's context is
shared by every thread (src/backend/cuda/kernels/context.rs:203-212).

* One device program run from four threads, each on its own stream: every
  run is ordered after the previous one on the GPU, so each thread reads
  bits equal to a single-threaded run's.
* Device-face split products from four threads on four streams, with sizes
  that regrow the shared split-k workspace mid-flight: each product equals
  the one computed alone."""
import threading

import numpy as np
import pytest

from poorgrad_amd import workloads
from tests.conftest import banner
from tests.gpu_util import assert_bitwise

pytestmark = pytest.mark.gpu


def test_one_program_run_from_four_threads(hip):
    import torch

    from poorgrad_amd.program import DeviceProgram

    banner("concurrency: one program, four threads")
    w = workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24)
    program = DeviceProgram(w.tape, w.roots, numerics=hip.FAST)
    params = [torch.from_numpy(a).cuda() for a in w.initial]
    for slot, p in enumerate(params):
        program.bind_parameter(slot, p)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    program.run()
    torch.cuda.synchronize()
    want = {r.id: program.read(r) for r in w.roots}
    failures = []

    def worker(index):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for _ in range(5):
                    program.run()
                    got = program.read(w.loss)
                    if got.view(np.uint32) != want[w.loss.id].view(np.uint32):
                        failures.append((index, float(got), float(want[w.loss.id])))
        except Exception as e:  # noqa: BLE001 - reported below
            failures.append((index, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not failures, failures
    torch.cuda.synchronize()
    for r in w.roots:
        assert_bitwise(program.read(r), want[r.id], f"after threads: node {r.id}")


def test_device_face_split_products_from_four_threads(hip):
    import torch

    from poorgrad_amd import device

    banner("concurrency: device-face split products, four threads")
    # The last shape's partials (12 splits of 1024 x 1024) are larger than
    # any computed before the threads start, so the workspace regrows while
    # other threads' products are in flight; its reference is computed after.
    shapes = [(256, 4096, 256), (512, 4096, 512), (384, 8192, 256), (640, 2048, 512), (1024, 8192, 1024)]
    g = torch.Generator(device="cuda").manual_seed(3)
    operands = [(torch.randn(m, k, device="cuda", generator=g), torch.randn(k, n, device="cuda", generator=g))
                for m, k, n in shapes]
    alone = [device.gemm(a, b, hip.FAST) for a, b in operands[:-1]]
    torch.cuda.synchronize()
    alone = [x.cpu().numpy() for x in alone]
    results = {}
    failures = []

    def worker(index):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for rep in range(6):
                    which = (index + rep) % len(shapes)
                    a, b = operands[which]
                    got = device.gemm(a, b, hip.FAST)
                    stream.synchronize()
                    results.setdefault(which, []).append(got.cpu().numpy())
        except Exception as e:  # noqa: BLE001 - reported below
            failures.append((index, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not failures, failures
    a, b = operands[-1]
    alone.append(device.gemm(a, b, hip.FAST).cpu().numpy())
    assert len(results.get(len(shapes) - 1, [])) > 0
    for which, products in results.items():
        for got in products:
            assert_bitwise(got, alone[which], f"threaded product {shapes[which]}")
