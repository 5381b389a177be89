#!/usr/bin/env python3
"""Benchmark of the MI355X execution backend on BASELINE.json's configs.

The headline: one GPT-2-small train step per "step" —
the recorded-gradients program (forward, loss, every parameter's gradient:
12 layers, d_model 768, 12 heads, context 1024, batch 8, vocab 50257, tied
embeddings) run by libtopos_hip from its HBM arena, then AdamW (lr 3e-4,
betas 0.9/0.999, epsilon 1e-8, decay 0.01 on rank >= 2 parameters) on the
device-resident parameters. Token ids are uniform over the vocabulary,
weights N(0, 0.02): synthetic data, inputs resident before timing starts.
``value`` is train steps/s in the fast posture (matrix-core products,
envelope fidelity; elementwise work is bit-exact in every posture).

Measured beside it, each in its own section of the JSON line:
* ``mlp``: the 784-128-10 step with SGD lr 0.01, steps/s;
* ``gemm_sweep``: forward A.B plus A^T.G and G.B^T for the four
  (M,N,K), TFLOP/s per product and per sweep, fast and exact;
* ``chains``: SiLU + bias, LayerNorm, row sum/max/softmax on
  [16384, 4096], GB/s of algorithmic traffic (five back-to-back launches per
  event pair, queued behind reads of an unrelated 1 GiB buffer so no host
  gaps open between them and the operands start outside the last-level cache);
* ``llama``: the Llama-style decoder's forward + backward (8
  layers, d_model 2048, 16 heads of 128, SwiGLU 5632, seq 2048, batch 2,
  vocab 32000), ms per step and product TFLOP/s;
* ``gpt2_exact`` (configs[3], exact posture): the same program with
  bit-identical kernels, ms per forward + backward.

The roofline object describes the step's dominant kernel class (most time in
a profiled step, HIP events around every launch on the library's stream);
``cpu_baseline`` times the CPU oracle — a single-threaded restatement of the
topos interpreter — on a bounded sample of the same step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--quick]
       python bench.py --only {mlp,gemm,chains,llama,gpt2_exact} [--steps K] [--warmup W]   (one section alone)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "GPT-2-small train steps/s; fp32 GEMM TFLOP/s + fused-op GB/s as % of peak"
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix, published
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
SWEEP = [(512, 512, 512), (1024, 4096, 1024), (4096, 4096, 4096), (8192, 768, 3072)]
CHAIN_ROWS, CHAIN_COLUMNS = 16384, 4096
CHAIN_REPEAT = 5  # back-to-back launches per event pair in the chains section
CHAIN_BYTES = {  # each distinct input read once, each output written once, fp32
    "silu_bias": 4 * (2 * CHAIN_ROWS * CHAIN_COLUMNS + CHAIN_COLUMNS),
    "layer_norm": 4 * (2 * CHAIN_ROWS * CHAIN_COLUMNS + 2 * CHAIN_COLUMNS),
    "row_sum": 4 * (CHAIN_ROWS * CHAIN_COLUMNS + CHAIN_ROWS),
    "row_max": 4 * (CHAIN_ROWS * CHAIN_COLUMNS + CHAIN_ROWS),
    "row_softmax": 4 * (2 * CHAIN_ROWS * CHAIN_COLUMNS),
}
ADAMW = {"rate": 3e-4, "beta1": 0.9, "beta2": 0.999, "epsilon": 1e-8, "decay": 0.01}
# HBM bytes per product launch of the step, measured with rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE over one step's product launches, each counter
# scaled by what it reads for a 256 MiB copy (x2.0 and x1.0): the summary
# profiles/gpt2_train_step_traffic.md holds the commands and the figures. A
# counter run cannot happen inside this process, so the figure is carried.
MEASURED_PRODUCT_TRAFFIC_BYTES = 473.0 * 2**20


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle leg")
    p.add_argument("--quick", action="store_true", help="the GPT-2 step only (no side sections)")
    p.add_argument("--only", choices=["mlp", "gemm", "bf16", "chains", "llama", "gpt2_exact", "windows"],
                   help="run one side section alone and print its JSON (a diagnostic, not the bench line)")
    p.add_argument("--profile-out", help="write the profiled step's launches (one line each) to this file")
    p.add_argument("--calibration-copy-mib", type=int, default=0,
                   help="copy this many MiB device-to-device once before the step (a known-size kernel for "
                        "scaling hardware byte counters)")
    return p.parse_args()


def matmul_flops(tape, roots) -> float:
    """2*m*n*k (times the batch) over the products the program evaluates."""
    from poorgrad_amd import topos as t

    wanted = [False] * len(tape.nodes)
    for r in roots:
        wanted[r.id] = True
    for i in range(len(tape.nodes) - 1, -1, -1):
        if wanted[i]:
            node = tape.nodes[i]
            links = node.operands[:1] if node.op in (t.BROADCAST, t.BROADCAST_ALONG) else node.operands
            for link in links:
                wanted[link] = True
    total = 0.0
    for i, node in enumerate(tape.nodes):
        if wanted[i] and node.op == t.MATMUL:
            k = tape.nodes[node.operands[0]].shape[-1]
            total += 2.0 * math.prod(node.shape) * k
    return total


def time_steps(torch, step, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return time.perf_counter() - start


def breakdown(profile) -> dict:
    """Per launch kind: count, total ms, share, and achieved rate."""
    total = sum(ms for _, ms, _, _, _ in profile)
    kinds = {}
    for kind, ms, flops, nbytes, _ in profile:
        k = kinds.setdefault(kind, {"launches": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        k["launches"] += 1
        k["ms"] += ms
        k["flops"] += flops
        k["bytes"] += nbytes
    out = {}
    for kind, k in sorted(kinds.items(), key=lambda kv: -kv[1]["ms"]):
        entry = {"launches": k["launches"], "ms": round(k["ms"], 3), "share": round(k["ms"] / total, 4)}
        if k["flops"]:
            entry["TFLOP/s"] = round(k["flops"] / (k["ms"] / 1e3) / 1e12, 2)
        entry["GB/s"] = round(k["bytes"] / (k["ms"] / 1e3) / 1e9, 1)
        out[kind] = entry
    return out


def gpt2_section(torch, n, args) -> dict:
    from poorgrad_amd import workloads
    from poorgrad_amd.program import AdamW, DeviceProgram

    log("recording the GPT-2-small train step")
    t0 = time.perf_counter()
    w = workloads.gpt2()
    record_s = time.perf_counter() - t0
    log(f"recorded {len(w.tape.nodes)} nodes in {record_s:.1f}s; planning and compiling")
    t0 = time.perf_counter()
    program = DeviceProgram(w.tape, w.roots, numerics=n.FAST)
    plan_s = time.perf_counter() - t0
    info = program.info
    log(f"planned in {plan_s:.1f}s: {info}")
    params = [torch.from_numpy(a).cuda() for a in w.initial]
    for slot, p in enumerate(params):
        program.bind_parameter(slot, p)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    optimizer = AdamW(params, ADAMW["beta1"], ADAMW["beta2"], ADAMW["epsilon"], ADAMW["decay"])
    program.run()
    torch.cuda.synchronize()
    gradients = [program.pointer(g) for g in w.gradients]
    first_loss = float(program.read(w.loss))
    log(f"first loss {first_loss:.5f} (ln V = {math.log(w.config['vocab']):.5f})")

    def step():
        program.run()
        optimizer.step(params, gradients, ADAMW["rate"])

    log(f"timing {args.steps} steps after {args.warmup} warmup")
    wall = time_steps(torch, step, args.steps, args.warmup)
    last_loss = float(program.read(w.loss))
    log(f"{wall / args.steps * 1e3:.1f} ms/step; loss after {args.steps + args.warmup + 1} runs: {last_loss:.5f}")
    profile = program.profile()
    torch.cuda.synchronize()
    flops = matmul_flops(w.tape, w.roots)
    return {"wall": wall, "workload": w, "program": program, "profile": profile, "flops": flops,
            "record_s": record_s, "plan_s": plan_s, "info": info, "first_loss": first_loss, "last_loss": last_loss}


def roofline(profile) -> dict:
    kinds = breakdown(profile)
    dominant = next(iter(kinds))
    launches = [p for p in profile if p[0] == dominant]
    ms = sum(p[1] for p in launches)
    if dominant == "gemm":
        achieved = sum(p[2] for p in launches) / (ms / 1e3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 3), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                "traffic": round(MEASURED_PRODUCT_TRAFFIC_BYTES),
                "algorithmic_bytes_per_launch": round(sum(p[3] for p in launches) / len(launches)),
                "kernel": f"gemm_dma_kernel / gemm_mfma_kernel (with split_reduce_kernel): the step's "
                          f"{len(launches)} product launches, algorithmic 2*m*n*k over their event-timed duration",
                "ms_per_step": round(ms, 3)}
    achieved = sum(p[3] for p in launches) / (ms / 1e3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": f"{dominant}: the step's {len(launches)} launches", "ms_per_step": round(ms, 3)}


def cpu_sample() -> dict:
    """The oracle interpreter on one 64-token sequence of the GPT-2-small
    train step (full width, depth and vocabulary), in this process, which the
    caller has pinned to one core. Returns the seconds and the sample's
    product flops."""
    import numpy as np

    from oracle import interpreter
    from poorgrad_amd import workloads

    w = workloads.gpt2(batch=1, context=64)
    inputs = [None] * len(w.tape.input_shapes)
    for slot, (indices, one) in w.selection_inputs.items():
        inputs[slot] = interpreter.Sel(indices, w.tape.input_shapes[slot][1], one)
    start = time.perf_counter()
    with np.errstate(all="ignore"):
        interpreter.run(w.tape, w.roots, w.initial, inputs)
    seconds = time.perf_counter() - start
    return {"seconds": seconds, "flops": matmul_flops(w.tape, w.roots)}


def cpu_leg(full_flops: float) -> dict:
    """Times cpu_sample() in a child process pinned to one core (the
    reference interpreter is single-threaded), then extrapolates to the full
    step by the ratio of product flops (97% of the step's arithmetic)."""
    import subprocess

    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[0]
    code = ("import json, os, sys; sys.path.insert(0, %r); os.sched_setaffinity(0, {%d}); "
            "import bench; r = bench.cpu_sample(); r['affinity'] = sorted(os.sched_getaffinity(0)); "
            "print(json.dumps(r))" % (str(Path(__file__).resolve().parent), core))
    env = dict(os.environ, OMP_NUM_THREADS="1", OPENBLAS_NUM_THREADS="1", MKL_NUM_THREADS="1")
    child = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=900)
    if child.returncode != 0:
        raise RuntimeError(f"cpu leg failed: {child.stderr[-2000:]}")
    sample = json.loads(child.stdout.strip().splitlines()[-1])
    seconds, sample_flops = sample["seconds"], sample["flops"]
    step_seconds = seconds * full_flops / sample_flops
    return {"value": round(1.0 / step_seconds, 8), "unit": "steps/s", "cores": 1, "kind": "port",
            "host_cpus": os.cpu_count(), "allowed_cpus": len(allowed), "pinned_core": sample["affinity"],
            "sample": f"the interpreter restatement (oracle/) on the same GPT-2-small train step at batch 1, "
                      f"context 64 ({sample_flops / 1e9:.1f} GFLOP of products, {seconds:.1f} s on core "
                      f"{core} of {os.cpu_count()} host CPUs, one thread), scaled by product flops to the full "
                      f"step ({full_flops / 1e12:.2f} TFLOP): {step_seconds / 60:.1f} min per step"}


def mlp_section(torch, n, steps: int, warmup: int) -> dict:
    from poorgrad_amd import workloads
    from poorgrad_amd.program import DeviceProgram, sgd_step

    w = workloads.mlp()
    program = DeviceProgram(w.tape, w.roots, numerics=n.EXACT)
    params = [torch.from_numpy(a).cuda() for a in w.initial]
    for slot, p in enumerate(params):
        program.bind_parameter(slot, p)
    held = []
    for slot, a in w.dense_inputs.items():
        t = torch.from_numpy(a).cuda()
        held.append(t)
        program.bind_input(slot, t)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    program.run()
    gradients = [program.pointer(g) for g in w.gradients]

    def step(run):
        run()
        for p, g in zip(params, gradients):
            sgd_step(p, g, 0.01)

    reps = max(20, steps * 10)
    eager = time_steps(torch, lambda: step(program.run), reps, warmup)
    # The program as one captured HIP graph per step (the launches are a few
    # microseconds each, so host launch time dominates an eager step).
    wall = time_steps(torch, lambda: step(program.replay), reps, warmup)
    return {"steps/s": round(reps / wall, 2), "us_per_step": round(wall / reps * 1e6, 1),
            "eager_us_per_step": round(eager / reps * 1e6, 1), "program": "graph replay",
            "launches_per_step": program.info["launches"] + len(params), "posture": "exact (bit-identical)",
            "gflop_per_step": round(3 * matmul_flops(w.tape, [w.loss]) / 1e9, 4)}


def gpt2_exact_section(torch, n, steps: int, warmup: int) -> dict:
    """configs[3] in the exact posture: the same recorded-gradients program
    planned with bit-identical kernels (fixed-k-order products, ordered
    folds), forward + backward without the optimizer. Two runs must give the
    same loss bits."""
    from poorgrad_amd import workloads
    from poorgrad_amd.program import DeviceProgram

    w = workloads.gpt2()
    program = DeviceProgram(w.tape, w.roots, numerics=n.EXACT)
    params = [torch.from_numpy(a).cuda() for a in w.initial]
    for slot, p in enumerate(params):
        program.bind_parameter(slot, p)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    program.run()
    torch.cuda.synchronize()
    first = program.read(w.loss)
    reps = max(1, min(steps, 3))
    wall = time_steps(torch, program.run, reps, min(warmup, 1))
    again = program.read(w.loss)
    flops = matmul_flops(w.tape, w.roots)
    ms = wall / reps * 1e3
    return {"ms_per_step": round(ms, 2), "products_TFLOP/s": round(flops / (ms / 1e3) / 1e12, 2),
            "loss": float(first), "loss_bits_repeat": bool(first.tobytes() == again.tobytes()),
            "launches_per_step": program.info["launches"], "posture": "exact (bit-identical)"}


def llama_section(torch, n, steps: int, warmup: int) -> dict:
    """the Llama-style decoder's forward + backward (loss and every
    gradient; no optimizer) through the fast-posture program. Weights are drawn
    on the device (N(0, 0.02), torch generator seed 7; RMSNorm scales 1)."""
    from poorgrad_amd import workloads
    from poorgrad_amd.program import DeviceProgram

    w = workloads.llama(host_weights=False)
    t0 = time.perf_counter()
    program = DeviceProgram(w.tape, w.roots, numerics=n.FAST)
    plan_s = time.perf_counter() - t0
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    params = [torch.ones(shape, device="cuda") if len(shape) == 1 else
              torch.empty(shape, device="cuda").normal_(0.0, 0.02, generator=gen) for shape in w.initial]
    for slot, p in enumerate(params):
        program.bind_parameter(slot, p)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    program.run()
    torch.cuda.synchronize()
    loss = float(program.read(w.loss))
    wall = time_steps(torch, program.run, steps, warmup)
    profile = program.profile()
    flops = matmul_flops(w.tape, w.roots)
    ms = wall / steps * 1e3
    gemm = breakdown(profile).get("gemm", {})
    return {"config": w.config, "ms_per_step": round(ms, 2), "tflop_per_step_products": round(flops / 1e12, 3),
            "products_TFLOP/s": round(flops / (ms / 1e3) / 1e12, 2), "gemm": gemm,
            "launches_per_step": program.info["launches"], "arena_gib": round(program.info["arena_bytes"] / 2**30, 2),
            "plan_s": round(plan_s, 1), "loss": loss}


def event_times(torch, launches, steps: int, warmup: int, repeat: int = 1, lead=None) -> dict:
    """Seconds per launch of each labelled launch: per step, `repeat`
    back-to-back launches of it between two events (the labels interleave,
    so each is timed after the others have run). `lead`, when given, is
    enqueued before each group's first event: device work long enough that
    the group's launches are all queued before the device reaches them, so
    host launch time does not open gaps between them."""
    for _ in range(warmup):
        for _, fn in launches:
            fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    marks = []
    for _ in range(steps):
        for label, fn in launches:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            if lead is not None:
                lead()
            e0.record(stream)
            for _ in range(repeat):
                fn()
            e1.record(stream)
            marks.append((label, e0, e1))
    torch.cuda.synchronize()
    per = {}
    for label, e0, e1 in marks:
        per.setdefault(label, []).append(e0.elapsed_time(e1) / 1e3 / repeat)
    return {label: sum(v) / len(v) for label, v in per.items()}


def gemm_section(torch, n, steps: int, warmup: int) -> dict:
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    stream = torch.cuda.current_stream().cuda_stream
    products = []
    for (M, N, K) in SWEEP:
        A = torch.randn(M, K, device="cuda", generator=gen)
        B = torch.randn(K, N, device="cuda", generator=gen)
        G = torch.randn(M, N, device="cuda", generator=gen)
        shape = f"{M}x{N}x{K}"
        for label, a, ast, b, bst, m, k, n_ in (
                (f"forward {shape}", A, (K, 1), B, (N, 1), M, K, N),
                (f"a_t_g {shape}", A, (1, K), G, (N, 1), K, M, N),
                (f"g_b_t {shape}", G, (N, 1), B, (1, N), M, N, K)):
            out = torch.empty(m, n_, device="cuda")
            products.append((label, 2.0 * m * n_ * k, a, ast, b, bst, m, k, n_, out))
    result = {}
    # Each product queues behind a read of a 1 GiB buffer, so the host's
    # launch time (two launches for a split-k product) is not inside its
    # events: a 512-cube runs in a few microseconds of device time.
    busy = torch.ones(1 << 28, device="cuda")
    for posture, numerics in (("fast", n.FAST), ("exact", n.EXACT)):
        launches = []
        for label, _, a, ast, b, bst, m, k, n_, out in products:
            def fn(a=a, ast=ast, b=b, bst=bst, m=m, k=k, n_=n_, out=out):
                n.checked(n.lib.topos_hip_gemm_f32_device(a.data_ptr(), ast[0], ast[1], b.data_ptr(), bst[0], bst[1],
                                                          m, k, n_, numerics, out.data_ptr(), n_, stream), "gemm")
            launches.append((label, fn))
        reps = steps if posture == "fast" else max(1, min(steps, 3))
        per = event_times(torch, launches, reps, 1, lead=busy.sum)
        total_flops = sum(p[1] for p in products)
        total_s = sum(per.values())
        result[posture] = {
            "sweep_TFLOP/s": round(total_flops / total_s / 1e12, 2),
            "frac_of_fp32_peak": round(total_flops / total_s / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
            "products": {p[0]: round(p[1] / per[p[0]] / 1e12, 2) for p in products},
        }
    return result


def bf16_section(torch, n, steps: int, warmup: int) -> dict:
    """The sweep's products on bf16 operands (Bf16::gemm's contract: f32
    accumulation, one rounding), fast posture on the bf16 matrix cores,
    against MI355X's dense bf16 peak."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    stream = torch.cuda.current_stream().cuda_stream
    products = []
    for (M, N, K) in SWEEP:
        A = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16)
        B = torch.randn(K, N, device="cuda", generator=gen).to(torch.bfloat16)
        G = torch.randn(M, N, device="cuda", generator=gen).to(torch.bfloat16)
        shape = f"{M}x{N}x{K}"
        for label, a, ast, b, bst, m, k, n_ in (
                (f"forward {shape}", A, (K, 1), B, (N, 1), M, K, N),
                (f"a_t_g {shape}", A, (1, K), G, (N, 1), K, M, N),
                (f"g_b_t {shape}", G, (N, 1), B, (1, N), M, N, K)):
            out = torch.empty(m, n_, device="cuda", dtype=torch.bfloat16)
            products.append((label, 2.0 * m * n_ * k, a, ast, b, bst, m, k, n_, out))
    launches = []
    for label, _, a, ast, b, bst, m, k, n_, out in products:
        def fn(a=a, ast=ast, b=b, bst=bst, m=m, k=k, n_=n_, out=out):
            n.checked(n.lib.topos_hip_gemm_bf16_device(a.data_ptr(), ast[0], ast[1], b.data_ptr(), bst[0], bst[1],
                                                       m, k, n_, n.FAST, out.data_ptr(), n_, stream), "bf16 gemm")
        launches.append((label, fn))
    busy = torch.ones(1 << 28, device="cuda")
    per = event_times(torch, launches, steps, 1, lead=busy.sum)
    total_flops = sum(p[1] for p in products)
    total_s = sum(per.values())
    return {"sweep_TFLOP/s": round(total_flops / total_s / 1e12, 2),
            "frac_of_bf16_peak": round(total_flops / total_s / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
            "products": {p[0]: round(p[1] / per[p[0]] / 1e12, 2) for p in products}}


def chains_section(torch, n, steps: int, warmup: int) -> dict:
    import ctypes

    from poorgrad_amd import device

    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    x = torch.randn(CHAIN_ROWS, CHAIN_COLUMNS, device="cuda", generator=gen)
    b = torch.randn(CHAIN_COLUMNS, device="cuda", generator=gen)
    g = torch.randn(CHAIN_COLUMNS, device="cuda", generator=gen)
    one = torch.ones(1, device="cuda")
    y = torch.empty_like(x)
    stats = torch.empty(CHAIN_ROWS, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    lib = n.lib
    silu = device.Chain((CHAIN_ROWS, CHAIN_COLUMNS), [((CHAIN_COLUMNS, 1), 0), ((0, 1), 0), ((0, 0), 0)],
                        [(n.CHAIN_NEG, -1, 0), (n.CHAIN_EXP, 0, 0), (n.CHAIN_ADD, 1, -3), (n.CHAIN_DIV, -1, 2),
                         (n.CHAIN_ADD, 3, -2)], [4])
    ins = (ctypes.c_void_p * 3)(x.data_ptr(), b.data_ptr(), one.data_ptr())
    outs = (ctypes.c_void_p * 1)(y.data_ptr())

    def run_silu():
        n.checked(lib.topos_hip_chain_launch(silu._handle, ins, outs, stream), "silu chain")

    def rows(kind, out, numerics):
        return lambda: n.checked(lib.topos_hip_rows_f32_device(kind, x.data_ptr(), CHAIN_ROWS, CHAIN_COLUMNS, numerics,
                                                               out.data_ptr(), stream), "rows")

    def layer_norm(numerics):
        return lambda: n.checked(lib.topos_hip_layer_norm_f32_device(x.data_ptr(), CHAIN_ROWS, CHAIN_COLUMNS,
                                                                     g.data_ptr(), b.data_ptr(), 1e-5, numerics,
                                                                     y.data_ptr(), stream), "layer norm")

    # Reference points for what this device moves on the same tensor: a plain
    # read + write (torch's copy) and a generated chain with one addition
    # (x + b), against which the SiLU + bias chain, also one read and one
    # write per element, is measured; the fast row sum is the read-only one.
    add_bias = device.Chain((CHAIN_ROWS, CHAIN_COLUMNS), [((CHAIN_COLUMNS, 1), 0), ((0, 1), 0)],
                            [(n.CHAIN_ADD, -1, -2)], [0])

    def run_add_bias():
        n.checked(lib.topos_hip_chain_launch(add_bias._handle, ins, outs, stream), "add chain")

    launches = [("silu_bias", run_silu), ("reference_copy", lambda: y.copy_(x)), ("reference_add_bias", run_add_bias)]
    bytes_of = {"silu_bias": CHAIN_BYTES["silu_bias"], "reference_copy": 8 * CHAIN_ROWS * CHAIN_COLUMNS,
                "reference_add_bias": CHAIN_BYTES["silu_bias"]}
    for posture, numerics in (("exact", n.EXACT), ("fast", n.FAST)):
        for name, fn in (("layer_norm", layer_norm(numerics)), ("row_sum", rows(n.ROWS_SUM, stats, numerics)),
                         ("row_max", rows(n.ROWS_MAX, stats, numerics)),
                         ("row_softmax", rows(n.ROWS_SOFTMAX, y, numerics))):
            launches.append((f"{name}/{posture}", fn))
            bytes_of[f"{name}/{posture}"] = CHAIN_BYTES[name]
    # Each group of launches queues behind two reads of a 1 GiB buffer (about
    # 0.3 ms of device work that writes nothing back and leaves the 256 MB
    # last-level cache holding that buffer, not the chain's operands).
    busy = torch.ones(1 << 28, device="cuda")
    per = event_times(torch, launches, steps, warmup, repeat=CHAIN_REPEAT, lead=lambda: (busy.sum(), busy.sum()))
    return {label: {"us": round(t * 1e6, 1), "GB/s": round(bytes_of[label] / t / 1e9, 1),
                    "frac": round(bytes_of[label] / t / 1e9 / HBM_PEAK_GBS, 4)} for label, t in per.items()}


def windows_section(torch, n, steps: int, warmup: int) -> dict:
    """The reference's pattern bench (benches/pattern.rs:22-107) as device
    programs — max_pool over [64,32,28,28], conv2d [64,16,14,14] x
    [32,16,3,3] padding 1, BatchNorm over [256,512] — and the MNIST example's
    convolutional train step (examples/mnist/main.rs, batch 64, forward and
    recorded gradients), each timed as one program run, in both postures."""
    import numpy as np

    from poorgrad_amd import topos as t
    from poorgrad_amd import workloads
    from poorgrad_amd.program import DeviceProgram

    def fill(count, multiplier, modulus, shift, scale):
        index = np.arange(count, dtype=np.int64)
        return (((index * multiplier) % modulus).astype(np.float32) - np.float32(shift)) / np.float32(scale)

    def pattern(kind):
        tape = t.Tape()
        if kind == "pool":
            x = tape.input((64, 32, 28, 28))
            return tape, [t.max_pool(x, 2, 2)], {x.node.slot: fill(64 * 32 * 28 * 28, 5, 13, 6.0, 4.0).reshape(x.shape)}
        if kind == "conv":
            x = tape.input((64, 16, 14, 14))
            w = tape.input((32, 16, 3, 3))
            out = t.conv2d(x, w, tape.leaf(t.Constant((32,), 0.01)), 1, 1)
            return tape, [out], {x.node.slot: fill(64 * 16 * 14 * 14, 7, 23, 11.0, 8.0).reshape(x.shape),
                                 w.node.slot: fill(32 * 16 * 9, 3, 17, 8.0, 16.0).reshape(w.shape)}
        x = tape.input((256, 512))
        out, _, _ = t.batch_norm(x, tape.leaf(t.Constant((512,), 1.0)), tape.leaf(t.Constant((512,), 0.0)),
                                 tape.leaf(t.Constant((1,), 1e-5)))
        return tape, [out], {x.node.slot: fill(256 * 512, 11, 29, 14.0, 8.0).reshape(x.shape)}

    result = {}
    reps = max(20, steps * 10)
    for posture, numerics in (("exact", n.EXACT), ("fast", n.FAST)):
        for kind in ("pool", "conv", "batch_norm", "mnist_step"):
            if kind == "mnist_step":
                w = workloads.cnn()
                program = DeviceProgram(w.tape, w.roots, numerics=numerics)
                held = [torch.from_numpy(a).cuda() for a in w.initial]
                for slot, p in enumerate(held):
                    program.bind_parameter(slot, p)
                feeds = w.dense_inputs
                for slot, (indices, one) in w.selection_inputs.items():
                    program.bind_selection(slot, indices, one)
            else:
                tape, roots, feeds = pattern(kind)
                program = DeviceProgram(tape, roots, numerics=numerics)
                held = []
            for slot, a in feeds.items():
                tensor = torch.from_numpy(np.ascontiguousarray(a)).cuda()
                held.append(tensor)
                program.bind_input(slot, tensor)
            program.run()
            wall = time_steps(torch, program.replay, reps, warmup)
            result[f"{kind}/{posture}"] = {"us": round(wall / reps * 1e6, 1), "launches": program.info["launches"]}
            del program, held
    return result


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the value is one MI355X's throughput at --gpus 1", file=sys.stderr)
        return 2
    import torch

    from poorgrad_amd import _native as n

    if n.status() != n.OK:
        print(f"HIP backend unavailable: {n.status_reason()}", file=sys.stderr)
        return 1
    if args.calibration_copy_mib:
        count = args.calibration_copy_mib * (1 << 20) // 4
        source = torch.ones(count, device="cuda")
        torch.empty_like(source).copy_(source)
        torch.cuda.synchronize()
        del source
    if args.only:
        sections = {"mlp": mlp_section, "gemm": gemm_section, "bf16": bf16_section, "chains": chains_section,
                    "llama": llama_section, "gpt2_exact": gpt2_exact_section, "windows": windows_section}
        print(json.dumps({args.only: sections[args.only](torch, n, args.steps, args.warmup)}), flush=True)
        return 0
    g = gpt2_section(torch, n, args)
    ms_per_step = g["wall"] / args.steps * 1e3
    line = {
        "metric": METRIC,
        "value": round(args.steps / g["wall"], 4),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: token ids uniform over the vocabulary (splitmix64 seed 13), weights N(0, 0.02)",
        "config": {"workload": "gpt2_small_train_step (BASELINE configs[3]): recorded-gradients program + AdamW "
                               "on device, fast posture",
                   "layers": 12, "d_model": 768, "heads": 12, "context": 1024, "batch": 8, "vocab": 50257,
                   "optimizer": dict(ADAMW), "tflop_per_step_products": round(g["flops"] / 1e12, 3),
                   "nodes": len(g["workload"].tape.nodes), "launches_per_step": g["info"]["launches"],
                   "arena_gib": round(g["info"]["arena_bytes"] / 2**30, 2),
                   "plan_s": round(g["plan_s"], 1)},
        "roofline": roofline(g["profile"]),
        "cpu_baseline": None,
        "step_breakdown": breakdown(g["profile"]),
        "products_TFLOP/s": round(g["flops"] / (ms_per_step / 1e3) / 1e12, 2),
        "loss": {"first": g["first_loss"], "after_steps": g["last_loss"]},
    }
    full_flops = g["flops"]
    if args.profile_out:
        with open(args.profile_out, "w") as f:
            for i, (kind, ms, flops, nbytes, what) in enumerate(g["profile"]):
                rate = f"{flops / ms / 1e9:.1f} TFLOP/s" if flops else f"{nbytes / ms / 1e6:.0f} GB/s"
                f.write(f"{i}\t{kind}\t{ms * 1e3:.1f} us\t{rate}\t{what}\n")
    del g
    if not args.quick:
        log("mlp step (configs[0])")
        line["mlp"] = mlp_section(torch, n, args.steps, args.warmup)
        log("gemm sweep (configs[1])")
        line["gemm_sweep"] = gemm_section(torch, n, args.steps, args.warmup)
        log("bf16 products (configs[1] shapes on bf16 operands)")
        line["gemm_sweep_bf16"] = bf16_section(torch, n, args.steps, args.warmup)
        log("chains (configs[2])")
        line["chains"] = chains_section(torch, n, args.steps, args.warmup)
        log("llama forward + backward (configs[4])")
        line["llama"] = llama_section(torch, n, args.steps, args.warmup)
        log("gpt2 step, exact posture (configs[3])")
        line["gpt2_exact"] = gpt2_exact_section(torch, n, args.steps, args.warmup)
        log("window programs (the reference's pattern bench, the MNIST convolutional step)")
        line["windows"] = windows_section(torch, n, args.steps, args.warmup)
    if not args.no_cpu_baseline:
        log("cpu baseline: the oracle interpreter on one core")
        line["cpu_baseline"] = cpu_leg(full_flops)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
