#!/usr/bin/env python3
"""Benchmark of the MI355X execution backend on BASELINE.json's configs.

A step is one pass of the hot path over one batch of synthetic input already
resident in HBM:

* ``gemm_sweep`` (configs[1], the default workload): the fp32 product sweep
  through the graph matmul, forward plus both backward products
  (A.B, A^T.G, G.B^T, src/function/matmul.rs:71-91) for (M,N,K) in
  {(512,512,512), (1024,4096,1024), (4096,4096,4096), (8192,768,3072)};
  the transposed operands are stride views, never copies. ``value`` is the
  sweep's TFLOP/s in the fast (matrix-core) posture.
* ``chains`` are measured beside it on x:[16384,4096]:
  SiLU + bias, LayerNorm, row sum, row max and row softmax, as GB/s of
  algorithmic traffic (each distinct input read once, each output written
  once) against the 8 TB/s HBM peak.

The roofline object describes the dominant kernel (the launch class that takes
the most time in the timed region), timed with HIP events on the stream the
library launches on. The CPU baseline times the CPU oracle (a single-threaded
restatement of the topos interpreter's arithmetic, the reference's own
single-threaded CPU path) on a bounded sample of the same sweep on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "GPT-2-small train steps/s; fp32 GEMM TFLOP/s + fused-op GB/s as % of peak"
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
SWEEP = [(512, 512, 512), (1024, 4096, 1024), (4096, 4096, 4096), (8192, 768, 3072)]
CHAIN_ROWS, CHAIN_COLUMNS = 16384, 4096
# Algorithmic bytes per launch: each distinct input read once, each output
# written once, fp32.
CHAIN_BYTES = {
    "silu_bias": 4 * (2 * CHAIN_ROWS * CHAIN_COLUMNS + CHAIN_COLUMNS),
    "layer_norm": 4 * (2 * CHAIN_ROWS * CHAIN_COLUMNS + 2 * CHAIN_COLUMNS),
    "row_sum": 4 * (CHAIN_ROWS * CHAIN_COLUMNS + CHAIN_ROWS),
    "row_max": 4 * (CHAIN_ROWS * CHAIN_COLUMNS + CHAIN_ROWS),
    "row_softmax": 4 * (2 * CHAIN_ROWS * CHAIN_COLUMNS),
}


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=30)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle leg")
    p.add_argument("--no-chains", action="store_true", help="time the GEMM sweep only")
    p.add_argument("--cpu-fraction", type=float, default=1.0 / 16,
                   help="share of each sweep product's output rows the CPU leg computes")
    return p.parse_args()


class Products:
    """The sweep's operands in HBM and its twelve products as launch closures."""

    def __init__(self, torch, n, seed: int = 7):
        self.torch, self.n = torch, n
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        self.entries = []  # (label, m, k, n, launch(numerics))
        self.host = []     # for the CPU leg: (label, a, a_strides, b, b_strides, m, k, n) lazily
        for (M, N, K) in SWEEP:
            A = torch.randn(M, K, device="cuda", generator=gen)
            B = torch.randn(K, N, device="cuda", generator=gen)
            G = torch.randn(M, N, device="cuda", generator=gen)
            C = torch.empty(M, N, device="cuda")
            dA = torch.empty(K, N, device="cuda")  # A^T . G  (K x N)
            dB = torch.empty(M, K, device="cuda")  # G . B^T  (M x K)
            shape = f"{M}x{N}x{K}"
            # forward: (M,N,K), A (K,1), B (N,1)
            self._add(f"forward {shape}", A, (K, 1), B, (N, 1), M, K, N, C)
            # A^T . G: left = A^T [K x M] strides (1, K); right = G [M x N]
            self._add(f"a_t_g {shape}", A, (1, K), G, (N, 1), K, M, N, dA)
            # G . B^T: left = G [M x N]; right = B^T [N x K] strides (1, N)
            self._add(f"g_b_t {shape}", G, (N, 1), B, (1, N), M, N, K, dB)

    def _add(self, label, a, a_st, b, b_st, m, k, n_, out):
        lib, stream = self.n.lib, self.torch.cuda.current_stream().cuda_stream

        def launch(numerics, a=a, b=b, out=out):
            code = lib.topos_hip_gemm_f32_device(a.data_ptr(), a_st[0], a_st[1], b.data_ptr(), b_st[0], b_st[1],
                                                 m, k, n_, numerics, out.data_ptr(), n_, stream)
            if code != self.n.OK:
                raise self.n.HipError(code, f"gemm {label}")

        self.entries.append((label, m, k, n_, launch))
        self.host.append((label, a, a_st, b, b_st, m, k, n_))

    @property
    def flops(self) -> float:
        return sum(2.0 * m * k * n_ for _, m, k, n_, _ in self.entries)


def time_launches(torch, launches, steps: int, warmup: int):
    """Runs `steps` timed passes over `launches` (label, flops_or_bytes, fn),
    bracketing each launch with HIP events on the current stream. Returns the
    wall time of the timed region (s) and per-label mean launch time (s)."""
    for _ in range(warmup):
        for _, _, fn in launches:
            fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    marks = []
    start = time.perf_counter()
    for _ in range(steps):
        for label, _, fn in launches:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            marks.append((label, e0, e1))
    torch.cuda.synchronize()
    wall = time.perf_counter() - start
    per = {}
    for label, e0, e1 in marks:
        per.setdefault(label, []).append(e0.elapsed_time(e1) / 1e3)
    return wall, {label: sum(v) / len(v) for label, v in per.items()}


def cpu_leg(products, fraction: float) -> dict:
    """The CPU oracle on a bounded sample: the first `fraction` of every sweep
    product's output rows (rows are independent, bit-identical to the whole
    product), one core."""
    import numpy as np

    import oracle

    flops, seconds = 0.0, 0.0
    for label, a, a_st, b, b_st, m, k, n_ in products.host:
        ah = a.cpu().numpy().ravel()
        bh = b.cpu().numpy().ravel()
        rows = max(1, int(round(m * fraction)))
        t0 = time.perf_counter()
        oracle.gemm(ah, a_st, bh, b_st, m, k, n_, rows=(0, rows))
        seconds += time.perf_counter() - t0
        flops += 2.0 * rows * k * n_
        del ah, bh
    _ = np
    return {"value": flops / seconds / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"first {fraction:.4g} of the output rows of each of the 12 sweep products "
                      f"({flops / 1e9:.1f} GFLOP, {seconds:.1f} s), exact fixed-k-order arithmetic, "
                      f"single thread (the reference library has no threads)"}


def chains(torch, n, device, steps: int, warmup: int) -> dict:
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
    # x / (exp(-x) + 1) + b (examples/llama/model.rs:258 plus a bias broadcast along axis 0)
    silu = device.Chain((CHAIN_ROWS, CHAIN_COLUMNS), [((CHAIN_COLUMNS, 1), 0), ((0, 1), 0), ((0, 0), 0)],
                        [(n.CHAIN_NEG, -1, 0), (n.CHAIN_EXP, 0, 0), (n.CHAIN_ADD, 1, -3), (n.CHAIN_DIV, -1, 2),
                         (n.CHAIN_ADD, 3, -2)], [4])
    import ctypes

    ins = (ctypes.c_void_p * 3)(x.data_ptr(), b.data_ptr(), one.data_ptr())
    outs = (ctypes.c_void_p * 1)(y.data_ptr())

    def run_silu():
        n.checked(lib.topos_hip_chain_launch(silu._handle, ins, outs, stream), "silu chain")

    def rows(kind, out, numerics):
        def fn():
            n.checked(lib.topos_hip_rows_f32_device(kind, x.data_ptr(), CHAIN_ROWS, CHAIN_COLUMNS, numerics,
                                                    out.data_ptr(), stream), "rows")
        return fn

    def layer_norm(numerics):
        def fn():
            n.checked(lib.topos_hip_layer_norm_f32_device(x.data_ptr(), CHAIN_ROWS, CHAIN_COLUMNS, g.data_ptr(),
                                                          b.data_ptr(), 1e-5, numerics, y.data_ptr(), stream),
                      "layer norm")
        return fn

    launches = [("silu_bias", CHAIN_BYTES["silu_bias"], run_silu)]
    for posture, numerics in (("exact", n.EXACT), ("fast", n.FAST)):
        launches += [
            (f"layer_norm/{posture}", CHAIN_BYTES["layer_norm"], layer_norm(numerics)),
            (f"row_sum/{posture}", CHAIN_BYTES["row_sum"], rows(n.ROWS_SUM, stats, numerics)),
            (f"row_max/{posture}", CHAIN_BYTES["row_max"], rows(n.ROWS_MAX, stats, numerics)),
            (f"row_softmax/{posture}", CHAIN_BYTES["row_softmax"], rows(n.ROWS_SOFTMAX, y, numerics)),
        ]
    _, per = time_launches(torch, launches, steps, warmup)
    out = {}
    for label, nbytes, _ in launches:
        t = per[label]
        gbs = nbytes / t / 1e9
        out[label] = {"us": round(t * 1e6, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                      "bytes": nbytes}
    return out


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the value is one MI355X's throughput at --gpus 1", file=sys.stderr)
        return 2
    import torch

    from poorgrad_amd import _native as n
    from poorgrad_amd import device

    if n.status() != n.OK:
        print(f"HIP backend unavailable: {n.status_reason()}", file=sys.stderr)
        return 1
    products = Products(torch, n)
    fast = [(label, 2.0 * m * k * n_, (lambda fn=fn: fn(n.FAST))) for label, m, k, n_, fn in products.entries]
    exact = [(label, 2.0 * m * k * n_, (lambda fn=fn: fn(n.EXACT))) for label, m, k, n_, fn in products.entries]
    print(f"[bench] gemm sweep fast: {args.steps} steps after {args.warmup} warmup", file=sys.stderr, flush=True)
    wall, per = time_launches(torch, fast, args.steps, args.warmup)
    sweep_flops = products.flops
    value = sweep_flops * args.steps / wall / 1e12
    # Dominant launch class: the most time in the timed region.
    label, flops, _ = max(fast, key=lambda e: per[e[0]])
    achieved = flops / per[label] / 1e12
    per_product = {lab: {"us": round(per[lab] * 1e6, 1), "TFLOP/s": round(f / per[lab] / 1e12, 2)}
                   for lab, f, _ in fast}
    print("[bench] gemm sweep exact", file=sys.stderr, flush=True)
    exact_steps = max(1, min(args.steps, 5))
    exact_wall, exact_per = time_launches(torch, exact, exact_steps, 1)
    exact_value = sweep_flops * exact_steps / exact_wall / 1e12
    chain_results = None
    if not args.no_chains:
        print("[bench] chains", file=sys.stderr, flush=True)
        chain_results = chains(torch, n, device, args.steps, args.warmup)
    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline (oracle, one core)", file=sys.stderr, flush=True)
        cpu = cpu_leg(products, args.cpu_fraction)
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "gemm_sweep (BASELINE configs[1]): forward A.B plus A^T.G and G.B^T as stride "
                               "views, fast (matrix-core) posture, A,B,G ~ N(0,1)",
                   "shapes_mnk": SWEEP, "products_per_step": len(fast), "gflop_per_step": round(sweep_flops / 1e9, 3)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": f"gemm_mfma_kernel ({label})", "us_per_launch": round(per[label] * 1e6, 2)},
        "cpu_baseline": cpu,
        "gemm_products": per_product,
        "exact_sweep": {"TFLOP/s": round(exact_value, 3), "frac_of_fp32_peak": round(exact_value / FP32_MFMA_PEAK_TFLOPS, 4),
                        "per_product_us": {lab: round(t * 1e6, 1) for lab, t in exact_per.items()}},
        "chains": chain_results,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
