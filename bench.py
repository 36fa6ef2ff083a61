#!/usr/bin/env python
"""Benchmark of the quantized-weight matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--no-cpu]

Workload (one "step"): one EXL3 dense linear at the decode-GEMV shape, a
4096 x 14336 matrix at 4 bits per weight (bits_x2 8, mul1 codebook), M = 1
fp16 activation row ~N(0,1), fp16 output; seeded uniform trellis words,
suh / svh = +-1 x N(1, 0.05).  Twelve distinct weight copies (353 MB, more
than the 256 MB Infinity Cache) are used round-robin so every step streams
its weights from HBM.  The K timed steps run as replays of a HIP graph of
back-to-back calls, timed with HIP events on the stream they run on.

value = algorithmic bytes per step / time per step, in GB/s, where the bytes
are the packed weights + suh/svh + activations + output
(K*N*bits/8 + 2(K+N) + 2MK + 2MN).  roofline.achieved is the same figure
for the dominant kernel (see DESIGN.md for how it relates to the rocprof
trace), against the 8 TB/s HBM peak.

cpu_baseline: the reference's CPU dequantize-then-matmul path (LUT decode of
every tile, FP64 block Hadamards, FP64 matmul; oracle/exl3_torch_ref.py) on
the same matrix shape, timed on this host's cores for about --cpu-seconds.

Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vllm-cmp170hx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "EXL3 M=1 GEMV HBM GB/s (% peak); int4 MoE tokens/s + MFMA util at 256 tok"
HBM_PEAK_GBS = 8000.0
K_IN, N_OUT, BITS_X2, CODEBOOK, ROWS = 4096, 14336, 8, 2, 1
COPIES = 12
GRAPH_CALLS = 120


def gemv_bytes(k: int, n: int, bits_x2: int, rows: int) -> int:
    return k * n * bits_x2 // 16 + 2 * (k + n) + 2 * rows * k + 2 * rows * n


def make_matrix(torch, gen, device, k, n, bits_x2):
    trellis = torch.randint(-(2 ** 15), 2 ** 15, (k // 16, n // 16, 8 * bits_x2), dtype=torch.int16,
                            device=device, generator=gen)

    def scales(size):
        sign = torch.randint(0, 2, (size,), device=device, generator=gen).float() * 2 - 1
        mag = 1.0 + 0.05 * torch.randn(size, device=device, generator=gen)
        return (sign * mag).half()

    return trellis, scales(k), scales(n)


def gpu_gemv(args, torch):
    from vllm_mi355x.kernels.exl3 import ops

    ops.ensure_extension()
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device)
    gen.manual_seed(1234)
    mats = [make_matrix(torch, gen, device, K_IN, N_OUT, BITS_X2) for _ in range(COPIES)]
    x = torch.randn(ROWS, K_IN, device=device, generator=gen).half()
    out = torch.empty(ROWS, N_OUT, dtype=torch.float16, device=device)
    ws = torch.empty(ops.linear_workspace_size(ROWS, K_IN, N_OUT), dtype=torch.float32, device=device)

    def call(i):
        t, suh, svh = mats[i % COPIES]
        ops.linear_out(x, t, suh, svh, BITS_X2, CODEBOOK, K_IN, N_OUT, out, ws)

    for i in range(COPIES):  # eager warm-up (loads the library, first launches)
        call(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(GRAPH_CALLS):
                call(i)
    torch.cuda.synchronize()
    warm_reps = max(1, -(-args.warmup // GRAPH_CALLS))
    reps = max(1, -(-args.steps // GRAPH_CALLS))
    with torch.cuda.stream(stream):
        for _ in range(warm_reps):
            graph.replay()
        stream.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(reps):
            graph.replay()
        end.record(stream)
        end.synchronize()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    steps = reps * GRAPH_CALLS
    return total_ms / steps, steps, warm_reps * GRAPH_CALLS


def cpu_baseline(seconds: float, torch):
    from oracle.exl3_torch_ref import DenseDecoder, linear_fp64

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(99)
    trellis = torch.randint(-(2 ** 15), 2 ** 15, (K_IN // 16, N_OUT // 16, 8 * BITS_X2),
                            dtype=torch.int16, generator=g)
    suh = torch.randn(K_IN, generator=g).half()
    svh = torch.randn(N_OUT, generator=g).half()
    x = torch.randn(ROWS, K_IN, generator=g).half()
    dec = DenseDecoder(BITS_X2, CODEBOOK)
    linear_fp64(dec, x, trellis, suh, svh, N_OUT)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        linear_fp64(dec, x, trellis, suh, svh, N_OUT)
        times.append(time.perf_counter() - t0)
    per_call = statistics.median(times)
    gbs = gemv_bytes(K_IN, N_OUT, BITS_X2, ROWS) / per_call / 1e9
    return {
        "value": round(gbs, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} calls (median {per_call * 1e3:.1f} ms) of the {K_IN}x{N_OUT} "
                   "4-bit mul1 M=1 linear via the reference's CPU path restated in torch "
                   "(65536-entry LUT decode of every tile, FP64 block H128, FP64 matmul)"),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=1200)
    parser.add_argument("--warmup", type=int, default=120)
    parser.add_argument("--cpu-seconds", type=float, default=15.0)
    parser.add_argument("--no-cpu", action="store_true")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the hot path is a single-GPU kernel; see DESIGN.md for how it would shard)",
              file=sys.stderr)
        return 2

    import torch

    ms, steps, warm = gpu_gemv(args, torch)
    nbytes = gemv_bytes(K_IN, N_OUT, BITS_X2, ROWS)
    gbs = nbytes / (ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": (f"exl3_linear GEMV {K_IN}x{N_OUT} bits_x2={BITS_X2} mul1 M={ROWS} "
                         "fp16 in/out"),
            "k": K_IN, "n": N_OUT, "bits_per_weight": BITS_X2 / 2, "codebook": "mul1",
            "rows": ROWS, "weight_copies": COPIES, "bytes_per_step": nbytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds, torch)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
