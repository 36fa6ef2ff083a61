#!/usr/bin/env python
"""Benchmark of the quantized-weight matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--no-cpu]
                    [--no-extras] [--only prefill|exl3_moe|marlin|moe_prefill] [--copy-mb MB]

Headline workload (one "step"): one EXL3 dense linear at the decode-GEMV
shape, a 4096 x 14336 matrix at 4 bits per weight (bits_x2 8, mul1
codebook), M = 1 fp16 activation row ~N(0,1), fp16 output; seeded uniform
trellis words, suh / svh = +-1 x N(1, 0.05).  Twelve distinct weight copies
(353 MB, more than the 256 MB Infinity Cache) are used round-robin so every
step streams its weights from HBM.  Exactly --warmup untimed steps run
first, then exactly --steps timed steps as replays of HIP graphs of
back-to-back calls (uploaded before the timed region), timed with HIP
events on the stream they run on.  The other workloads of the line run
before the headline, so the GPU is at its sustained clock when the timed
steps start (from a cold start the first ~20 ms run ~2.5% slower).

value = algorithmic bytes per step / time per step, in GB/s, where the bytes
are the packed weights + suh/svh + activations + output
(K*N*bits/8 + 2(K+N) + 2MK + 2MN).  roofline.achieved is that figure per
launch of the one kernel a step runs (the fused GEMV and finish), against
the 8 TB/s HBM peak; roofline.traffic is the HBM bytes per launch measured
with rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's readings,
read from the committed profile summary when it is there.

The same line also carries:
  int4_moe   the Marlin-format int4 fused MoE (128 experts, hidden 2048,
             intermediate 768, top-8, fp16, |N(0,0.02)| group-128 scales,
             router logits ~N(0,1) -> softmax top-8) at 1, 16, 64 and 256
             tokens: tokens/s, HBM GB/s over the touched experts' bytes,
             and MFMA utilisation against the 2.5 PFLOP/s fp16 peak;
  exl3_gemv_configs  the same linear at M = 4 and 8, at 3 and 2 bits per
             weight, and the transposed 14336 x 4096 matrix: GB/s;
  exl3_prefill  the 8192 x 28672 4-bit linear at M = 2048 (and 512, 8192):
             TFLOP/s;
  exl3_moe   the 3-bit EXL3 MoE (256 routed experts + 1 shared, hidden
             7168, intermediate 2048, top-8 from Zipf(1.1)-skewed logits)
             at 64 decode tokens (and 2048 prefill tokens): tokens/s and
             HBM GB/s;
  exl3_moe_prefill  moe_out_prefill's served configuration (256 experts,
             hidden 2560, intermediate 640, bits_x2 10, top-10, bf16) at
             2048 tokens (and 65, 512, 3460), beside the run-time-format
             moe_out on the same call;
  (the many-row EXL3 lines at the default FP16 high + low activation
  parts, and again with the FP16-only opt-in)
and the CPU baselines: the reference's CPU dequantize-then-matmul paths
(oracle/exl3_torch_ref.py, oracle/marlin_torch_ref.py) on this host's
cores, each on a bounded sample of its workload.

Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vllm-cmp170hx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "EXL3 M=1 GEMV HBM GB/s (% peak); int4 MoE tokens/s + MFMA util at 256 tok"
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
K_IN, N_OUT, BITS_X2, CODEBOOK, ROWS = 4096, 14336, 8, 2, 1
COPIES = 12
GRAPH_CALLS = 120
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "exl3_gemv_4096x14336_4bit_m1_traffic.md")


def gemv_bytes(k: int, n: int, bits_x2: int, rows: int) -> int:
    return k * n * bits_x2 // 16 + 2 * (k + n) + 2 * rows * k + 2 * rows * n


def make_matrix(torch, gen, device, k, n, bits_x2, scales="sign"):
    """Seeded trellis words and scales: "sign" = +-1 x N(1, 0.05) (the
    benchmark description), "test" = suh ~ N(0, 1), svh ~ 0.05 N(0, 1) (the
    reference's tests, test_exl3_kernels.py:174-180)."""
    trellis = torch.randint(-(2 ** 15), 2 ** 15, (k // 16, n // 16, 8 * bits_x2), dtype=torch.int16,
                            device=device, generator=gen)

    def sign_scales(size):
        sign = torch.randint(0, 2, (size,), device=device, generator=gen).float() * 2 - 1
        mag = 1.0 + 0.05 * torch.randn(size, device=device, generator=gen)
        return (sign * mag).half()

    if scales == "test":
        return (trellis, torch.randn(k, device=device, generator=gen).half(),
                (0.05 * torch.randn(n, device=device, generator=gen)).half())
    return trellis, sign_scales(k), sign_scales(n)


def _hip_graph_upload(torch, graph, stream) -> None:
    """hipGraphUpload of a captured graph's executable: its first replay in
    a timed region then pays no upload."""
    import ctypes
    lib = ctypes.CDLL("libamdhip64.so")
    lib.hipGraphUpload.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.hipGraphUpload.restype = ctypes.c_int
    rc = lib.hipGraphUpload(ctypes.c_void_p(graph.raw_cuda_graph_exec()), ctypes.c_void_p(stream.cuda_stream))
    if rc != 0:
        raise RuntimeError(f"hipGraphUpload failed ({rc})")


def time_steps_exact(torch, calls, warmup, steps, per_graph=120):
    """ms per call over exactly `steps` timed calls after exactly `warmup`
    untimed ones.  The first warm-up call runs eagerly (the library's first
    launches), the others as one graph replayed before the timed region;
    the timed calls are replays of a graph of per_graph calls plus one graph
    of the remainder, all graphs uploaded first.  HIP events on the replay
    stream bracket the timed replays."""
    if warmup > 0:
        calls(0)
    torch.cuda.synchronize()
    per_graph = max(1, min(per_graph, steps))
    full, rem = divmod(steps, per_graph)
    stream = torch.cuda.Stream()

    def capture(first, size):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for i in range(first, first + size):
                    calls(i)
        return graph

    warm = capture(1, warmup - 1) if warmup > 1 else None
    timed = [(capture(warmup, per_graph), full)] if full else []
    if rem:
        timed.append((capture(warmup, rem), 1))
    torch.cuda.synchronize()
    for graph in ([warm] if warm is not None else []) + [g for g, _ in timed]:
        _hip_graph_upload(torch, graph, stream)
    stream.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        if warm is not None:
            warm.replay()
        start.record(stream)
        for graph, reps in timed:
            for _ in range(reps):
                graph.replay()
        end.record(stream)
        end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_graph(torch, calls, per_graph, warmup, steps):
    """(ms per call, timed calls, warm-up calls): calls(i) captured
    per_graph times in a HIP graph, replayed; HIP events on the replay
    stream bracket the timed replays."""
    for i in range(min(per_graph, 4)):  # eager warm-up (loads the library, first launches)
        calls(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(per_graph):
                calls(i)
    torch.cuda.synchronize()
    warm_reps = max(1, -(-warmup // per_graph))
    reps = max(1, -(-steps // per_graph))
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
    return start.elapsed_time(end) / (reps * per_graph), reps * per_graph, warm_reps * per_graph


def gemv_inputs(torch):
    """The headline's inputs: COPIES weight copies, one activation row, the
    output and the workspace."""
    from vllm_mi355x.kernels.exl3 import ops

    ops.ensure_extension()
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device)
    gen.manual_seed(1234)
    mats = [make_matrix(torch, gen, device, K_IN, N_OUT, BITS_X2) for _ in range(COPIES)]
    x = torch.randn(ROWS, K_IN, device=device, generator=gen).half()
    out = torch.empty(ROWS, N_OUT, dtype=torch.float16, device=device)
    ws = torch.empty(ops.linear_workspace_size(ROWS, K_IN, N_OUT), dtype=torch.float32, device=device)
    return mats, x, out, ws


def gpu_gemv(args, torch, inputs):
    from vllm_mi355x.kernels.exl3 import ops

    mats, x, out, ws = inputs

    def call(i):
        t, suh, svh = mats[i % COPIES]
        ops.linear_out(x, t, suh, svh, BITS_X2, CODEBOOK, K_IN, N_OUT, out, ws)

    ms = time_steps_exact(torch, call, args.warmup, args.steps, GRAPH_CALLS)
    # the same calls in a long loop (informational: replays of 120-call
    # graphs after 12000 untimed calls, the GPU's steady state)
    steady = None if args.no_steady else time_graph(torch, call, GRAPH_CALLS, 12000, 2400)[0]
    del mats
    return ms, args.steps, args.warmup, steady


def gpu_gemv_configs(args, torch):
    """The other small-M linear shapes of the decode workload: more rows,
    fewer bits per weight, and the transposed (down-projection) matrix.  Each
    rotates enough weight copies (>= 400 MB) that every call streams from
    HBM."""
    from vllm_mi355x.kernels.exl3 import ops

    device = torch.device("cuda:0")
    gen = torch.Generator(device=device)
    gen.manual_seed(4321)
    results = {}
    for name, k, n, bits_x2, rows in (("4bit_m4", K_IN, N_OUT, 8, 4), ("4bit_m8", K_IN, N_OUT, 8, 8),
                                      ("3bit_m1", K_IN, N_OUT, 6, 1), ("2bit_m1", K_IN, N_OUT, 4, 1),
                                      ("4bit_m1_14336x4096", N_OUT, K_IN, 8, 1)):
        nbytes = gemv_bytes(k, n, bits_x2, rows)
        copies = max(COPIES, -(-400_000_000 // nbytes))
        mats = [make_matrix(torch, gen, device, k, n, bits_x2) for _ in range(copies)]
        x = torch.randn(rows, k, device=device, generator=gen).half()
        out = torch.empty(rows, n, dtype=torch.float16, device=device)
        ws = torch.empty(ops.linear_workspace_size(rows, k, n), dtype=torch.float32, device=device)

        def call(i, mats=mats, x=x, out=out, ws=ws, k=k, n=n, bits_x2=bits_x2):
            t, suh, svh = mats[i % len(mats)]
            ops.linear_out(x, t, suh, svh, bits_x2, CODEBOOK, k, n, out, ws)

        ms, _, _ = time_graph(torch, call, GRAPH_CALLS, 240, 480)
        gbs = nbytes / (ms * 1e-3) / 1e9
        results[name] = {"k": k, "n": n, "bits_per_weight": bits_x2 / 2, "rows": rows,
                         "us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        del mats
    return results


def measured_traffic():
    """HBM bytes per GEMV launch from the committed FETCH_SIZE / WRITE_SIZE
    summary (copy-calibrated), or None."""
    try:
        text = open(TRAFFIC_SUMMARY).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, flags=re.M)
    return int(m.group(1)) if m else None


# ---- int4 Marlin MoE ------------------------------------------------------------------

MOE_E, MOE_H, MOE_N, MOE_TOPK = 128, 2048, 768, 8


def marlin_expert_bytes(h: int, n: int) -> int:
    return h * 2 * n // 2 + n * h // 2 + 2 * (h // 128 * 2 * n + n // 128 * h)


def marlin_layer(torch, gen, device):
    info = torch.iinfo(torch.int32)
    w1 = torch.randint(info.min, info.max, (MOE_E, MOE_H // 16, 4 * MOE_N), generator=gen,
                       device=device, dtype=torch.int32)
    w2 = torch.randint(info.min, info.max, (MOE_E, MOE_N // 16, 2 * MOE_H), generator=gen,
                       device=device, dtype=torch.int32)
    s1 = (torch.randn(MOE_E, MOE_H // 128, 2 * MOE_N, generator=gen, device=device) * 0.02).abs().half()
    s2 = (torch.randn(MOE_E, MOE_N // 128, MOE_H, generator=gen, device=device) * 0.02).abs().half()
    return w1, w2, s1, s2


def softmax_topk(torch, logits, k):
    p = torch.softmax(logits.float(), -1)
    w, ids = torch.topk(p, k, -1)
    return (w / w.sum(-1, keepdim=True)).float().contiguous(), ids.to(torch.int32).contiguous()


def gpu_marlin_moe(torch, tokens=(1, 16, 64, 256)):
    """Two copies of the layer (622 MB) and 16 routings per token count,
    rotated call by call, so the weights a call touches stream from HBM: at
    one token the 16 routings use disjoint experts (8 each, 16 x 8 = all
    128), so 32 consecutive calls touch 622 MB, more than the 256 MB
    Infinity Cache; at more tokens each call touches 82-128 experts
    (200-311 MB)."""
    from vllm_mi355x.kernels.marlin_moe import extension, fused

    extension.require_extension()
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device)
    gen.manual_seed(4)
    layers = [marlin_layer(torch, gen, device) for _ in range(2)]
    per_expert = marlin_expert_bytes(MOE_H, MOE_N)
    routings_n = 16
    results = {}
    for T in tokens:
        x = torch.randn(T, MOE_H, generator=gen, device=device).half()
        routings = []
        if T == 1:
            perm = torch.randperm(MOE_E, generator=torch.Generator().manual_seed(41))
            for r in range(routings_n):
                ids = perm[MOE_TOPK * r:MOE_TOPK * (r + 1)].view(1, MOE_TOPK).to(torch.int32).to(device)
                w = torch.softmax(torch.randn(1, MOE_TOPK, generator=gen, device=device), -1).float()
                routings.append((w.contiguous(), ids.contiguous()))
        else:
            for r in range(routings_n):
                routings.append(softmax_topk(torch, torch.randn(T, MOE_E, generator=gen, device=device),
                                             MOE_TOPK))
        out = torch.empty_like(x)
        ws = {}

        def call(i):
            w1, w2, s1, s2 = layers[i % 2]
            tw, ti = routings[(i // 2) % routings_n]
            fused.fused_marlin_moe(x, w1, w2, s1, s2, tw, ti, workspace=ws, output=out)

        ms, _, _ = time_graph(torch, call, 2 * routings_n, 64, 320)
        touched = statistics.mean(int(torch.unique(ti).numel()) for _, ti in routings)
        nbytes = touched * per_expert + 2 * 2 * T * MOE_H
        flops = 2 * T * MOE_TOPK * (MOE_H * 2 * MOE_N + MOE_N * MOE_H)
        gbs = nbytes / (ms * 1e-3) / 1e9
        tflops = flops / (ms * 1e-3) / 1e12
        results[str(T)] = {
            "us_per_forward": round(ms * 1e3, 2), "tokens_per_s": round(T / (ms * 1e-3)),
            "experts_touched": round(touched, 1), "hbm_gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "tflops": round(tflops, 2),
            "mfma_util": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4),
        }
    del layers
    return results


def cpu_marlin_moe(seconds: float, torch):
    """The reference's CPU path (unpack, FP64 dequant of every routed
    expert, FP64 matmuls with the fp16 rounding points) on 4 tokens of the
    same layer shape."""
    from oracle.marlin_torch_ref import moe_fp64

    g = torch.Generator().manual_seed(5)
    info = torch.iinfo(torch.int32)
    T = 4
    x = torch.randn(T, MOE_H, generator=g).half()
    tw, ti = softmax_topk(torch, torch.randn(T, MOE_E, generator=g), MOE_TOPK)
    used = torch.unique(ti)
    remap = torch.full((MOE_E,), -1, dtype=torch.int64)
    remap[used] = torch.arange(used.numel())
    local = remap[ti.long()]
    E = used.numel()
    w1 = torch.randint(info.min, info.max, (E, MOE_H // 16, 4 * MOE_N), generator=g, dtype=torch.int32)
    w2 = torch.randint(info.min, info.max, (E, MOE_N // 16, 2 * MOE_H), generator=g, dtype=torch.int32)
    s1 = (torch.randn(E, MOE_H // 128, 2 * MOE_N, generator=g) * 0.02).abs().half()
    s2 = (torch.randn(E, MOE_N // 128, MOE_H, generator=g) * 0.02).abs().half()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        moe_fp64(x, local, tw, w1, w2, s1, s2)
        times.append(time.perf_counter() - t0)
    per_call = statistics.median(times)
    return {
        "value": round(T / per_call, 2), "unit": "tokens/s", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} calls (median {per_call:.2f} s) of {T} tokens ({E} routed experts) "
                   "of the 128-expert 2048/768 top-8 int4 MoE via the reference's CPU path "
                   "restated in torch (unpack + FP64 dequant of every routed expert, FP64 matmuls "
                   "with the fp16 rounding points)"),
    }


# ---- EXL3 prefill and MoE ---------------------------------------------------------------

class _Fp16Tiles:
    """exl3_set_tile_precision(1) inside the block: the many-row tile GEMM on
    the FP16 high parts of the activations alone (the opt-in below the
    reference's precision); the default (high and low parts) after it."""

    def __enter__(self):
        from vllm_mi355x import _native
        self.lib = _native.load()
        _native.check(self.lib.exl3_set_tile_precision(1))

    def __exit__(self, *exc):
        from vllm_mi355x import _native
        _native.check(self.lib.exl3_set_tile_precision(0))
        return False


def gpu_exl3_prefill(torch, rows=2048, k=8192, n=28672, other_rows=(512, 8192)):
    """The many-row linear at the default precision (FP16 high and low
    activation parts, ~22 bits, as the reference's tensor-core kernels), and
    at the FP16-only opt-in under "fp16_only"."""
    from vllm_mi355x.kernels.exl3 import ops

    ops.ensure_extension()
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    t, suh, svh = make_matrix(torch, gen, device, k, n, 8)

    def measure(m):
        x = torch.randn(m, k, device=device, generator=gen).half()
        out = torch.empty(m, n, dtype=torch.float16, device=device)
        ws = torch.empty(ops.linear_workspace_size(m, k, n), dtype=torch.float32, device=device)

        def call(i):
            ops.linear_out(x, t, suh, svh, 8, CODEBOOK, k, n, out, ws)

        ms, _, _ = time_graph(torch, call, 4, 4, 12)
        tflops = 2 * m * k * n / (ms * 1e-3) / 1e12
        return {"ms": round(ms, 3), "tflops": round(tflops, 1),
                "mfma_util": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4)}

    result = {"workload": f"{k}x{n} 4-bit mul1, M={rows}, fp16", "precision": "fp16 hi+lo activations",
              **measure(rows)}
    result["by_rows"] = {str(m): measure(m) for m in other_rows}
    with _Fp16Tiles():
        result["fp16_only"] = {"precision": "fp16 activations (high parts alone)", **measure(rows),
                               "by_rows": {str(m): measure(m) for m in other_rows}}
    return result


def gpu_exl3_moe(torch, tokens=(64, 2048), experts=256, hidden=7168, inter=2048, topk=8, bits_x2=6):
    """The first token count is the line's headline; every count is in
    by_tokens.  The expert scales are the reference's test scales: with the
    +-1 x N(1, 0.05) scales of the benchmark description, random weights
    overflow FP16 in the down projection (the outputs would be infinite and
    carry no correctness check); the tests check this layer with the same
    scales."""
    from vllm_mi355x.kernels.exl3 import ops

    ops.ensure_extension()
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device)
    gen.manual_seed(9)
    local = experts + 1  # routed experts + the shared expert (local id `experts`)
    keep, ptrs, meta = [], [], []
    for _ in range(local):
        p, m = [], []
        for kk, nn in ((hidden, inter), (hidden, inter), (inter, hidden)):
            t, suh, svh = make_matrix(torch, gen, device, kk, nn, bits_x2, scales="test")
            keep += [t, suh, svh]
            p.append([t.data_ptr(), suh.data_ptr(), svh.data_ptr()])
            m.append([kk, nn, bits_x2, 2])
        ptrs.append(p)
        meta.append(m)
    ptrs = torch.tensor(ptrs, dtype=torch.int64, device=device)
    meta = torch.tensor(meta, dtype=torch.int64, device=device)
    # Zipf(1.1) expert popularity over a seeded permutation, softmax top-8,
    # plus the shared expert with weight 1 in slot 8
    ranks = torch.randperm(experts, generator=torch.Generator().manual_seed(10)).float() + 1.0
    bias = (-1.1 * torch.log(ranks)).to(device)
    emap = torch.arange(local, dtype=torch.int32, device=device)
    per_expert = 3 * hidden * inter * bits_x2 // 16 + 2 * 2 * (hidden + inter) + 2 * (hidden + inter)

    def measure(t_count):
        logits = torch.randn(t_count, experts, generator=gen, device=device) + bias
        tw, ti = softmax_topk(torch, logits, topk)
        ids = torch.cat([ti, torch.full((t_count, 1), experts, dtype=torch.int32, device=device)], 1)
        ids = ids.contiguous()
        weights = torch.cat([tw, torch.ones(t_count, 1, device=device)], 1).contiguous()
        x = torch.randn(t_count, hidden, generator=gen, device=device).half()
        out = torch.empty_like(x)
        ws = torch.empty(ops.moe_workspace_size_v2(t_count, hidden, inter, topk + 1, local),
                         dtype=torch.float32, device=device)

        def call(i):
            ops.moe_out_v2(x, ids, weights, ptrs, meta, emap, inter, bits_x2, out, ws)

        reps = 10 if t_count <= 256 else 2
        ms, _, _ = time_graph(torch, call, reps, reps, 5 * reps)
        if not torch.isfinite(out.float()).all():
            raise RuntimeError(f"EXL3 MoE bench: non-finite outputs at {t_count} tokens")
        touched = int(torch.unique(ids).numel())
        nbytes = touched * per_expert + 2 * 2 * t_count * hidden
        flops = 2 * 3 * hidden * inter * t_count * (topk + 1)
        gbs = nbytes / (ms * 1e-3) / 1e9
        tflops = flops / (ms * 1e-3) / 1e12
        return {"us_per_forward": round(ms * 1e3, 1), "tokens_per_s": round(t_count / (ms * 1e-3)),
                "experts_touched": touched, "hbm_gbs": round(gbs, 1),
                "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "tflops": round(tflops, 1),
                "mfma_util": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4)}

    by_tokens = {str(t_count): measure(t_count) for t_count in tokens}
    with _Fp16Tiles():
        fp16_only = {str(t_count): measure(t_count) for t_count in tokens if t_count > 256}
    del keep
    return {"workload": (f"{experts}+1 experts, {hidden}/{inter}, {bits_x2 / 2:g}-bit mul1, top-{topk} "
                         f"Zipf(1.1), {tokens[0]} tokens, fp16"),
            "precision": "fp16 hi+lo activations",
            **by_tokens[str(tokens[0])], "by_tokens": by_tokens,
            "fp16_only": {"precision": "tile GEMM on fp16 activations (high parts alone)",
                          "by_tokens": fp16_only}}


def gpu_exl3_moe_prefill(torch, tokens=(2048, 65, 512, 3460), experts=256, hidden=2560, inter=640,
                         topk=10, bits_x2=10):
    """The one configuration the reference's moe_out_prefill serves
    (csrc/exl3/moe_prefill.h:9-14): 256 local experts, hidden 2560,
    intermediate 640, every matrix bits_x2 10 mul1, top-10 from softmax of
    ~N(0, 1) logits, bf16 activations, 65 to 3460 rows, through
    _exl3_C::moe_out_prefill; the same 2048-row call through moe_out (the
    run-time-format GEMV in 8-row tasks, what moe_out_prefill ran before it
    had a many-row kernel) for comparison.  The first count is the line's
    headline."""
    from vllm_mi355x.kernels.exl3 import ops

    ops.ensure_extension()
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device)
    gen.manual_seed(11)
    keep, ptrs, meta = [], [], []
    for _ in range(experts):
        p, m = [], []
        for kk, nn in ((hidden, inter), (hidden, inter), (inter, hidden)):
            t, suh, svh = make_matrix(torch, gen, device, kk, nn, bits_x2, scales="test")
            keep += [t, suh, svh]
            p.append([t.data_ptr(), suh.data_ptr(), svh.data_ptr()])
            m.append([kk, nn, bits_x2, 2])
        ptrs.append(p)
        meta.append(m)
    ptrs = torch.tensor(ptrs, dtype=torch.int64, device=device)
    meta = torch.tensor(meta, dtype=torch.int64, device=device)
    emap = torch.arange(experts, dtype=torch.int32, device=device)
    per_expert = 3 * hidden * inter * bits_x2 // 16 + 2 * 2 * (hidden + inter) + 2 * (hidden + inter)

    def measure(t_count, op):
        tw, ti = softmax_topk(torch, torch.randn(t_count, experts, generator=gen, device=device), topk)
        x = torch.randn(t_count, hidden, generator=gen, device=device).bfloat16()
        out = torch.empty_like(x)
        ws = torch.empty(ops.moe_workspace_size(t_count, hidden, inter, topk, experts),
                         dtype=torch.float32, device=device)
        fn = getattr(torch.ops._exl3_C, op)

        def call(i):
            fn(x, ti, tw, ptrs, meta, emap, inter, out, ws)

        reps = 4
        ms, _, _ = time_graph(torch, call, reps, reps, 3 * reps)
        if not torch.isfinite(out.float()).all():
            raise RuntimeError(f"EXL3 MoE prefill bench: non-finite outputs at {t_count} tokens")
        touched = int(torch.unique(ti).numel())
        nbytes = touched * per_expert + 2 * 2 * t_count * hidden
        flops = 2 * 3 * hidden * inter * t_count * topk
        gbs = nbytes / (ms * 1e-3) / 1e9
        tflops = flops / (ms * 1e-3) / 1e12
        return {"us_per_forward": round(ms * 1e3, 1), "tokens_per_s": round(t_count / (ms * 1e-3)),
                "experts_touched": touched, "hbm_gbs": round(gbs, 1),
                "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "tflops": round(tflops, 1),
                "mfma_util": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4)}

    by_tokens = {str(t): measure(t, "moe_out_prefill") for t in tokens}
    with _Fp16Tiles():
        fp16_only = {str(tokens[0]): measure(tokens[0], "moe_out_prefill")}
    runtime_gemv = measure(tokens[0], "moe_out")
    del keep
    head = by_tokens[str(tokens[0])]
    return {"workload": (f"moe_out_prefill {experts} experts, {hidden}/{inter}, bits_x2 {bits_x2} mul1, "
                         f"top-{topk}, {tokens[0]} tokens, bf16"),
            "precision": "fp16 hi+lo activations", **head, "by_tokens": by_tokens,
            "fp16_only": {"precision": "tile GEMM on fp16 activations (high parts alone)",
                          "by_tokens": fp16_only},
            "runtime_decode_gemv": {"op": "moe_out (run-time-format GEMV, 8-row tasks)",
                                    **runtime_gemv,
                                    "speedup_of_moe_out_prefill": round(
                                        runtime_gemv["us_per_forward"] / head["us_per_forward"], 2)}}


def cpu_model() -> str:
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        m = re.search(r"^Model name:\s*(.+)$", out, flags=re.M)
        if m:
            return m.group(1).strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        m = re.search(r"^model name\s*:\s*(.+)$", open("/proc/cpuinfo").read(), flags=re.M)
        return m.group(1).strip() if m else "unknown"
    except OSError:
        return "unknown"


def _time_cpu_linear(torch, k, n, seconds, dtype, seed):
    """Median seconds per call of the reference's CPU dequantize-then-matmul
    on a k x n 4-bit mul1 matrix with +-1 x N(1, 0.05) scales and one fp16
    row ~N(0, 1), and the number of calls timed (1 warm-up first)."""
    from oracle.exl3_torch_ref import DenseDecoder, linear_fp64

    g = torch.Generator().manual_seed(seed)
    trellis = torch.randint(-(2 ** 15), 2 ** 15, (k // 16, n // 16, 8 * BITS_X2), dtype=torch.int16,
                            generator=g)

    def scales(size):
        sign = torch.randint(0, 2, (size,), generator=g).float() * 2 - 1
        return (sign * (1.0 + 0.05 * torch.randn(size, generator=g))).half()

    suh, svh = scales(k), scales(n)
    x = torch.randn(ROWS, k, generator=g).half()
    dec = DenseDecoder(BITS_X2, CODEBOOK)
    linear_fp64(dec, x, trellis, suh, svh, n, dtype)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        linear_fp64(dec, x, trellis, suh, svh, n, dtype)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(seconds: float, torch):
    """The reference's CPU dequantize-then-matmul path (LUT decode of every
    tile, block H128, matmul) on this host: the headline 4096 x 14336
    shape in FP64 (the line's value) and FP32, and the 4096 x 4096
    CPU-plumbing configuration in both."""
    per_call, calls = _time_cpu_linear(torch, K_IN, N_OUT, seconds, torch.float64, 99)
    per32, calls32 = _time_cpu_linear(torch, K_IN, N_OUT, seconds / 2, torch.float32, 98)
    c1_64, c1_calls = _time_cpu_linear(torch, 4096, 4096, seconds / 3, torch.float64, 97)
    c1_32, c1_calls32 = _time_cpu_linear(torch, 4096, 4096, seconds / 3, torch.float32, 96)
    gb = gemv_bytes(K_IN, N_OUT, BITS_X2, ROWS) / 1e9
    gb_c1 = gemv_bytes(4096, 4096, BITS_X2, ROWS) / 1e9
    return {
        "value": round(gb / per_call, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{calls} calls (median {per_call * 1e3:.1f} ms) of the {K_IN}x{N_OUT} 4-bit mul1 "
                   "M=1 linear via the reference's CPU path restated in torch (65536-entry LUT decode "
                   "of every tile, FP64 block H128, FP64 matmul), +-1 x N(1, 0.05) scales"),
        "fp32": {"value": round(gb / per32, 4), "unit": "GB/s", "ms_per_call": round(per32 * 1e3, 2),
                 "calls": calls32},
        "cpu_plumbing_4096x4096": {
            "fp64": {"value": round(gb_c1 / c1_64, 4), "unit": "GB/s", "ms_per_call": round(c1_64 * 1e3, 2),
                     "calls": c1_calls},
            "fp32": {"value": round(gb_c1 / c1_32, 4), "unit": "GB/s", "ms_per_call": round(c1_32 * 1e3, 2),
                     "calls": c1_calls32},
        },
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=1200)
    parser.add_argument("--warmup", type=int, default=120)
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--no-extras", action="store_true",
                        help="only the headline GEMV (profiling runs)")
    parser.add_argument("--only", choices=("prefill", "exl3_moe", "marlin", "moe_prefill"), default=None,
                        help="profiling runs: only this workload, its JSON on one line (not the "
                             "benchmark line)")
    parser.add_argument("--no-steady", action="store_true",
                        help="counter runs: leave out the steady-state loop (14,400 more calls) "
                             "beside the timed steps")
    parser.add_argument("--copy-mb", type=int, default=0,
                        help="also run 10 plain device copies of this many MiB (the counter "
                             "calibration of FETCH_SIZE / WRITE_SIZE)")
    args = parser.parse_args()
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be positive and --warmup nonnegative", file=sys.stderr)
        return 2
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the hot path is a single-GPU kernel; multi-GPU sharding is not built here)",
              file=sys.stderr)
        return 2

    import torch

    torch.set_num_threads(os.cpu_count() or 1)

    def calibration_copies():
        if args.copy_mb:
            src = torch.ones(args.copy_mb << 18, dtype=torch.float32, device="cuda:0")
            dst = torch.empty_like(src)
            for _ in range(10):
                dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst

    if args.only:
        run = {"prefill": gpu_exl3_prefill, "exl3_moe": gpu_exl3_moe, "marlin": gpu_marlin_moe,
               "moe_prefill": gpu_exl3_moe_prefill}[args.only]
        result = run(torch)
        calibration_copies()
        print(json.dumps({args.only: result}))
        return 0
    # the headline's inputs are written first: the other workloads' reads
    # and writes have long evicted them from the Infinity Cache when its
    # timed steps run
    headline_inputs = gemv_inputs(torch)
    extras = {}
    if not args.no_extras:
        # before the headline: the GPU is then at its sustained clock
        moe = gpu_marlin_moe(torch)
        at256 = moe["256"]
        extras["int4_moe"] = {
            "workload": "Marlin int4 fused MoE, 128 experts, hidden 2048, inter 768, top-8, fp16",
            "tokens_per_s_at_256": at256["tokens_per_s"],
            "mfma_util_at_256": at256["mfma_util"],
            "hbm_frac_at_256": at256["hbm_frac"],
            "bound_at_256": "hbm",
            "by_tokens": moe,
        }
        extras["exl3_prefill"] = gpu_exl3_prefill(torch)
        extras["exl3_moe"] = gpu_exl3_moe(torch)
        extras["exl3_moe_prefill"] = gpu_exl3_moe_prefill(torch)
        extras["exl3_gemv_configs"] = gpu_gemv_configs(args, torch)
    ms, steps, warm, steady_ms = gpu_gemv(args, torch, headline_inputs)
    del headline_inputs
    calibration_copies()
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
        "steady_state": None if steady_ms is None else {
            "note": "the same step in a long loop: 2400 timed calls after 12000 untimed ones",
            "us_per_step": round(steady_ms * 1e3, 3),
            "gbs": round(nbytes / (steady_ms * 1e-3) / 1e9, 2),
            "hbm_frac": round(nbytes / (steady_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
        },
    }
    result.update(extras)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds, torch)
        if not args.no_extras:
            result["int4_moe"]["cpu_baseline"] = cpu_marlin_moe(args.cpu_seconds, torch)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
