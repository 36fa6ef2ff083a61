"""The reference's CPU dequantize-then-matmul path for the Marlin int4 MoE,
restated in torch.

TEST INFRASTRUCTURE ONLY (the cpu_baseline leg of bench.py and the tests).

The reference's product code has no CPU path; its CPU-capable reference is
the test harness's _dequant + reference_fp64
(tests/kernels/test_ampere_pp_marlin_prefill.py:332-389): every routed
expert's packed weights are unpacked from the Marlin layout and scaled in
FP64, then FP64 matmuls with the incumbent's activation-dtype rounding
points (w13 rows, SiLU, h, w2 rows, router-weight product) and an FP64 sum
over the slots.  This module is that path on torch CPU tensors, with the
unpacking done by index tables built from the layout of
csrc/ampere_marlin/decode_orig.cu:10-19.
"""

from __future__ import annotations

from functools import lru_cache

import torch

# nibble i of NVIDIA lane (c, g): k offset 2c + _KK[i], n offset g + _NN[i]
_KK = (0, 8, 0, 8, 1, 9, 1, 9)
_NN = (0, 0, 8, 8, 0, 0, 8, 8)


@lru_cache(maxsize=None)
def _positions(K: int, N: int) -> torch.Tensor:
    """Flat (k * N + n) of every nibble, in packed order [K/16][N/64][32][4][8]."""
    r = torch.arange(K // 16).view(-1, 1, 1, 1, 1)
    t = torch.arange(N // 64).view(1, -1, 1, 1, 1)
    lane = torch.arange(32).view(1, 1, -1, 1, 1)
    j = torch.arange(4).view(1, 1, 1, -1, 1)
    kk = torch.tensor(_KK).view(1, 1, 1, 1, -1)
    nn = torch.tensor(_NN).view(1, 1, 1, 1, -1)
    k = 16 * r + 2 * (lane % 4) + kk
    n = 64 * t + 16 * j + lane // 4 + nn
    return (k * N + n).reshape(-1)


@lru_cache(maxsize=None)
def _scale_columns(N: int) -> torch.Tensor:
    c = torch.arange(N)
    return (c // 64) * 64 + 8 * (c % 8) + (c % 64) // 8


def dequant_fp64(w: torch.Tensor, s: torch.Tensor, K: int, N: int) -> torch.Tensor:
    """(q - 8) * s in FP64, [K, N], of int32 [K/16, 2N] and scales [K/128, N]."""
    words = w.reshape(-1, 1).to(torch.int64) & 0xFFFFFFFF
    shifts = 4 * torch.arange(8, dtype=torch.int64).view(1, -1)
    nibbles = ((words >> shifts) & 15).reshape(-1).to(torch.float64)
    q = torch.empty(K * N, dtype=torch.float64)
    q[_positions(K, N)] = nibbles
    scales = s.to(torch.float64)[:, _scale_columns(N)].repeat_interleave(128, dim=0)
    return (q.view(K, N) - 8.0) * scales


def _round(v: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return v.to(dtype).to(torch.float64)


def moe_fp64(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
             w1: torch.Tensor, w2: torch.Tensor, s1: torch.Tensor, s2: torch.Tensor,
             clamp: float = float("inf")) -> torch.Tensor:
    """reference_fp64 of the reference test: [M, K] FP64 before the final
    rounding, every routed expert dequantized for the call."""
    dtype = x.dtype
    M, K = x.shape
    N = w2.shape[1] * 16
    x64 = x.to(torch.float64)
    wr = _round(topk_weights.to(torch.float32), dtype)
    acc = torch.zeros(M, K, dtype=torch.float64)
    for e in torch.unique(topk_ids).tolist():
        if e < 0 or e >= w1.shape[0]:
            continue
        rows, slot = (topk_ids == e).nonzero(as_tuple=True)
        h1 = _round(x64[rows] @ dequant_fp64(w1[e], s1[e], K, 2 * N), dtype)
        gate = h1[:, :N].clamp(max=clamp)
        up = h1[:, N:].clamp(min=-clamp, max=clamp)
        h = _round(_round(gate / (1.0 + torch.exp(-gate)), dtype) * up, dtype)
        y = _round(h @ dequant_fp64(w2[e], s2[e], N, K), dtype)
        acc.index_add_(0, rows, _round(y * wr[rows, slot].unsqueeze(1), dtype))
    return acc
