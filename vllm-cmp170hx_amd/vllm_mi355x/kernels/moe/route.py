"""MoE router + block alignment on the device (vllm_sm80/kernels/moe/route.py:
``moe_route``, ``align_sizes``, ``pad_supported``, ``warmup``).

    x [M, K] bf16 (unit column stride), weight [E, K] bf16, bias [E] fp32
      -> logits [M, E] f32, topk_weights [M, topk] f32, topk_ids [M, topk] i32,
         sorted_ids [mnp] i32, expert_ids [nblk] i32, num_tokens_post_pad [1] i32

Two launches (libvllm_mi355x.so ``moe_route``): the router GEMV on the
matrix cores (one fixed FP32 summation order), then one workgroup that
routes every row (sigmoid + bias keys, top-k with ties to the lower expert,
renormalize, scale) and aligns the ids exactly as ``moe_align_block_size``.
No host sync and no allocation when ``out`` is given: graph-capturable.
``scoring="softmax"`` routes by softmax probabilities instead (bias unused).
"""

from __future__ import annotations

import torch

from ... import _native
from .align import align_sizes

_SCORING = {"softmax": 0, "sigmoid": 1}


def pad_supported(M: int, hidden: int = 4096) -> bool:
    """Whether ``is_padding`` is taken at this shape (every M here)."""
    return M >= 1 and hidden % 128 == 0


def warmup(*args, **kwargs) -> None:
    """Nothing to compile ahead of time (the kernels are prebuilt)."""


def moe_route(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, topk: int = 8,
              block_size: int = 8, num_experts: int = 288, renormalize: bool = True,
              routed_scaling_factor: float = 2.5, out=None, is_padding: torch.Tensor | None = None,
              scoring: str = "sigmoid"):
    """Router GEMV + top-k + Marlin block alignment; returns (logits,
    topk_weights, topk_ids, sorted_ids, expert_ids, num_tokens_post_pad)."""
    M, K = x.shape
    E = weight.shape[0]
    if E != num_experts:
        raise AssertionError(f"weight has {E} experts, expected {num_experts}")
    if weight.shape[1] != K or not weight.is_contiguous():
        raise AssertionError("weight must be a contiguous [E, K] matrix")
    if x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype:
        raise AssertionError("x and weight: bf16 (or fp16) of one dtype")
    if x.stride(1) != 1:
        raise AssertionError("x needs a unit column stride")
    if scoring not in _SCORING:
        raise ValueError(f"unknown scoring {scoring!r}")
    if scoring == "sigmoid":
        if bias is None or bias.dtype != torch.float32 or tuple(bias.shape) != (E,):
            raise AssertionError("bias: fp32 [E]")
        bias = bias.contiguous()
    if not (1 <= topk <= num_experts):
        raise AssertionError("topk out of range")
    dev = x.device
    mnp, nblk = align_sizes(M * topk, num_experts, block_size)
    if out is None:
        logits = torch.empty((M, E), dtype=torch.float32, device=dev)
        topk_w = torch.empty((M, topk), dtype=torch.float32, device=dev)
        topk_ids = torch.empty((M, topk), dtype=torch.int32, device=dev)
        sorted_ids = torch.empty((mnp,), dtype=torch.int32, device=dev)
        expert_ids = torch.empty((nblk,), dtype=torch.int32, device=dev)
        ntpp = torch.empty((1,), dtype=torch.int32, device=dev)
    else:
        logits, topk_w, topk_ids, sorted_ids, expert_ids, ntpp = out
        if not logits.is_contiguous() or tuple(logits.shape) != (M, E):
            raise AssertionError("logits: contiguous fp32 [M, E]")
    pad = None
    if is_padding is not None:
        if tuple(is_padding.shape) != (M,) or not is_padding.is_contiguous():
            raise AssertionError("is_padding: contiguous [M]")
        pad = is_padding.view(torch.uint8) if is_padding.dtype == torch.bool else is_padding
    with torch.cuda.device(dev):
        status = _native.load().moe_route(
            x.data_ptr(), _native.BF16 if x.dtype == torch.bfloat16 else _native.FP16, M, K,
            x.stride(0), weight.data_ptr(), 0 if bias is None else bias.data_ptr(), E, topk,
            _SCORING[scoring], int(bool(renormalize)), float(routed_scaling_factor), block_size,
            0 if pad is None else pad.data_ptr(), logits.data_ptr(), topk_w.data_ptr(),
            topk_ids.data_ptr(), sorted_ids.data_ptr(), sorted_ids.numel(), expert_ids.data_ptr(),
            expert_ids.numel(), ntpp.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    _native.check(status)
    return logits, topk_w, topk_ids, sorted_ids, expert_ids, ntpp
