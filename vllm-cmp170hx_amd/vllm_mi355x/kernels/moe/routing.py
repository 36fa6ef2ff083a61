"""The slot-order top-k sum (vllm_sm80/kernels/moe/routing.py:579-600) and its
shared-expert fold (vllm_sm80/kernels/moe/sum.py:18-56) on gfx950."""

from __future__ import annotations

import torch

from ... import _native

_DTYPE_CODES = {torch.bfloat16: _native.BF16, torch.float16: _native.FP16}


def moe_sum(inp: torch.Tensor, out: torch.Tensor | None = None,
            topk_ids: torch.Tensor | None = None, num_experts: int = 0) -> torch.Tensor:
    """[M, topk, H] -> [M, H]: FP32 sum over the slots in slot order, rounded
    once.  With topk_ids (int32 [M, topk]), slots whose id is outside
    [0, num_experts) add nothing."""
    M, topk, H = inp.shape
    if inp.dtype not in _DTYPE_CODES or not inp.is_contiguous():
        raise RuntimeError("moe_sum: contiguous bf16 or fp16 input")
    if out is None:
        out = torch.empty((M, H), dtype=inp.dtype, device=inp.device)
    if out.dtype != inp.dtype or not out.is_contiguous() or out.shape != (M, H):
        raise RuntimeError("moe_sum: out must be a contiguous [M, H] of the input dtype")
    ids = None
    if topk_ids is not None:
        ids = topk_ids.to(torch.int32).contiguous()
        if ids.numel() != M * topk or ids.device != inp.device:
            raise RuntimeError("moe_sum: topk_ids must be [M, topk] on the input's device")
    with torch.cuda.device(inp.device):
        status = _native.load().moe_sum(
            inp.data_ptr(), _DTYPE_CODES[inp.dtype], M, topk, H,
            0 if ids is None else ids.data_ptr(), int(num_experts), out.data_ptr(),
            torch.cuda.current_stream(inp.device).cuda_stream)
    _native.check(status)
    return out


def moe_sum_add(inp: torch.Tensor, shared: torch.Tensor) -> torch.Tensor:
    """shared + moe_sum(inp) in one kernel (sum.py:18-56): the routed FP32
    slot-order sum rounded to the dtype, then one rounded add of the shared
    expert's output; inp [M, topk, H], shared [M, H] (any strides)."""
    M, topk, H = inp.shape
    if inp.dtype not in _DTYPE_CODES or not inp.is_contiguous():
        raise RuntimeError("moe_sum_add: contiguous bf16 or fp16 input")
    if shared.shape != (M, H) or shared.dtype != inp.dtype or shared.device != inp.device:
        raise RuntimeError("moe_sum_add: shared must be [M, H] of the input dtype and device")
    out = torch.empty((M, H), dtype=inp.dtype, device=inp.device)
    if M == 0:
        return out
    with torch.cuda.device(inp.device):
        status = _native.load().moe_sum_add(
            inp.data_ptr(), _DTYPE_CODES[inp.dtype], M, topk, H, shared.data_ptr(),
            shared.stride(0), shared.stride(1), out.data_ptr(),
            torch.cuda.current_stream(inp.device).cuda_stream)
    _native.check(status)
    return out
