"""Deterministic MoE block alignment (vllm_sm80/kernels/moe/align.py:233-273,
spec tests/kernels/moe_align_reference.py): routed rows grouped by expert,
ranked by ascending flat index inside an expert, each expert padded to the
block size with the sentinel numel, on one gfx950 workgroup."""

from __future__ import annotations

import torch

from ... import _native


def align_sizes(numel: int, num_experts: int, block_size: int) -> tuple[int, int]:
    """(sorted size, block count) as upstream moe_align_block_size sizes its
    outputs."""
    max_pad = numel + num_experts * (block_size - 1)
    if numel < num_experts:
        max_pad = min(numel * block_size, max_pad)
    return max_pad, (max_pad + block_size - 1) // block_size


def kernel_moe_align_block_size(topk_ids: torch.Tensor, num_experts: int, block_size: int,
                                sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor,
                                num_tokens_post_pad: torch.Tensor,
                                expert_map: torch.Tensor | None,
                                scatter_idx: torch.Tensor | None) -> None:
    """Writes the alignment out-params (GPU tensors only).  scatter_idx, if
    given, receives each routed row's own index (-1 for dropped rows)."""
    if not topk_ids.is_cuda:
        raise ValueError("the deterministic MoE alignment needs GPU tensors")
    for t, name in ((topk_ids, "topk_ids"), (sorted_token_ids, "sorted_token_ids"),
                    (expert_ids, "expert_ids"), (num_tokens_post_pad, "num_tokens_post_pad")):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != topk_ids.device:
            raise RuntimeError(f"{name} must be a contiguous int32 tensor on the ids' device")
    emap = None
    if expert_map is not None:
        emap = expert_map.to(torch.int32).contiguous()
        if emap.numel() < num_experts or emap.device != topk_ids.device:
            raise RuntimeError("expert_map needs num_experts entries on the ids' device")
    with torch.cuda.device(topk_ids.device):
        status = _native.load().moe_align_block_size(
            topk_ids.data_ptr(), topk_ids.numel(), int(num_experts), int(block_size),
            0 if emap is None else emap.data_ptr(), sorted_token_ids.data_ptr(),
            sorted_token_ids.numel(), expert_ids.data_ptr(), expert_ids.numel(),
            num_tokens_post_pad.data_ptr(), torch.cuda.current_stream(topk_ids.device).cuda_stream)
    _native.check(status)
    if scatter_idx is not None:
        flat = topk_ids.reshape(-1).long()
        ok = (flat >= 0) & (flat < num_experts)
        if emap is not None:
            ok = ok & (emap.long()[torch.where(ok, flat, 0)] >= 0)
        idx = torch.arange(flat.numel(), device=flat.device)
        scatter_idx.reshape(-1).copy_(torch.where(ok, idx, -1))


def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int, block_size: int,
                         sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor,
                         num_tokens_post_pad: torch.Tensor,
                         expert_map: torch.Tensor | None = None) -> None:
    """The out-param form of upstream _moe_C.moe_align_block_size."""
    kernel_moe_align_block_size(topk_ids, num_experts, block_size, sorted_token_ids, expert_ids,
                                num_tokens_post_pad, expert_map, None)


def align(topk_ids: torch.Tensor, num_experts: int, block_size: int,
          expert_map: torch.Tensor | None = None):
    """Fresh (sorted_ids, expert_ids, num_tokens_post_pad), sized as upstream
    moe_align_block_size sizes them."""
    size, blocks = align_sizes(topk_ids.numel(), num_experts, block_size)
    dev = topk_ids.device
    sorted_ids = torch.empty(size, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(blocks, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
    kernel_moe_align_block_size(ids.contiguous(), num_experts, block_size, sorted_ids,
                                expert_ids, ntpp, expert_map, None)
    return sorted_ids, expert_ids, ntpp
