"""MoE routing helpers on gfx950: the deterministic block alignment and the
slot-order top-k sum (vllm_sm80/kernels/moe/align.py, routing.py)."""

from .align import align, kernel_moe_align_block_size, moe_align_block_size
from .routing import moe_sum, moe_sum_add

__all__ = ["align", "kernel_moe_align_block_size", "moe_align_block_size", "moe_sum",
           "moe_sum_add"]
