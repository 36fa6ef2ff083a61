"""MoE routing helpers on gfx950: the deterministic block alignment and the
slot-order top-k sum and the router with alignment (vllm_sm80/kernels/moe/align.py,
routing.py, route.py)."""

from .align import align, kernel_moe_align_block_size, moe_align_block_size
from .route import moe_route
from .routing import moe_sum, moe_sum_add

__all__ = ["align", "kernel_moe_align_block_size", "moe_align_block_size", "moe_route", "moe_sum",
           "moe_sum_add"]
