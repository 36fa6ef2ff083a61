"""Marlin-format int4 fused MoE on gfx950 (vllm_sm80/kernels/marlin_moe)."""

from .fused import fused_marlin_moe, marlin_dequant, workspace_shapes

__all__ = ["fused_marlin_moe", "marlin_dequant", "workspace_shapes"]
