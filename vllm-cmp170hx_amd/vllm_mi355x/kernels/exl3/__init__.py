"""EXL3 trellis-coded weights (reference: vllm_sm80/kernels/exl3)."""
