"""Operator bindings, laid out as vllm_sm80.kernels is."""
