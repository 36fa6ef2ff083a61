"""MI355X (gfx950) drop-in for the quantized-weight matmul path of the
vllm_sm80 plugin: EXL3 trellis-coded linear layers and the Marlin-layout
int4 fused MoE, on hand-written HIP kernels behind a C-ABI library."""

__version__ = "0.1.0"
