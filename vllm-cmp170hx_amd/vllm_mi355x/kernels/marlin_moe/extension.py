"""Loads and validates the _ampere_marlin_C operators (the reference's
vllm_sm80/kernels/marlin_moe/extension.py contract: build_info handshake,
operator argument names and types), backed by libvllm_mi355x.so."""

from __future__ import annotations

import torch

from . import _C

_OPS = None
_SCHEMA_ARGUMENTS = {
    "decode_gemm_orig": (
        "a w s sorted eids ntpp topk_w topk n_slots K N w13 rows cfg ctr out",
        "Tensor Tensor Tensor Tensor Tensor Tensor Tensor int int int int bool int int Tensor Tensor",
        "int",
    ),
    "decode_act_orig": (
        "part ids ksplit n_slots Nh limit h",
        "Tensor Tensor int int int float Tensor",
        "",
    ),
}
_PREFILL_TILE_SCHEMA = (
    "a c_or_none b_q_weight b_bias_or_none b_scales a_scales global_scale "
    "b_zeros_or_none workspace sorted_token_ids expert_ids num_tokens_past_padded "
    "topk_weights moe_block_size top_k mul_topk_weights b_type_id size_m size_n "
    "size_k use_atomic_add use_fp32_reduce is_zp_float thread_k thread_n "
    "blocks_per_sm c_tmp redo"
)


def _validate() -> None:
    built = _C.build_info()
    if built["abi_version"] != _C.ABI_VERSION:
        raise ValueError(f"abi_version mismatch: {built['abi_version']}")
    for name, (names, types, returns) in _SCHEMA_ARGUMENTS.items():
        qualified = f"_ampere_marlin_C::{name}"
        schema = torch._C._dispatch_find_schema_or_throw(qualified, "").schema()
        actual = (" ".join(a.name for a in schema.arguments),
                  " ".join(str(a.type) for a in schema.arguments),
                  " ".join(str(a.type) for a in schema.returns))
        if actual != (names, types, returns):
            raise ValueError(f"incompatible operator schema: {qualified}")
        if not torch._C._dispatch_has_kernel_for_dispatch_key(qualified, "CUDA"):
            raise ValueError(f"missing GPU implementation: {qualified}")
    schema = torch._C._dispatch_find_schema_or_throw("_ampere_marlin_C::prefill_tile_gemm",
                                                    "").schema()
    if " ".join(a.name for a in schema.arguments) != _PREFILL_TILE_SCHEMA:
        raise ValueError("incompatible operator schema: prefill_tile_gemm")


def require_extension():
    """torch.ops._ampere_marlin_C, registered and validated; raises when
    libvllm_mi355x.so is missing or incompatible (never compiles)."""
    global _OPS
    if _OPS is None:
        try:
            _C.register()
            _validate()
        except (ImportError, OSError, AttributeError, RuntimeError, ValueError) as exc:
            raise RuntimeError(
                "Marlin MoE requires libvllm_mi355x.so, built for gfx950: build it with "
                f"python vllm-cmp170hx_amd/build.py. Detail: {exc}") from exc
        _OPS = torch.ops._ampere_marlin_C
    return _OPS


def prefill_tile_op():
    """(op, None) for prefill_tile_gemm, or (None, reason)."""
    try:
        return require_extension().prefill_tile_gemm, None
    except RuntimeError as exc:
        return None, str(exc)


def decode_v2_op():
    """(op, None) for decode_gemm_v2, or (None, reason)."""
    try:
        return require_extension().decode_gemm_v2, None
    except RuntimeError as exc:
        return None, str(exc)
