"""ctypes binding of libvllm_mi355x.so, the C-ABI library of the hand-written
gfx950 kernels (declared in include/vllm_mi355x.h).

There is no fallback: if the library is missing or fails to load, every
operator raises.  Build it with ``python vllm-cmp170hx_amd/build.py``.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIBRARY_NAME = "libvllm_mi355x.so"
LIBRARY_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIBRARY_NAME)
# The host-only torch custom classes the reference's loader requires
# (csrc/torch_classes.cpp), loaded with torch.ops.load_library.
TORCH_CLASSES_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                  "libvllm_mi355x_torch.so")
ABI_VERSION = 1

BF16, FP16, FP32 = 0, 1, 2
OK = 0

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_vp = ctypes.c_void_p

# name -> (restype, argtypes), mirroring include/vllm_mi355x.h
SIGNATURES = {
    "vllm_mi355x_last_error": (ctypes.c_char_p, []),
    "vllm_mi355x_abi_version": (c_int, []),
    "exl3_linear_workspace_size": (c_i64, [c_i64, c_i64, c_i64]),
    "exl3_linear_prefill_rows": (c_int, []),
    "exl3_linear_out": (c_int, [
        c_vp, c_int, c_i64, c_i64,            # x, x_dtype, rows, x_cols
        c_vp, c_i64, c_i64, c_i64,            # trellis, tiles_k, tiles_n, trellis_words
        c_vp, c_i64, c_vp, c_i64,             # suh, suh_numel, svh, svh_numel
        c_i64, c_i64, c_i64, c_i64,           # bits_x2, codebook, logical_in, logical_out
        c_vp, c_int, c_i64, c_i64,            # out, out_dtype, out_rows, out_cols
        c_vp, c_i64, c_vp,                    # workspace, workspace_numel, stream
    ]),
    "exl3_linear_out_scratch": (c_int, [
        c_vp, c_int, c_i64, c_i64,            # x, x_dtype, rows, x_cols
        c_vp, c_i64, c_i64, c_i64,            # trellis, tiles_k, tiles_n, trellis_words
        c_vp, c_i64, c_vp, c_i64,             # suh, suh_numel, svh, svh_numel
        c_i64, c_i64, c_i64, c_i64,           # bits_x2, codebook, logical_in, logical_out
        c_vp, c_int, c_i64, c_i64,            # out, out_dtype, out_rows, out_cols
        c_vp,                                 # stream
    ]),
    "exl3_linear_scratch_rows": (c_i64, [c_i64, c_i64]),
    "exl3_decode": (c_int, [c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp]),
    "exl3_ple_decode_out": (c_int, [
        c_vp, c_i64, c_i64, c_vp,             # packed_rows, rows, words, global_ids
        c_vp, c_i64, c_vp, c_vp,              # head_bias, heads, head_offsets, head_vocab_sizes
        c_i64, c_i64, c_i64, c_i64,           # dim, owner_lo, owner_hi, bits
        c_vp, c_vp,                           # out, stream
    ]),
    "exl3_set_gemv_finish": (c_int, [c_int]),
    "exl3_counter_fallbacks": (c_i64, []),
    "exl3_set_moe_tile_rows": (c_int, [c_int]),
    "exl3_set_tile_precision": (c_int, [c_int]),
    "exl3_set_prefill_kernel": (c_int, [c_int]),
    "exl3_set_gemv_blocks": (c_int, [c_int]),
    "exl3_set_gemv_groups": (c_int, [c_int]),
    "exl3_moe_workspace_size": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64]),
    "exl3_moe_out": (c_int, [
        c_vp, c_int, c_i64, c_i64,            # x, x_dtype, rows, hidden
        c_vp, c_int, c_vp, c_i64,             # topk_ids, ids64, topk_weights, topk
        c_vp, c_vp, c_i64,                    # packed_ptrs, packed_meta, local_experts
        c_vp, c_int, c_i64,                   # expert_map, map64, global_experts
        c_i64, c_i64,                         # intermediate_size, bits_x2
        c_vp, c_int, c_vp, c_i64,             # out, out_dtype, workspace, workspace_numel
        ctypes.c_float, c_vp,                 # swiglu_limit, stream
    ]),
    "marlin_moe_gemm": (c_int, [
        c_vp, c_int, c_i64, c_i64,            # a, act_dtype, a_rows, a_stride
        c_vp, c_vp, c_i64,                    # w, scales, experts
        c_vp, c_i64, c_vp, c_i64, c_vp,       # sorted, numel, expert_ids, numel, ntpp
        c_vp, c_i64, c_i64,                   # topk_w, top_k, n_slots
        c_i64, c_i64, c_i64, c_int, c_i64,    # K, N, block_size, mode, ksplit
        c_vp, c_i64, c_vp, c_i64, c_i64,      # part, part_numel, out, out_stride, out_rows
        c_vp,                                 # stream
    ]),
    "marlin_moe_gemm_direct": (c_int, [
        c_vp, c_int, c_i64, c_i64,            # a_perm, act_dtype, a_rows, a_stride
        c_vp, c_vp, c_i64,                    # w, scales, experts
        c_vp, c_i64, c_vp, c_i64, c_vp,       # sorted, numel, expert_ids, numel, ntpp
        c_vp, c_i64, c_i64,                   # topk_w, top_k, n_slots
        c_i64, c_i64, c_i64, c_int, c_i64,    # K, N, block_size, mode, ksplit
        ctypes.c_float,                       # limit
        c_vp, c_i64, c_vp, c_i64, c_i64,      # part, part_numel, out, out_stride, out_rows
        c_vp,                                 # stream
    ]),
    "marlin_permute_act": (c_int, [c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp]),
    "marlin_moe_align_permute": (c_int, [
        c_vp, c_i64, c_i64, c_i64, c_vp,      # topk_ids, numel, num_experts, block_size, expert_map
        c_vp, c_i64, c_vp, c_i64, c_vp,       # sorted, numel, expert_ids, numel, ntpp
        c_vp, c_int, c_i64, c_i64, c_i64,     # a, act_dtype, rows, cols, a_stride
        c_vp, c_i64, c_vp,                    # out, out_stride, stream
    ]),
    "marlin_moe_w2_sum": (c_int, [
        c_vp, c_int, c_i64, c_i64, c_vp,      # a, act_dtype, a_rows, a_stride, w
        c_vp, c_i64, c_vp, c_i64, c_vp,       # scales, experts, expert_ids, numel, topk_w
        c_i64, c_i64, c_i64, c_i64, c_i64,    # top_k, n_slots, K, N, block_size
        c_vp, c_i64, c_i64, c_vp, c_vp,       # out, out_stride, out_rows, sum_out, stream
    ]),
    "marlin_moe_act": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, ctypes.c_float, c_vp, c_int,
                               c_vp]),
    "marlin_moe_w13_act": (c_int, [
        c_vp, c_int, c_i64, c_i64, c_vp,      # a, act_dtype, a_rows, a_stride, w
        c_vp, c_i64,                          # scales, experts
        c_vp, c_i64, c_vp, c_i64, c_vp,       # sorted, numel, expert_ids, numel, ntpp
        c_vp, c_i64, c_i64,                   # ids, top_k, n_slots
        c_i64, c_i64, c_i64, c_i64,           # K, N, block_size, ksplit
        ctypes.c_float,                       # limit
        c_vp, c_i64, c_vp, c_i64, c_i64,      # part, part_numel, h, h_stride, h_rows
        c_vp,                                 # stream
    ]),
    "marlin_dequant": (c_int, [c_vp, c_vp, c_int, c_i64, c_i64, c_vp, c_vp]),
    "moe_sum": (c_int, [c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp]),
    "moe_sum_add": (c_int, [c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp]),
    "moe_align_block_size": (c_int, [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64,
                                     c_vp, c_vp]),
    "moe_route": (c_int, [
        c_vp, c_int, c_i64, c_i64, c_i64,        # x, x_dtype, M, K, x_stride
        c_vp, c_vp, c_i64, c_i64,                # weight, bias, num_experts, topk
        c_int, c_int, ctypes.c_float, c_i64,     # scoring, renormalize, scale, block_size
        c_vp, c_vp, c_vp, c_vp,                  # is_padding, logits, topk_weights, topk_ids
        c_vp, c_i64, c_vp, c_i64, c_vp,          # sorted, numel, expert_ids, numel, ntpp
        c_vp,                                    # stream
    ]),
    "moe_split_align": (c_int, [
        c_vp, c_i64, c_i64, c_vp, c_vp, c_i64,  # topk_ids, numel, num_experts, expert_map, cover, rows
        c_vp, c_vp, c_vp, c_vp, c_vp,            # sorted lists 64 / 48 / 32 / 16, sorted_numel[4]
        c_vp, c_vp, c_vp, c_vp, c_vp,            # expert-id lists, eids_numel[4]
        c_vp, c_vp,                              # ntpp[4], stream
    ]),
}

_lib = None
_lock = threading.Lock()


class NativeError(RuntimeError):
    """A check of the native library failed (the reference raises
    RuntimeError from TORCH_CHECK for the same conditions)."""


def load() -> ctypes.CDLL:
    """The loaded library; raises if it is missing or of another ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIBRARY_PATH):
            raise ImportError(
                f"{LIBRARY_NAME} is not built ({LIBRARY_PATH} is missing): run "
                "python vllm-cmp170hx_amd/build.py")
        lib = ctypes.CDLL(LIBRARY_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.vllm_mi355x_abi_version()
        if version != ABI_VERSION:
            raise ImportError(f"{LIBRARY_NAME} ABI {version}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def last_error() -> str:
    return load().vllm_mi355x_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    if status != OK:
        raise NativeError(last_error())


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
