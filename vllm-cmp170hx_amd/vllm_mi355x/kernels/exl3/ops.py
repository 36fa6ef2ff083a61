"""EXL3 operator bindings with the reference's Python API
(vllm_sm80/kernels/exl3/ops.py), on the gfx950 library.

The functions keep the reference's names, arguments, return values and
error behaviour (RuntimeError for a failed check); the compute runs in
hand-written HIP kernels behind ``torch.ops._exl3_C``.
"""

from __future__ import annotations

from functools import lru_cache

import torch

from . import _C

_loaded = False

# One fixed FP32 scratch per (device, stream) for the ``exl3_linear`` custom
# op; rows are processed in chunks whose workspace fits it
# (ops.py:31-33, :1431-1452 of the reference).
LINEAR_SCRATCH_ELEMENTS = 8 << 20

# Output dtypes of the dense linear: BF16 / FP16 round the FP32 result once;
# FP32 stores it (reference ops.py:114, plus FP16 for FP16 models).
LINEAR_OUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)

# The operators the reference's loader requires (ops.py:193-207), plus this
# library's decode.
_OPERATORS = ("linear_out", "linear_out_splitk", "moe_out", "moe_out_v2", "moe_out_prefill",
              "ple_decode_out", "ple_read_rows", "linear_workspace_size",
              "linear_splitk_splits", "moe_workspace_size", "moe_workspace_size_v2",
              "moe_workspace_size_prefill", "exl3_decode")


def _linear_fake(x, trellis, suh, svh, bits_x2, codebook, logical_in, logical_out, out,
                 workspace):
    torch._check(x.dtype in (torch.bfloat16, torch.float16))
    torch._check(out.dtype in LINEAR_OUT_DTYPES)
    torch._check(out.shape[0] == x.shape[0])
    torch._check(out.shape[1] == logical_out)
    torch._check(x.shape[1] == logical_in)
    torch._check(workspace.dtype == torch.float32)


def _moe_fake(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
              intermediate_size, out, workspace, swiglu_limit=0.0):
    torch._check(x.dtype in (torch.bfloat16, torch.float16))
    torch._check(out.dtype == x.dtype)
    torch._check(out.shape == x.shape)
    torch._check(topk_ids.shape == topk_weights.shape)
    torch._check(workspace.dtype == torch.float32)


def _moe_v2_fake(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
                 intermediate_size, bits_x2, out, workspace, swiglu_limit=0.0):
    _moe_fake(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
              intermediate_size, out, workspace, swiglu_limit)


def _ple_fake(packed_rows, global_ids, head_bias, head_offsets, head_vocab_sizes, owner_lo,
              owner_hi, bits, out):
    torch._check(out.dtype == torch.bfloat16)
    torch._check(out.shape[0] == packed_rows.shape[0])
    torch._check(out.shape[1] == head_bias.shape[1])
    torch._check(global_ids.numel() == packed_rows.shape[0])


# Classes the reference's loader requires (ops.py:205): registered by
# libvllm_mi355x_torch.so, raising when used.
_CLASSES = ("PleHostReader", "EngramHostFetch")


def _validate_extension() -> None:
    built = _C.build_info()
    if built["abi_version"] != _C.ABI_VERSION:
        raise ValueError(f"abi_version mismatch: {built['abi_version']} vs {_C.ABI_VERSION}")
    for name in _OPERATORS:
        torch._C._dispatch_find_schema_or_throw(f"_exl3_C::{name}", "")
    for name in _CLASSES:
        getattr(torch.classes._exl3_C, name)


def ensure_extension() -> None:
    """Loads and registers the operators once (reference ops.py:279-308)."""
    global _loaded
    if _loaded:
        return
    try:
        _C.register()
        _validate_extension()
    except (ImportError, OSError, AttributeError, RuntimeError, ValueError) as exc:
        raise RuntimeError(
            "EXL3 requires libvllm_mi355x.so, built for gfx950: build it with "
            f"python vllm-cmp170hx_amd/build.py. Detail: {exc}") from exc
    for name in ("linear_out", "linear_out_splitk"):
        torch.library.register_fake(f"_exl3_C::{name}")(_linear_fake)
    for name in ("moe_out", "moe_out_prefill", "moe_out_mixed"):
        torch.library.register_fake(f"_exl3_C::{name}")(_moe_fake)
    for name in ("moe_out_v2", "moe_out_v2_fold", "moe_out_v2_mixed", "moe_out_prefill_v2",
                 "moe_out_prefill_try", "moe_out_prefill_try_mixed", "moe_out_v2_try",
                 "moe_out_v2_try_mixed"):
        torch.library.register_fake(f"_exl3_C::{name}")(_moe_v2_fake)
    torch.library.register_fake("_exl3_C::linear_out_prefill")(_linear_fake)
    torch.library.register_fake("_exl3_C::ple_decode_out")(_ple_fake)
    _loaded = True


@lru_cache(maxsize=None)
def linear_workspace_size(max_rows: int, padded_in: int, padded_out: int) -> int:
    ensure_extension()
    return torch.ops._exl3_C.linear_workspace_size(max_rows, padded_in, padded_out)


@lru_cache(maxsize=None)
def linear_row_chunk(padded_in: int, padded_out: int) -> int:
    """The most rows whose linear workspace fits the fixed scratch."""
    rows, limit = 0, LINEAR_SCRATCH_ELEMENTS
    while rows < limit:
        middle = (rows + limit + 1) // 2
        if linear_workspace_size(middle, padded_in, padded_out) <= LINEAR_SCRATCH_ELEMENTS:
            rows = middle
        else:
            limit = middle - 1
    if rows == 0:
        raise ValueError("One EXL3 matrix row exceeds the fixed linear scratch")
    return rows


def linear_out(x, trellis, suh, svh, bits_x2: int, codebook: int, logical_in: int,
               logical_out: int, out, workspace) -> None:
    ensure_extension()
    torch.ops._exl3_C.linear_out(x, trellis, suh, svh, bits_x2, codebook, logical_in,
                                 logical_out, out, workspace)


def linear_out_splitk(x, trellis, suh, svh, bits_x2: int, codebook: int, logical_in: int,
                      logical_out: int, out, workspace) -> None:
    """linear_out's contract (arguments, checks, workspace)."""
    ensure_extension()
    torch.ops._exl3_C.linear_out_splitk(x, trellis, suh, svh, bits_x2, codebook, logical_in,
                                        logical_out, out, workspace)


def linear_splitk_splits(rows: int, padded_out: int, sms: int, bits_x2: int,
                         codebook: int) -> int:
    ensure_extension()
    return torch.ops._exl3_C.linear_splitk_splits(rows, padded_out, sms, bits_x2, codebook)


@lru_cache(maxsize=None)
def moe_workspace_size(max_rows: int, hidden_size: int, intermediate_size: int, topk: int,
                       local_experts: int) -> int:
    ensure_extension()
    return torch.ops._exl3_C.moe_workspace_size(max_rows, hidden_size, intermediate_size, topk,
                                                local_experts)


@lru_cache(maxsize=None)
def moe_workspace_size_v2(max_rows: int, hidden_size: int, intermediate_size: int, topk: int,
                          local_experts: int) -> int:
    ensure_extension()
    return torch.ops._exl3_C.moe_workspace_size_v2(max_rows, hidden_size, intermediate_size, topk,
                                                   local_experts)


def moe_launch_rows(hidden: int, intermediate_size: int, topk: int) -> int:
    """Most rows one MoE launch takes: its workspace rows (rows * topk
    assignments of the padded hidden / intermediate width, FP32) are
    addressed with 32-bit byte offsets, so larger calls run in row chunks
    (the reference chunks its calls the same way, quant.py:1898-1910)."""
    kmax = max(-(-hidden // 128) * 128, -(-intermediate_size // 128) * 128)
    return max(1, (2 ** 31 - 1) // (4 * kmax * max(1, topk)))


def _chunked_moe(op, x, topk_ids, topk_weights, args, out, workspace, tail, row_chunk):
    rows = x.shape[0]
    chunk = row_chunk or moe_launch_rows(x.shape[1], args[3], topk_ids.shape[1])
    if rows <= chunk:
        op(x, topk_ids, topk_weights, *args, out, workspace, *tail)
        return
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        op(x[r0:r1], topk_ids[r0:r1], topk_weights[r0:r1], *args, out[r0:r1], workspace, *tail)


def moe_out(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
            intermediate_size: int, out, workspace, swiglu_limit: float = 0.0,
            row_chunk: int | None = None) -> None:
    """Routed experts; swiglu_limit > 0 clamps the FP32 gate from above and
    up on both sides before SiLU(gate) * up (reference ops.py:585-616).
    Calls above moe_launch_rows rows (or ``row_chunk``) run in row chunks,
    the workspace sized for one chunk."""
    ensure_extension()
    _chunked_moe(torch.ops._exl3_C.moe_out, x, topk_ids, topk_weights,
                 (packed_ptrs, packed_meta, expert_map, intermediate_size), out, workspace,
                 (swiglu_limit,), row_chunk)


def moe_out_v2(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
               intermediate_size: int, bits_x2: int, out, workspace,
               swiglu_limit: float = 0.0, row_chunk: int | None = None) -> None:
    """moe_out for a layer whose routed matrices all have rate bits_x2
    (mul1), with the decode specialized for that rate (row chunks as
    moe_out)."""
    ensure_extension()
    _chunked_moe(torch.ops._exl3_C.moe_out_v2, x, topk_ids, topk_weights,
                 (packed_ptrs, packed_meta, expert_map, intermediate_size, bits_x2), out, workspace,
                 (swiglu_limit,), row_chunk)


def ple_decode_out(packed_rows, global_ids, head_bias, head_offsets, head_vocab_sizes,
                   owner_lo: int, owner_hi: int, bits: int, out) -> None:
    """Selected rows of an EXL3 PLE table decoded to BF16 (reference
    ops.py:1301-1323)."""
    ensure_extension()
    torch.ops._exl3_C.ple_decode_out(packed_rows, global_ids, head_bias, head_offsets,
                                     head_vocab_sizes, owner_lo, owner_hi, bits, out)


def decode(trellis: torch.Tensor, bits_x2: int, codebook: int) -> torch.Tensor:
    """The exact FP16 weights W [padded_in, padded_out] of a packed matrix."""
    ensure_extension()
    out = torch.empty(16 * trellis.shape[0], 16 * trellis.shape[1], dtype=torch.float16,
                      device=trellis.device)
    torch.ops._exl3_C.exl3_decode(trellis, bits_x2, codebook, out)
    return out


_scratch: dict = {}


def _linear_scratch(device: torch.device) -> torch.Tensor:
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream)
    buf = _scratch.get(key)
    if buf is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("EXL3 scratch must be allocated before graph capture")
        buf = torch.empty(LINEAR_SCRATCH_ELEMENTS, dtype=torch.float32, device=device)
        _scratch[key] = buf
    return buf


def exl3_linear(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                bits_x2: int, codebook: int, logical_out: int, row_chunk: int | None = None,
                out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """torch.ops.vllm.exl3_linear of the reference (ops.py:1455-1486): the
    dense linear over row chunks of a fixed per-stream scratch."""
    ensure_extension()
    if row_chunk is None:
        row_chunk = linear_row_chunk(suh.numel(), svh.numel())
    workspace = _linear_scratch(x.device)
    out = torch.empty((x.shape[0], logical_out), dtype=out_dtype, device=x.device)
    for start in range(0, x.shape[0], row_chunk):
        linear_out(x[start:start + row_chunk], trellis, suh, svh, bits_x2, codebook,
                   x.shape[1], logical_out, out[start:start + row_chunk], workspace)
    return out
