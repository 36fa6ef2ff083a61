"""The ``_exl3_C`` operator library on ROCm: the reference's schemas
(csrc/exl3/module.cpp:12-67), each CUDA kernel implemented by a call into
libvllm_mi355x.so with the tensors' device pointers on torch's current
stream.  Tensor-level checks (device, dtype, contiguity, rank) are made here
with the reference's messages (csrc/exl3/common.h:42-61, dense.cu:85-93);
geometry, workspace and overlap checks are made by the native library.
"""

from __future__ import annotations

import os

import torch

from ... import _native

_DTYPE_CODES = {torch.bfloat16: _native.BF16, torch.float16: _native.FP16,
                torch.float32: _native.FP32}

# Bumped with the reference's own meaning (module.cpp:86-88): 3 = moe_out_v2
# takes bits_x2, 2 = the MoE operators take swiglu_limit.
ABI_VERSION = 3

SCHEMAS = {
    "linear_out": (
        "linear_out(Tensor x, Tensor trellis, Tensor suh, Tensor svh, "
        "int bits_x2, int codebook, int logical_in, int logical_out, "
        "Tensor(a!) out, Tensor(b!) workspace) -> ()"),
    "linear_out_splitk": (
        "linear_out_splitk(Tensor x, Tensor trellis, Tensor suh, Tensor svh, "
        "int bits_x2, int codebook, int logical_in, int logical_out, "
        "Tensor(a!) out, Tensor(b!) workspace) -> ()"),
    "linear_workspace_size": (
        "linear_workspace_size(int max_rows, int padded_in, int padded_out) -> int"),
    "linear_splitk_splits": (
        "linear_splitk_splits(int rows, int padded_out, int sms, int bits_x2, "
        "int codebook) -> int"),
    "exl3_decode": (
        "exl3_decode(Tensor trellis, int bits_x2, int codebook, Tensor(a!) out) -> ()"),
    "moe_out": (
        "moe_out(Tensor x, Tensor topk_ids, Tensor topk_weights, "
        "Tensor packed_ptrs, Tensor packed_meta, Tensor expert_map, "
        "int intermediate_size, Tensor(a!) out, Tensor(b!) workspace, "
        "float swiglu_limit=0.0) -> ()"),
    "moe_out_v2": (
        "moe_out_v2(Tensor x, Tensor topk_ids, Tensor topk_weights, "
        "Tensor packed_ptrs, Tensor packed_meta, Tensor expert_map, "
        "int intermediate_size, int bits_x2, Tensor(a!) out, "
        "Tensor(b!) workspace, float swiglu_limit=0.0) -> ()"),
    "moe_workspace_size": (
        "moe_workspace_size(int max_rows, int hidden_size, int intermediate_size, "
        "int topk, int local_experts) -> int"),
    "moe_workspace_size_v2": (
        "moe_workspace_size_v2(int max_rows, int hidden_size, int intermediate_size, "
        "int topk, int local_experts) -> int"),
    # PLE rows: ple_decode_out decodes selected rows on the GPU; ple_read_rows
    # (host file reads, outside this library's matmul path) is registered so
    # the reference's loader finds it, and raises when called.
    "ple_decode_out": (
        "ple_decode_out(Tensor packed_rows, Tensor global_ids, Tensor head_bias, "
        "Tensor head_offsets, Tensor head_vocab_sizes, int owner_lo, "
        "int owner_hi, int bits, Tensor(a!) out) -> ()"),
    "ple_read_rows": (
        "ple_read_rows(int fd, Tensor ids, Tensor(a!) dest, int count, "
        "int base, int row_bytes, int owner_lo, int owner_hi, "
        "Tensor head_offsets, Tensor head_vocab_sizes, int retries, "
        "int max_threads) -> Tensor"),
    "linear_prefill_applies": (
        "linear_prefill_applies(int rows, int padded_in, int padded_out, int bits_x2, "
        "int codebook) -> bool"),
    "set_prefill_schedule": "set_prefill_schedule(int mode) -> ()",
    "set_gemm_shape_override": "set_gemm_shape_override(int shape) -> ()",
    "moe_v2_draft_force_rows": "moe_v2_draft_force_rows(int rows) -> ()",
}

# The reference's variants with the same contracts (module.cpp:13-58 and the
# fragments of dense_prefill_tc.cu:619-631, moe_v2.cu:2234-2250,
# moe_prefill_v2.cu:1162-1175, moe_prefill_try.cu:1381-1399,
# moe_v2_try.cu:1542-1559): each is served by one of the operators above.
_LINEAR_ALIASES = ("linear_out_prefill",)
_MOE_ALIASES = ("moe_out_mixed",)                                  # moe_out's signature
_MOE_V2_ALIASES = ("moe_out_v2_fold", "moe_out_prefill_v2", "moe_out_prefill_try")
_MOE_V2_MIXED = ("moe_out_v2_mixed", "moe_out_prefill_try_mixed")  # any format per expert
_MOE_V2_TRY = ("moe_out_v2_try", "moe_out_v2_try_mixed")          # swiglu_limit required
_SIZE_ALIASES = ("moe_workspace_size_prefill", "moe_workspace_size_prefill_v2",
                 "moe_workspace_size_prefill_try", "moe_workspace_size_v2_try")


def _alias_schema(base: str, name: str) -> str:
    return SCHEMAS[base].replace(f"{base}(", f"{name}(", 1)


for _n in _LINEAR_ALIASES:
    SCHEMAS[_n] = _alias_schema("linear_out", _n)
for _n in _MOE_ALIASES + ("moe_out_prefill",):
    SCHEMAS[_n] = _alias_schema("moe_out", _n)
for _n in _MOE_V2_ALIASES + _MOE_V2_MIXED:
    SCHEMAS[_n] = _alias_schema("moe_out_v2", _n)
for _n in _MOE_V2_TRY:
    SCHEMAS[_n] = _alias_schema("moe_out_v2", _n).replace("float swiglu_limit=0.0",
                                                          "float swiglu_limit")
for _n in _SIZE_ALIASES:
    SCHEMAS[_n] = _alias_schema("moe_workspace_size", _n)

_library = None


def _check_tensor(t: torch.Tensor, x: torch.Tensor, dtypes, name: str) -> None:
    if not (t.is_cuda and t.device == x.device):
        raise RuntimeError(f"{name} must be on the input CUDA device")
    if t.dtype not in dtypes:
        raise RuntimeError(f"{name} has incorrect dtype")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def linear_out_impl(x, trellis, suh, svh, bits_x2, codebook, logical_in, logical_out, out,
                    workspace) -> None:
    if not x.is_cuda:
        raise RuntimeError("EXL3 x must be CUDA")
    _check_tensor(x, x, (torch.bfloat16, torch.float16), "x")
    _check_tensor(trellis, x, (torch.int16,), "trellis")
    _check_tensor(suh, x, (torch.float16,), "suh")
    _check_tensor(svh, x, (torch.float16,), "svh")
    if out.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise RuntimeError("EXL3 linear out must be BF16, FP16 or FP32")
    _check_tensor(out, x, (out.dtype,), "out")
    _check_tensor(workspace, x, (torch.float32,), "workspace")
    if not (x.dim() == 2 and trellis.dim() == 3 and suh.dim() == 1 and svh.dim() == 1
            and out.dim() == 2):
        raise RuntimeError(
            "EXL3 linear requires rank-2 x/out, rank-3 trellis and rank-1 scales")
    lib = _native.load()
    with torch.cuda.device(x.device):
        status = lib.exl3_linear_out(
            x.data_ptr(), _DTYPE_CODES[x.dtype], x.size(0), x.size(1),
            trellis.data_ptr(), trellis.size(0), trellis.size(1), trellis.size(2),
            suh.data_ptr(), suh.numel(), svh.data_ptr(), svh.numel(),
            int(bits_x2), int(codebook), int(logical_in), int(logical_out),
            out.data_ptr(), _DTYPE_CODES[out.dtype], out.size(0), out.size(1),
            workspace.data_ptr(), workspace.numel(), _stream(x.device))
    _native.check(status)


def linear_workspace_size_impl(max_rows, padded_in, padded_out) -> int:
    size = _native.load().exl3_linear_workspace_size(max_rows, padded_in, padded_out)
    if size < 0:
        raise RuntimeError(_native.last_error())
    return int(size)


def linear_splitk_splits_impl(rows, padded_out, sms, bits_x2, codebook) -> int:
    # One operator serves both entry points here: linear_out_splitk runs the
    # linear_out kernels (its contract: same arguments, checks, workspace).
    return 1


def decode_impl(trellis, bits_x2, codebook, out) -> None:
    if not trellis.is_cuda:
        raise RuntimeError("EXL3 trellis must be CUDA")
    _check_tensor(trellis, trellis, (torch.int16,), "trellis")
    _check_tensor(out, trellis, (torch.float16,), "out")
    if trellis.dim() != 3 or out.dim() != 2 or out.size(0) != 16 * trellis.size(0) \
            or out.size(1) != 16 * trellis.size(1):
        raise RuntimeError("EXL3 decode geometry mismatch")
    lib = _native.load()
    with torch.cuda.device(trellis.device):
        status = lib.exl3_decode(trellis.data_ptr(), trellis.size(0), trellis.size(1),
                                 trellis.size(2), int(bits_x2), int(codebook), out.data_ptr(),
                                 _stream(trellis.device))
    _native.check(status)


def _check_integer(t, x, name):
    if t.dtype not in (torch.int32, torch.int64):
        raise RuntimeError(f"{name} must have int32 or int64 dtype")
    _check_tensor(t, x, (t.dtype,), name)


def _moe_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map, intermediate_size,
              bits_x2, out, workspace, swiglu_limit) -> None:
    """Checks of csrc/exl3/moe.cu:323-364, then the native operator."""
    if not x.is_cuda:
        raise RuntimeError("EXL3 x must be CUDA")
    _check_tensor(x, x, (torch.bfloat16, torch.float16), "x")
    _check_integer(topk_ids, x, "topk_ids")
    _check_integer(expert_map, x, "expert_map")
    _check_tensor(topk_weights, x, (torch.float32,), "topk_weights")
    _check_tensor(packed_ptrs, x, (torch.int64,), "packed_ptrs")
    _check_tensor(packed_meta, x, (torch.int64,), "packed_meta")
    _check_tensor(out, x, (x.dtype,), "out")
    _check_tensor(workspace, x, (torch.float32,), "workspace")
    if not (x.dim() == 2 and out.dim() == 2 and topk_ids.dim() == 2 and topk_weights.dim() == 2
            and expert_map.dim() == 1 and packed_ptrs.dim() == 3 and packed_meta.dim() == 3):
        raise RuntimeError("EXL3 MoE tensor ranks mismatch")
    rows, hidden = x.shape
    if not (topk_ids.size(0) == rows and topk_weights.shape == topk_ids.shape
            and out.shape == x.shape):
        raise RuntimeError("EXL3 MoE row/topk/output geometry mismatch")
    experts = packed_ptrs.size(0)
    if not (packed_ptrs.size(1) == 3 and packed_ptrs.size(2) == 3 and packed_meta.size(0) == experts
            and packed_meta.size(1) == 3 and packed_meta.size(2) == 4):
        raise RuntimeError("EXL3 MoE pointer/metadata geometry mismatch")
    lib = _native.load()
    with torch.cuda.device(x.device):
        status = lib.exl3_moe_out(
            x.data_ptr(), _DTYPE_CODES[x.dtype], rows, hidden, topk_ids.data_ptr(),
            int(topk_ids.dtype == torch.int64), topk_weights.data_ptr(), topk_ids.size(1),
            packed_ptrs.data_ptr(), packed_meta.data_ptr(), experts, expert_map.data_ptr(),
            int(expert_map.dtype == torch.int64), expert_map.numel(), int(intermediate_size),
            int(bits_x2), out.data_ptr(), _DTYPE_CODES[out.dtype], workspace.data_ptr(),
            workspace.numel(), float(swiglu_limit), _stream(x.device))
    _native.check(status)


def moe_out_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
                 intermediate_size, out, workspace, swiglu_limit=0.0) -> None:
    _moe_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map, intermediate_size,
              0, out, workspace, swiglu_limit)


# The one rate every routed matrix of a moe_out_prefill call has: the
# reference's operator is built for bits_x2 10 with codebook 2 alone
# (csrc/exl3/moe_prefill.cu:37-40, :169-171).
MOE_PREFILL_BITS_X2 = 10


def moe_out_prefill_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
                         intermediate_size, out, workspace, swiglu_limit=0.0) -> None:
    """moe_out's schema at the reference's prefill operator's one rate: the
    fixed-rate path (tile GEMM for the experts with many routed rows, at
    any hidden / intermediate size); an expert of another format gets NaN
    rows where the reference's kernel traps."""
    _moe_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map, intermediate_size,
              MOE_PREFILL_BITS_X2, out, workspace, swiglu_limit)


def moe_out_v2_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
                    intermediate_size, bits_x2, out, workspace, swiglu_limit=0.0) -> None:
    if int(bits_x2) <= 0:
        raise RuntimeError("EXL3 MoE v2 needs the layer's bits_x2")
    _moe_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map, intermediate_size,
              bits_x2, out, workspace, swiglu_limit)


def moe_workspace_size_impl(max_rows, hidden_size, intermediate_size, topk, local_experts) -> int:
    size = _native.load().exl3_moe_workspace_size(max_rows, hidden_size, intermediate_size, topk,
                                                  local_experts)
    if size < 0:
        raise RuntimeError(_native.last_error())
    return int(size)


def moe_out_v2_mixed_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map,
                          intermediate_size, bits_x2, out, workspace, swiglu_limit=0.0) -> None:
    """The _mixed variants: every expert's own format, decoded at run time."""
    _moe_impl(x, topk_ids, topk_weights, packed_ptrs, packed_meta, expert_map, intermediate_size,
              0, out, workspace, swiglu_limit)


def _ple_check(t, name, dtype, ndim, device) -> None:
    """The reference's per-tensor checks and wording (csrc/exl3/ple.cu:150-165)."""
    if t is None:
        raise RuntimeError(f"ple_decode_out: {name} must be defined")
    if not t.is_cuda:
        raise RuntimeError(f"ple_decode_out: {name} must be a CUDA tensor (use a CUDA/UVA view "
                           "for pinned rows)")
    if t.device != device:
        raise RuntimeError(f"ple_decode_out: {name} must be on the output device")
    if t.dtype != dtype:
        raise RuntimeError(f"ple_decode_out: {name} has an invalid dtype")
    if t.dim() != ndim:
        raise RuntimeError(f"ple_decode_out: {name} must have {ndim} dimensions")
    if not t.is_contiguous():
        raise RuntimeError(f"ple_decode_out: {name} must be contiguous")


def ple_decode_out_impl(packed_rows, global_ids, head_bias, head_offsets, head_vocab_sizes,
                        owner_lo, owner_hi, bits, out) -> None:
    """Selected PLE rows decoded to BF16 (csrc/exl3/ple.cu:167-234)."""
    if out is None or not out.is_cuda:
        raise RuntimeError("ple_decode_out: out must be a defined CUDA tensor")
    device = out.device
    _ple_check(out, "out", torch.bfloat16, 2, device)
    _ple_check(packed_rows, "packed_rows", torch.int16, 2, device)
    _ple_check(global_ids, "global_ids", torch.int64, 1, device)
    _ple_check(head_bias, "head_bias", torch.float16, 2, device)
    _ple_check(head_offsets, "head_offsets", torch.int64, 1, device)
    _ple_check(head_vocab_sizes, "head_vocab_sizes", torch.int64, 1, device)
    rows, dim, heads = global_ids.size(0), out.size(1), head_bias.size(0)
    if not (out.size(0) == rows and packed_rows.size(0) == rows):
        raise RuntimeError("ple_decode_out: packed_rows must be [R, 1 + dim*bits/16] and out must "
                           "be [R, dim], with R = global_ids.numel()")
    if not (heads > 0 and head_bias.size(1) == dim and head_offsets.size(0) == heads
            and head_vocab_sizes.size(0) == heads):
        raise RuntimeError("ple_decode_out: head_bias must be [heads, dim] and offsets/vocab sizes "
                           "must be [heads], with heads > 0")
    lib = _native.load()
    with torch.cuda.device(device):
        status = lib.exl3_ple_decode_out(
            packed_rows.data_ptr(), rows, packed_rows.size(1), global_ids.data_ptr(),
            head_bias.data_ptr(), heads, head_offsets.data_ptr(), head_vocab_sizes.data_ptr(),
            dim, int(owner_lo), int(owner_hi), int(bits), out.data_ptr(), _stream(device))
    _native.check(status)


def ple_read_rows_unavailable(*args, **kwargs):
    raise NotImplementedError(
        "ple_read_rows reads compressed rows from files on the host; it is not part of the gfx950 "
        "quantized-matmul library")


def linear_prefill_applies_impl(rows, padded_in, padded_out, bits_x2, codebook) -> bool:
    """The large-M MFMA GEMM serves every format above the native library's
    own threshold (exl3_linear_prefill_rows), so this answer cannot drift
    from its dispatch."""
    return int(rows) > int(_native.load().exl3_linear_prefill_rows())


def _no_op(*args) -> None:
    """Tuning switches of the reference's sm_80 kernels; one kernel family
    serves every shape here."""


def build_info() -> dict:
    """The handshake the reference's loader compares (module.cpp:91-99);
    ROCm has no CUDA runtime, so cuda_version is 0 and hip_version is set."""
    hip = torch.version.hip or "0.0"
    major, minor = (int(v) for v in hip.split(".")[:2])
    return {
        "abi_version": ABI_VERSION,
        "torch_version": torch.__version__.split("+")[0],
        "cuda_version": 0,
        "hip_version": major * 1000 + minor * 10,
        "cxx11_abi": int(torch._C._GLIBCXX_USE_CXX11_ABI),
    }


def register() -> None:
    """Defines the _exl3_C operators once per process."""
    global _library
    if _library is not None:
        return
    _native.load()
    lib = torch.library.Library("_exl3_C", "DEF")
    for schema in SCHEMAS.values():
        lib.define(schema)
    # torch.classes._exl3_C.PleHostReader / EngramHostFetch (stubs that raise)
    if not os.path.exists(_native.TORCH_CLASSES_PATH):
        raise ImportError(f"{_native.TORCH_CLASSES_PATH} is not built: run "
                          "python vllm-cmp170hx_amd/build.py")
    torch.ops.load_library(_native.TORCH_CLASSES_PATH)
    lib.impl("linear_out", linear_out_impl, "CUDA")
    lib.impl("linear_out_splitk", linear_out_impl, "CUDA")
    lib.impl("exl3_decode", decode_impl, "CUDA")
    lib.impl("moe_out", moe_out_impl, "CUDA")
    lib.impl("moe_out_v2", moe_out_v2_impl, "CUDA")
    lib.impl("linear_workspace_size", linear_workspace_size_impl, "CompositeImplicitAutograd")
    lib.impl("moe_workspace_size", moe_workspace_size_impl, "CompositeImplicitAutograd")
    lib.impl("moe_workspace_size_v2", moe_workspace_size_impl, "CompositeImplicitAutograd")
    lib.impl("linear_splitk_splits", linear_splitk_splits_impl, "CompositeImplicitAutograd")
    for name in _LINEAR_ALIASES:
        lib.impl(name, linear_out_impl, "CUDA")
    for name in _MOE_ALIASES:
        lib.impl(name, moe_out_impl, "CUDA")
    lib.impl("moe_out_prefill", moe_out_prefill_impl, "CUDA")
    for name in _MOE_V2_ALIASES + _MOE_V2_TRY:
        lib.impl(name, moe_out_v2_impl, "CUDA")
    for name in _MOE_V2_MIXED:
        lib.impl(name, moe_out_v2_mixed_impl, "CUDA")
    for name in _SIZE_ALIASES:
        lib.impl(name, moe_workspace_size_impl, "CompositeImplicitAutograd")
    lib.impl("ple_decode_out", ple_decode_out_impl, "CUDA")
    lib.impl("ple_read_rows", ple_read_rows_unavailable, "CompositeImplicitAutograd")
    lib.impl("linear_prefill_applies", linear_prefill_applies_impl, "CompositeImplicitAutograd")
    for name in ("set_prefill_schedule", "set_gemm_shape_override", "moe_v2_draft_force_rows"):
        lib.impl(name, _no_op, "CompositeImplicitAutograd")
    _library = lib
