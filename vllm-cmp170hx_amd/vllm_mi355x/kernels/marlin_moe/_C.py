"""The ``_ampere_marlin_C`` operator library on ROCm: the reference's schemas
(csrc/ampere_marlin/decode_orig.cu:403-411, decode_v2.cu:395-399,
prefill_tiles.cu:12-26), each implemented by a call into libvllm_mi355x.so
with the tensors' device pointers on torch's current stream.

The reference's tuning arguments (decode ``rows`` beyond the K split it
implies, ``cfg``; prefill ``thread_k`` / ``thread_n`` / ``blocks_per_sm``,
``c_tmp``, ``redo``, ``workspace``) select among its compiled sm_80 tiles;
here one grouped kernel serves every shape, so they are accepted and checked
for type only.  The work counters ``ctr`` are left as they are (zero).
"""

from __future__ import annotations

import math

import torch

from ... import _native

_DTYPE_CODES = {torch.bfloat16: _native.BF16, torch.float16: _native.FP16}

MODE_PARTIAL, MODE_STORE, MODE_TOPK, MODE_SWIGLU = 0, 1, 2, 3

# build_info keys (ampere_marlin/module.cpp:9-15): abi_version 1, prefill
# schedule version 2 (extension.py:47).
ABI_VERSION = 1
PREFILL_SCHEDULE_VERSION = 2

SCHEMAS = {
    "decode_gemm_orig": (
        "decode_gemm_orig(Tensor a, Tensor w, Tensor s, Tensor sorted, Tensor eids, Tensor ntpp, "
        "Tensor topk_w, int topk, int n_slots, int K, int N, bool w13, int rows, int cfg, "
        "Tensor(c!) ctr, Tensor(o!) out) -> int"),
    "decode_gemm_v2": (
        "decode_gemm_v2(Tensor a, Tensor w, Tensor s, Tensor sorted, Tensor eids, Tensor ntpp, "
        "Tensor topk_w, int topk, int n_slots, int K, int N, bool w13, int rows, int cfg, "
        "Tensor(c!) ctr, Tensor(o!) out) -> int"),
    "decode_act_orig": (
        "decode_act_orig(Tensor part, Tensor ids, int ksplit, int n_slots, int Nh, float limit, "
        "Tensor(h!) h) -> ()"),
    "prefill_tile_gemm": (
        "prefill_tile_gemm(Tensor(a!) a, Tensor? c_or_none, Tensor(b!) b_q_weight, "
        "Tensor? b_bias_or_none, Tensor(d!) b_scales, Tensor? a_scales, Tensor? global_scale, "
        "Tensor? b_zeros_or_none, Tensor(e!) workspace, Tensor sorted_token_ids, "
        "Tensor(f!) expert_ids, Tensor(g!) num_tokens_past_padded, Tensor(h!) topk_weights, "
        "int moe_block_size, int top_k, bool mul_topk_weights, int b_type_id, int size_m, "
        "int size_n, int size_k, bool use_atomic_add, bool use_fp32_reduce, bool is_zp_float, "
        "int thread_k, int thread_n, int blocks_per_sm, Tensor(c!) c_tmp, "
        "Tensor(r!)? redo=None) -> Tensor"),
}

_library = None


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _on(t: torch.Tensor, device: torch.device, name: str) -> None:
    _require(t.is_cuda and t.device == device, f"{name} must be on the activation device")


def gemm(a, w, s, sorted_ids, expert_ids, ntpp, topk_w, top_k, n_slots, K, N, block_size, mode,
         ksplit, part=None, out=None) -> None:
    """marlin_moe_gemm on torch tensors (checks of decode_orig.cu:361-375).
    sorted_ids = ntpp = None: identity routing, block b is slot b alone and
    expert_ids[b] its local expert (one expert id per slot)."""
    _require(a.dtype in _DTYPE_CODES and a.dim() == 2 and a.stride(1) == 1,
             "a: bf16 or fp16, unit inner stride")
    _require(s.dtype == a.dtype, "scales must have the activation dtype")
    _require(w.dtype == torch.int32 and w.is_contiguous() and s.is_contiguous(),
             "weights contiguous")
    _require(w.dim() == 3 and w.size(1) * 16 == K and w.size(2) == 2 * N,
             "w: int32 [E, K/16, 2N]")
    _require(s.dim() == 3 and s.size(0) == w.size(0) and s.size(1) * 128 == K and s.size(2) == N,
             "s: [E, K/128, N]")
    identity = sorted_ids is None
    _require(identity == (ntpp is None), "sorted ids and num_tokens_post_pad come together")
    _require(expert_ids.dtype == torch.int32 and expert_ids.is_contiguous() and
             (identity or (sorted_ids.dtype == torch.int32 and ntpp.dtype == torch.int32)),
             "routing dtypes")
    for t, name in ((w, "w"), (s, "s"), (sorted_ids, "sorted"), (expert_ids, "eids"),
                    (ntpp, "ntpp")):
        if t is not None:
            _on(t, a.device, name)
    if topk_w is not None:
        _require(topk_w.dtype == torch.float32 and topk_w.is_contiguous(), "topk weights fp32")
        _on(topk_w, a.device, "topk_w")
    lib = _native.load()
    if out is not None:
        _on(out, a.device, "out")
        _require(out.dtype == a.dtype and out.dim() == 2 and out.stride(1) == 1,
                 "out: activation dtype, unit inner stride")
    if part is not None:
        _on(part, a.device, "part")
        _require(part.dtype == torch.float32 and part.is_contiguous(), "w13 partial buffer")
    with torch.cuda.device(a.device):
        status = lib.marlin_moe_gemm(
            a.data_ptr(), _DTYPE_CODES[a.dtype], a.size(0), a.stride(0), w.data_ptr(),
            s.data_ptr(), w.size(0), 0 if identity else sorted_ids.data_ptr(),
            0 if identity else sorted_ids.numel(),
            expert_ids.data_ptr(), expert_ids.numel(), 0 if identity else ntpp.data_ptr(),
            0 if topk_w is None else topk_w.data_ptr(), int(top_k), int(n_slots), int(K), int(N),
            int(block_size), int(mode), int(ksplit),
            0 if part is None else part.data_ptr(), 0 if part is None else part.numel(),
            0 if out is None else out.data_ptr(), 0 if out is None else out.stride(0),
            0 if out is None else out.size(0), _stream(a.device))
    _native.check(status)


def gemm_direct(a_perm, w, s, sorted_ids, expert_ids, ntpp, topk_w, top_k, n_slots, K, N,
                block_size, mode, ksplit=1, limit=math.inf, part=None, out=None) -> None:
    """marlin_moe_gemm_direct on torch tensors: gemm's contract on k-permuted
    activations (permute_act), plus mode MODE_SWIGLU (out = h, permuted)."""
    _require(a_perm.dtype in _DTYPE_CODES and a_perm.dim() == 2 and a_perm.stride(1) == 1,
             "a: bf16 or fp16, unit inner stride")
    _require(s.dtype == a_perm.dtype and w.dtype == torch.int32 and w.is_contiguous()
             and s.is_contiguous(), "weights contiguous, scales of the activation dtype")
    _require(w.dim() == 3 and w.size(1) * 16 == K and w.size(2) == 2 * N, "w: int32 [E, K/16, 2N]")
    _require(s.dim() == 3 and s.size(0) == w.size(0) and s.size(1) * 128 == K and s.size(2) == N,
             "s: [E, K/128, N]")
    for t, name in ((w, "w"), (s, "s"), (sorted_ids, "sorted"), (expert_ids, "eids"),
                    (ntpp, "ntpp")):
        _on(t, a_perm.device, name)
    if topk_w is not None:
        _require(topk_w.dtype == torch.float32 and topk_w.is_contiguous(), "topk weights fp32")
    if out is not None:
        _require(out.dtype == a_perm.dtype and out.dim() == 2 and out.stride(1) == 1,
                 "out: activation dtype, unit inner stride")
    if part is not None:
        _require(part.dtype == torch.float32 and part.is_contiguous(), "w13 partial buffer")
    lib = _native.load()
    with torch.cuda.device(a_perm.device):
        status = lib.marlin_moe_gemm_direct(
            a_perm.data_ptr(), _DTYPE_CODES[a_perm.dtype], a_perm.size(0), a_perm.stride(0),
            w.data_ptr(), s.data_ptr(), w.size(0), sorted_ids.data_ptr(), sorted_ids.numel(),
            expert_ids.data_ptr(), expert_ids.numel(), ntpp.data_ptr(),
            0 if topk_w is None else topk_w.data_ptr(), int(top_k), int(n_slots), int(K), int(N),
            int(block_size), int(mode), int(ksplit), float(limit),
            0 if part is None else part.data_ptr(), 0 if part is None else part.numel(),
            0 if out is None else out.data_ptr(), 0 if out is None else out.stride(0),
            0 if out is None else out.size(0), _stream(a_perm.device))
    _native.check(status)


def permute_act(a, out) -> None:
    """marlin_permute_act: out[r][p(k)] = a[r][k], the k order gemm_direct reads."""
    _require(a.dtype in _DTYPE_CODES and out.dtype == a.dtype and a.dim() == 2 and out.dim() == 2
             and a.stride(1) == 1 and out.stride(1) == 1 and out.shape == a.shape,
             "a, out: same shape and dtype, unit inner stride")
    _on(out, a.device, "out")
    lib = _native.load()
    with torch.cuda.device(a.device):
        status = lib.marlin_permute_act(a.data_ptr(), _DTYPE_CODES[a.dtype], a.size(0), a.size(1),
                                        a.stride(0), out.data_ptr(), out.stride(0),
                                        _stream(a.device))
    _native.check(status)


def align_permute(topk_ids, num_experts, block_size, sorted_ids, expert_ids, ntpp, a, out) -> None:
    """marlin_moe_align_permute: the deterministic alignment of topk_ids and
    permute_act(a, out) in one launch."""
    _require(topk_ids.dtype == torch.int32 and topk_ids.is_contiguous(), "topk_ids: int32")
    for t, name in ((sorted_ids, "sorted_ids"), (expert_ids, "expert_ids"), (ntpp, "ntpp")):
        _require(t.dtype == torch.int32 and t.is_contiguous(), f"{name}: contiguous int32")
        _on(t, topk_ids.device, name)
    _require(a.dtype in _DTYPE_CODES and out.dtype == a.dtype and a.dim() == 2 and out.dim() == 2
             and a.stride(1) == 1 and out.stride(1) == 1 and out.shape == a.shape,
             "a, out: same shape and dtype, unit inner stride")
    _on(a, topk_ids.device, "a")
    _on(out, topk_ids.device, "out")
    with torch.cuda.device(a.device):
        status = _native.load().marlin_moe_align_permute(
            topk_ids.data_ptr(), topk_ids.numel(), int(num_experts), int(block_size), None,
            sorted_ids.data_ptr(), sorted_ids.numel(), expert_ids.data_ptr(), expert_ids.numel(),
            ntpp.data_ptr(), a.data_ptr(), _DTYPE_CODES[a.dtype], a.size(0), a.size(1), a.stride(0),
            out.data_ptr(), out.stride(0), _stream(a.device))
    _native.check(status)


def w13_act(a, w, s, sorted_ids, expert_ids, ntpp, ids, top_k, n_slots, K, N, block_size, ksplit,
            limit, part, h) -> None:
    """marlin_moe_w13_act on torch tensors: gemm(..., MODE_PARTIAL, ksplit,
    part=part) then act(part, ids, ksplit, n_slots, N // 2, limit, h), in one
    launch while arrival counters are free."""
    _require(a.dtype in _DTYPE_CODES and a.dim() == 2 and a.stride(1) == 1,
             "a: bf16 or fp16, unit inner stride")
    _require(s.dtype == a.dtype, "scales must have the activation dtype")
    _require(w.dtype == torch.int32 and w.is_contiguous() and s.is_contiguous(),
             "weights contiguous")
    _require(w.dim() == 3 and w.size(1) * 16 == K and w.size(2) == 2 * N,
             "w: int32 [E, K/16, 2N]")
    _require(s.dim() == 3 and s.size(0) == w.size(0) and s.size(1) * 128 == K and s.size(2) == N,
             "s: [E, K/128, N]")
    identity = sorted_ids is None
    _require(identity == (ntpp is None), "sorted ids and num_tokens_post_pad come together")
    _require(expert_ids.dtype == torch.int32 and expert_ids.is_contiguous() and
             ids.dtype == torch.int32 and ids.is_contiguous() and ids.numel() >= n_slots and
             (identity or (sorted_ids.dtype == torch.int32 and ntpp.dtype == torch.int32)),
             "routing dtypes")
    for t, name in ((w, "w"), (s, "s"), (sorted_ids, "sorted"), (expert_ids, "eids"),
                    (ntpp, "ntpp"), (ids, "ids"), (part, "part"), (h, "h")):
        if t is not None:
            _on(t, a.device, name)
    _require(part.dtype == torch.float32 and part.is_contiguous(), "w13 partial buffer")
    _require(h.dtype == a.dtype and h.dim() == 2 and h.is_contiguous() and h.size(1) == N // 2,
             "h: activation dtype, contiguous rows of N / 2")
    with torch.cuda.device(a.device):
        status = _native.load().marlin_moe_w13_act(
            a.data_ptr(), _DTYPE_CODES[a.dtype], a.size(0), a.stride(0), w.data_ptr(),
            s.data_ptr(), w.size(0), 0 if identity else sorted_ids.data_ptr(),
            0 if identity else sorted_ids.numel(),
            expert_ids.data_ptr(), expert_ids.numel(), 0 if identity else ntpp.data_ptr(),
            ids.data_ptr(), int(top_k), int(n_slots), int(K), int(N), int(block_size),
            int(ksplit), float(limit), part.data_ptr(), part.numel(), h.data_ptr(), h.stride(0),
            h.size(0), _stream(a.device))
    _native.check(status)


def w2_sum(a, w, s, expert_ids, topk_w, top_k, n_slots, K, N, block_size, c3, out) -> None:
    """marlin_moe_w2_sum on torch tensors, identity routing (block b is slot b,
    expert_ids[b] its local expert, a one row per slot): gemm(..., MODE_TOPK,
    out=c3) then moe_sum(c3 as [n_slots / top_k, top_k, N], out, expert_ids),
    in one launch while arrival counters are free."""
    _require(a.dtype in _DTYPE_CODES and a.dim() == 2 and a.stride(1) == 1,
             "a: bf16 or fp16, unit inner stride")
    _require(s.dtype == a.dtype, "scales must have the activation dtype")
    _require(w.dtype == torch.int32 and w.is_contiguous() and s.is_contiguous(),
             "weights contiguous")
    _require(w.dim() == 3 and w.size(1) * 16 == K and w.size(2) == 2 * N,
             "w: int32 [E, K/16, 2N]")
    _require(s.dim() == 3 and s.size(0) == w.size(0) and s.size(1) * 128 == K and s.size(2) == N,
             "s: [E, K/128, N]")
    _require(expert_ids.dtype == torch.int32 and expert_ids.is_contiguous(), "routing dtypes")
    _require(topk_w.dtype == torch.float32 and topk_w.is_contiguous(), "topk weights fp32")
    _require(c3.dtype == a.dtype and c3.is_contiguous() and c3.numel() >= n_slots * N,
             "c3: contiguous slot rows of N")
    _require(out.dtype == a.dtype and out.is_contiguous() and out.numel() >= n_slots // top_k * N,
             "out: contiguous token rows of N")
    for t, name in ((w, "w"), (s, "s"), (expert_ids, "eids"), (topk_w, "topk_w"), (c3, "c3"),
                    (out, "out")):
        _on(t, a.device, name)
    with torch.cuda.device(a.device):
        status = _native.load().marlin_moe_w2_sum(
            a.data_ptr(), _DTYPE_CODES[a.dtype], a.size(0), a.stride(0), w.data_ptr(),
            s.data_ptr(), w.size(0), expert_ids.data_ptr(), expert_ids.numel(),
            topk_w.data_ptr(), int(top_k), int(n_slots), int(K), int(N), int(block_size),
            c3.data_ptr(), int(N), c3.numel() // N, out.data_ptr(), _stream(a.device))
    _native.check(status)


def act(part, ids, ksplit, n_slots, nh, limit, h) -> None:
    """marlin_moe_act on torch tensors."""
    _require(part.dtype == torch.float32 and part.is_contiguous(), "part: fp32")
    _require(ids.dtype == torch.int32 and ids.is_contiguous(), "ids: int32")
    _require(h.dtype in _DTYPE_CODES and h.is_contiguous(), "h: bf16 or fp16")
    _require(part.numel() >= ksplit * n_slots * 2 * nh and h.numel() >= n_slots * nh
             and ids.numel() >= n_slots, "act: buffers too small")
    _on(ids, part.device, "ids")
    _on(h, part.device, "h")
    with torch.cuda.device(part.device):
        status = _native.load().marlin_moe_act(part.data_ptr(), ids.data_ptr(), int(ksplit),
                                               int(n_slots), int(nh), float(limit), h.data_ptr(),
                                               _DTYPE_CODES[h.dtype], _stream(part.device))
    _native.check(status)


def decode_gemm_orig_impl(a, w, s, sorted, eids, ntpp, topk_w, topk, n_slots, K, N, w13, rows,
                          cfg, ctr, out) -> int:
    """w13: FP32 partials part[ks][slot][N] with ksplit = K / 16 / rows;
    w2 (one k-slice, rows = K / 16): out[slot][N] = RN(RN(sum) * RN(w)).
    Returns ksplit (decode_orig.cu:377-401)."""
    _require(a.is_cuda, "a must be CUDA")
    _require(a.dtype in _DTYPE_CODES and a.stride(1) == 1 and a.stride(0) % 2 == 0,
             "a: bf16, unit inner stride, even row stride")
    _require(K % 128 == 0 and N % 64 == 0, "K % 128, N % 64")
    _require(topk_w.dtype == torch.float32 and sorted.dtype == torch.int32
             and eids.dtype == torch.int32 and ntpp.dtype == torch.int32, "routing dtypes")
    _require(ctr.dtype == torch.int32 and ctr.numel() >= 2 and ctr.is_contiguous(),
             "ctr: 2 int32 work counters, zero before the first call")
    _require(rows > 0 and (K // 16) % rows == 0, "K must be a multiple of R k16 rows")
    ksplit = K // 16 // rows
    _require((K // 128) % ksplit == 0, f"unsupported rows={rows} w13={w13} cfg={cfg}")
    if w13:
        _require(out.dtype == torch.float32 and out.numel() >= ksplit * n_slots * N,
                 "w13 partial buffer")
        gemm(a, w, s, sorted, eids, ntpp, topk_w, topk, n_slots, K, N, 8, MODE_PARTIAL, ksplit,
             part=out)
    else:
        _require(ksplit == 1 and out.dtype == a.dtype and out.numel() >= n_slots * N, "w2 output")
        gemm(a, w, s, sorted, eids, ntpp, topk_w, 1, n_slots, K, N, 8, MODE_TOPK, 1,
             out=out.view(-1)[:n_slots * N].view(n_slots, N))
    return ksplit


def decode_act_orig_impl(part, ids, ksplit, n_slots, Nh, limit, h) -> None:
    _require(ksplit > 0 and Nh > 0, "act: ksplit > 0, Nh > 0")
    act(part, ids, ksplit, n_slots, Nh, limit, h)


def prefill_tile_gemm_impl(a, c_or_none, b_q_weight, b_bias_or_none, b_scales, a_scales,
                           global_scale, b_zeros_or_none, workspace, sorted_token_ids, expert_ids,
                           num_tokens_past_padded, topk_weights, moe_block_size, top_k,
                           mul_topk_weights, b_type_id, size_m, size_n, size_k, use_atomic_add,
                           use_fp32_reduce, is_zp_float, thread_k, thread_n, blocks_per_sm, c_tmp,
                           redo=None):
    """The Marlin MoE GEMM (upstream moe_wna16_marlin_gemm contract) for
    uint4b8 group-128 weights without zero points, bias or activation
    scales: C[sid][n] = RN(sum_k a[sid / top_k][k] W_e[k][n]) (times the
    router weight, RN, if mul_topk_weights) for every routed sid."""
    _require(a.is_cuda, "a must be CUDA")
    _require(b_bias_or_none is None and a_scales is None and global_scale is None
             and b_zeros_or_none is None and not is_zp_float,
             "only uint4b8 group-128 weights without zero points, bias or activation scales")
    _require(a.dim() == 2 and a.size(1) == size_k and a.size(0) >= size_m, "a: [size_m, size_k]")
    n_slots = size_m * top_k
    if c_or_none is None:
        c = torch.empty((n_slots, size_n), dtype=a.dtype, device=a.device)
    else:
        c = c_or_none
        _require(c.numel() >= n_slots * size_n, "c too small")
        c = c.view(-1)[:n_slots * size_n].view(n_slots, size_n)
    gemm(a, b_q_weight, b_scales, sorted_token_ids, expert_ids, num_tokens_past_padded,
         topk_weights.reshape(-1) if mul_topk_weights else None, top_k, n_slots, size_k, size_n,
         moe_block_size, MODE_TOPK if mul_topk_weights else MODE_STORE, 1, out=c)
    return c


def build_info() -> dict:
    """The handshake of ampere_marlin/module.cpp:9-15; ROCm has no CUDA
    runtime, so cuda_version is 0 and hip_version is set."""
    hip = torch.version.hip or "0.0"
    major, minor = (int(v) for v in hip.split(".")[:2])
    return {
        "abi_version": ABI_VERSION,
        "torch_version": torch.__version__.split("+")[0],
        "cuda_version": 0,
        "hip_version": major * 1000 + minor * 10,
        "cxx11_abi": int(torch._C._GLIBCXX_USE_CXX11_ABI),
        "prefill_schedule_version": PREFILL_SCHEDULE_VERSION,
    }


def register() -> None:
    """Defines the _ampere_marlin_C operators once per process."""
    global _library
    if _library is not None:
        return
    _native.load()
    lib = torch.library.Library("_ampere_marlin_C", "DEF")
    for schema in SCHEMAS.values():
        lib.define(schema)
    lib.impl("decode_gemm_orig", decode_gemm_orig_impl, "CUDA")
    lib.impl("decode_gemm_v2", decode_gemm_orig_impl, "CUDA")
    lib.impl("decode_act_orig", decode_act_orig_impl, "CUDA")
    lib.impl("prefill_tile_gemm", prefill_tile_gemm_impl, "CUDA")
    _library = lib
