"""Fused Marlin int4 MoE forward on gfx950.

The launch sequence of the reference's decode path
(vllm_sm80/kernels/marlin_moe/decode.py:301-339) and of upstream
fused_marlin_moe: deterministic block alignment -> w13 grouped GEMM (FP32
k-split partials) -> SwiGLU with the optional clamp -> w2 grouped GEMM with
the router weight (RN(RN(sum) * RN(w))) -> slot-order top-k sum.  Rounding
points are the reference's; the block size and the w13 K split are chosen
here for gfx950 (one aligned block holds up to 64 tokens of one expert, so
an expert's weights are streamed once per block).

Weights: w1 int32 [E, K/16, 4N] (gate columns 0..N-1, up N..2N-1), w2
int32 [E, N/16, 2K], scales [E, K/128, 2N] / [E, N/128, K] of the
activation dtype, hidden_states [M, K] bf16 or fp16.
"""

from __future__ import annotations

import math

import torch

from . import _C
from . import split_align as split_align_mod
from ..moe.align import align_sizes, kernel_moe_align_block_size
from ..moe.routing import moe_sum


def choose_block_size(tokens: int, topk: int, experts: int) -> int:
    """Tokens per aligned block: enough that most experts fit in one block
    (their weights are then read once), at most 64."""
    per_expert = tokens * topk / max(experts, 1)
    for bs, limit in ((8, 4), (16, 10), (32, 22)):
        if per_expert <= limit:
            return bs
    return 64


def choose_w13_ksplit(blocks: int, n13: int, k: int, bs: int, target: int = 768) -> int:
    """K split of the w13 GEMM: enough workgroups to cover the GPU, at least
    one 128-k group per wavefront."""
    groups = k // 128
    tiles_per_wg = 1 if bs <= 32 else 4
    wgs = max(1, blocks) * max(1, n13 // 64 // tiles_per_wg)
    ksplit = 1
    waves_k = 4 if bs <= 32 else 1
    while (wgs * ksplit < target and groups % (2 * ksplit) == 0
           and groups // (2 * ksplit) >= waves_k):
        ksplit *= 2
    return ksplit


def workspace_shapes(tokens: int, topk: int, hidden: int, inter: int, experts: int,
                     block_size: int, ksplit: int, direct: bool = False) -> dict:
    slots = tokens * topk
    size, blocks = align_sizes(slots, experts, block_size)
    shapes = {"sorted": (size,), "expert_ids": (blocks,), "ntpp": (1,), "h": (slots, inter),
              "c3": (slots, hidden)}
    if direct:
        shapes["xp"] = (tokens, hidden)
    else:
        shapes["part"] = (ksplit * slots * 2 * inter,)
    return shapes


# workgroups the direct w13 must have to be chosen (tuned on MI355X)
_DIRECT_MIN_WORKGROUPS = 384


def direct_applies(tokens: int, topk: int, hidden: int, inter: int, experts: int,
                   block_size: int) -> bool:
    """The direct path (k-permuted activations, weights through an LDS ring,
    SwiGLU fused into w13) needs blocks of at most 32 tokens, whole 256-column
    gate / up pairs, and enough routed blocks for its four-tile workgroups
    to fill the GPU (the expected touched experts times the w13 workgroups
    per block)."""
    if block_size > 32 or (2 * inter) % 256 != 0 or hidden % 32 != 0:
        return False
    slots = tokens * topk
    touched = experts * (1.0 - (1.0 - 1.0 / max(experts, 1)) ** slots)
    return touched * (2 * inter // 256) >= _DIRECT_MIN_WORKGROUPS


def marlin_dequant(w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """W [K, N] of one packed matrix (int32 [K/16, 2N], scales [K/128, N]):
    RN((q - 8) * s) through the GEMM's own fragment and dequant code."""
    from ... import _native
    K, N = w.size(0) * 16, w.size(1) // 2
    out = torch.empty((K, N), dtype=s.dtype, device=w.device)
    with torch.cuda.device(w.device):
        status = _native.load().marlin_dequant(
            w.data_ptr(), s.data_ptr(), _C._DTYPE_CODES[s.dtype], K, N, out.data_ptr(),
            torch.cuda.current_stream(w.device).cuda_stream)
    _native.check(status)
    return out


def fused_marlin_moe(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                     w1_scale: torch.Tensor, w2_scale: torch.Tensor, topk_weights: torch.Tensor,
                     topk_ids: torch.Tensor, clamp_limit: float | None = None,
                     expert_map: torch.Tensor | None = None, block_size: int | None = None,
                     ksplit: int | None = None, workspace: dict | None = None,
                     output: torch.Tensor | None = None, path: str | None = None) -> torch.Tensor:
    """out [M, K] = sum over the top-k slots (slot order) of
    RN(RN(w2_e(h)) * RN(router weight)), h = RN(RN(SiLU(min(g, L))) *
    clamp(u, -L, L)), (g | u) = RN(w1_e(x)).  Slots routed outside the local
    experts (id out of range, or mapped to -1) add nothing.

    path: None (automatic), "staged" (activations staged in LDS per
    workgroup, any block size and K split), "direct" (k-permuted
    activations, SwiGLU fused into w13; blocks of at most 32 tokens, K split
    1) or "split" (the staged kernels over the split-cover block lists of
    split_align: one w13 and one w2 launch per list, as the reference's
    prefill.run, marlin_moe/prefill.py:381-447).  All give the same sums: a
    row's sums depend only on its own activations, expert and K split."""
    M, K = hidden_states.shape
    E = w1.size(0)
    N = w2.size(1) * 16
    topk = topk_ids.size(1)
    if w1.shape != (E, K // 16, 4 * N) or w2.shape != (E, N // 16, 2 * K):
        raise RuntimeError("unsupported packed weight layout")
    if w1_scale.shape != (E, K // 128, 2 * N) or w2_scale.shape != (E, N // 128, K):
        raise RuntimeError("scales are not group-128")
    if hidden_states.dtype not in _C._DTYPE_CODES or w1_scale.dtype != hidden_states.dtype \
            or w2_scale.dtype != hidden_states.dtype:
        raise RuntimeError("activations and scales must share a bf16 or fp16 dtype")
    if topk_weights.shape != topk_ids.shape or topk_ids.size(0) != M:
        raise RuntimeError("routing shape mismatch")
    out = output if output is not None else torch.empty_like(hidden_states)
    if M == 0:
        return out
    limit = math.inf if clamp_limit is None else float(clamp_limit)
    slots = M * topk
    ids = topk_ids.to(torch.int32).contiguous()
    local = ids
    if expert_map is not None:
        emap = expert_map.to(torch.int32)
        inside = (ids >= 0) & (ids < emap.numel())
        local = torch.where(inside, emap[torch.where(inside, ids, 0).long()], -1).contiguous()
    bs = block_size or choose_block_size(M, topk, E)
    if path is None:
        direct = ksplit in (None, 1) and direct_applies(M, topk, K, N, E, bs)
    elif path == "split":
        return _split_path(hidden_states, w1, w2, w1_scale, w2_scale, topk_weights, local, out,
                           limit, E, ksplit, workspace)
    elif path in ("direct", "staged"):
        direct = path == "direct"
        if direct and (ksplit not in (None, 1) or bs > 32 or (2 * N) % 256 != 0 or K % 32 != 0):
            raise RuntimeError("the direct path takes blocks of <= 32 tokens, K split 1, "
                               "intermediate % 128 == 0 and hidden % 32 == 0")
    else:
        raise RuntimeError(f"unknown path {path!r}")
    blocks_est = min(slots, E)
    ks = 1 if direct else (ksplit or choose_w13_ksplit(blocks_est, 2 * N, K, bs))
    shapes = workspace_shapes(M, topk, K, N, E, bs, ks, direct)
    ws = workspace if workspace is not None else {}
    buf = {}
    for name, shape in shapes.items():
        dtype = {"part": torch.float32, "h": hidden_states.dtype, "xp": hidden_states.dtype,
                 "c3": hidden_states.dtype}.get(name, torch.int32)
        t = ws.get(name)
        numel = math.prod(shape)
        if t is None or t.numel() < numel or t.dtype != dtype:
            t = torch.empty(numel, dtype=dtype, device=hidden_states.device)
            ws[name] = t
        buf[name] = t.view(-1)[:numel].view(shape)
    tw = topk_weights.to(torch.float32).contiguous().view(-1)
    if direct:
        # the alignment and the w13 GEMM's k-permuted input in one launch
        _C.align_permute(local, E, bs, buf["sorted"], buf["expert_ids"], buf["ntpp"], hidden_states,
                         buf["xp"])
        _C.gemm_direct(buf["xp"], w1, w1_scale, buf["sorted"], buf["expert_ids"], buf["ntpp"], None,
                       topk, slots, K, 2 * N, bs, _C.MODE_SWIGLU, 1, limit, out=buf["h"])
        _C.gemm_direct(buf["h"], w2, w2_scale, buf["sorted"], buf["expert_ids"], buf["ntpp"], tw, 1,
                       slots, N, K, bs, _C.MODE_TOPK, 1, out=buf["c3"])
        moe_sum(buf["c3"].view(M, topk, K), out, local, E)
        return out
    if M == 1 and path is None:
        # one token: its top-k slots route to distinct experts, so each slot
        # is its own block (identity routing, no alignment launch)
        sorted_ids, expert_ids, ntpp = None, local.view(-1), None
    else:
        kernel_moe_align_block_size(local, E, bs, buf["sorted"], buf["expert_ids"], buf["ntpp"],
                                    None, None)
        sorted_ids, expert_ids, ntpp = buf["sorted"], buf["expert_ids"], buf["ntpp"]
    if N % 64 == 0:
        # the w13 partials and their SwiGLU in one launch
        _C.w13_act(hidden_states, w1, w1_scale, sorted_ids, expert_ids, ntpp, local.view(-1),
                   topk, slots, K, 2 * N, bs, ks, limit, buf["part"], buf["h"])
    else:
        _C.gemm(hidden_states, w1, w1_scale, sorted_ids, expert_ids, ntpp, None,
                topk, slots, K, 2 * N, bs, _C.MODE_PARTIAL, ks, part=buf["part"])
        _C.act(buf["part"], local.view(-1), ks, slots, N, limit, buf["h"])
    if sorted_ids is None:
        # identity routing: the w2 rows and their top-k sum in one launch
        _C.w2_sum(buf["h"], w2, w2_scale, expert_ids, tw, topk, slots, N, K, bs, buf["c3"], out)
        return out
    _C.gemm(buf["h"], w2, w2_scale, sorted_ids, expert_ids, ntpp, tw, 1, slots,
            N, K, bs, _C.MODE_TOPK, 1, out=buf["c3"])
    moe_sum(buf["c3"].view(M, topk, K), out, local, E)
    return out


def _split_path(hidden_states, w1, w2, w1_scale, w2_scale, topk_weights, local, out, limit, E,
                ksplit, workspace):
    """The staged kernels over the split-cover lists (prefill.py:381-447's
    run): every routed row is computed once, in the block list its expert's
    cover puts it in."""
    M, K = hidden_states.shape
    N = w2.size(1) * 16
    topk = local.size(1)
    slots = M * topk
    ws = workspace if workspace is not None else {}
    key = ("split", slots, E, hidden_states.device)
    sbuf = ws.get(key)
    if sbuf is None:
        sbuf = split_align_mod.buffers(slots, E, hidden_states.device)
        ws[key] = sbuf
    lists = split_align_mod.split_align(local, E, sbuf)
    ks = ksplit or choose_w13_ksplit(min(slots, E), 2 * N, K, 64)
    shapes = {"part": (ks * slots * 2 * N,), "h": (slots, N), "c3": (slots, K)}
    buf = {}
    for name, shape in shapes.items():
        dtype = torch.float32 if name == "part" else hidden_states.dtype
        numel = math.prod(shape)
        t = ws.get(name)
        if t is None or t.numel() < numel or t.dtype != dtype:
            t = torch.empty(numel, dtype=dtype, device=hidden_states.device)
            ws[name] = t
        buf[name] = t.view(-1)[:numel].view(shape)
    tw = topk_weights.to(torch.float32).contiguous().view(-1)
    for bs, sorted_ids, expert_ids, ntpp in lists:
        _C.gemm(hidden_states, w1, w1_scale, sorted_ids, expert_ids, ntpp, None, topk, slots, K,
                2 * N, bs, _C.MODE_PARTIAL, ks, part=buf["part"])
    _C.act(buf["part"], local.view(-1), ks, slots, N, limit, buf["h"])
    for bs, sorted_ids, expert_ids, ntpp in lists:
        _C.gemm(buf["h"], w2, w2_scale, sorted_ids, expert_ids, ntpp, tw, 1, slots, N, K, bs,
                _C.MODE_TOPK, 1, out=buf["c3"])
    moe_sum(buf["c3"].view(M, topk, K), out, local, E)
    return out
