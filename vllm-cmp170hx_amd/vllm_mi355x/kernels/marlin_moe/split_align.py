"""Split-cover MoE block alignment for the Marlin int4 MoE at prefill sizes
(vllm_sm80/kernels/marlin_moe/split_align.py:173-224: ``SIZES``, ``COST``,
``cover_table``, ``buffers``, ``split_align``).

Padding every expert's rows to one block size wastes most of the last block
of each expert when experts hold a few dozen rows.  Here the routed rows are
sorted by expert into one block list per size in ``SIZES``; an expert with r
rows gets the cheapest multiset of blocks covering r under the per-block
cost model ``COST``, its rows (stable flat order) fill its largest blocks
first, and only its last block is padded.  One Marlin GEMM launch per list
then computes every routed row exactly once.

The lists are built on the device by one workgroup (``moe_split_align`` in
libvllm_mi355x.so): counts, the cover from the table, per-list exclusive
scans over experts, expert ids per block, and the stable scatter.  No host
sync and fixed buffers, so the call is graph-capturable; calls that share a
buffer set must be ordered on one stream.
"""

from __future__ import annotations

import torch

from ... import _native

SIZES = (64, 48, 32, 16)
# per-block cost of one Marlin m-block pass over w13 and w2 (the reference's
# model, split_align.py:45-46); only relative values matter
COST = {64: 33.3, 48: 26.4, 32: 20.3, 16: 14.1}


def cover_table(R: int) -> torch.Tensor:
    """int32 [R + 1, len(SIZES)] (CPU): blocks of each size in the cheapest
    cover of r rows, r = 0..R.  Dynamic programme over r; among equally cheap
    choices the smaller block size is taken for the last block."""
    best = [0.0] * (R + 1)
    last = [0] * (R + 1)
    for r in range(1, R + 1):
        choice = None
        for size in SIZES:
            cand = (COST[size] + best[max(r - size, 0)], size)
            if choice is None or cand < choice:
                choice = cand
        best[r], last[r] = choice
    table = [[0] * len(SIZES)]
    for r in range(1, R + 1):
        row = list(table[max(r - last[r], 0)])
        row[SIZES.index(last[r])] += 1
        table.append(row)
    return torch.tensor(table, dtype=torch.int32)


def buffers(t_max: int, E: int, device: torch.device) -> dict:
    """Scratch for ``split_align`` at up to ``t_max`` routed rows (M * topk)."""
    return {
        "t_max": t_max,
        "E": E,
        "tab": cover_table(t_max).to(device),
        "s": [torch.empty(t_max + bs * E, device=device, dtype=torch.int32) for bs in SIZES],
        "e": [torch.empty((t_max + bs * E) // bs + 1, device=device, dtype=torch.int32)
              for bs in SIZES],
        "ntpp": torch.empty(len(SIZES), device=device, dtype=torch.int32),
        "numels": torch.tensor([[t_max + bs * E for bs in SIZES],
                                [(t_max + bs * E) // bs + 1 for bs in SIZES]], dtype=torch.int64),
    }


def split_align(topk_ids: torch.Tensor, E: int, buf: dict,
                expert_map: torch.Tensor | None = None):
    """-> [(block_size, sorted_ids, expert_ids, ntpp_1elem)], one per size in
    ``SIZES``, in the buffers ``buf`` (from ``buffers``)."""
    ids = topk_ids.reshape(-1)
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    ids = ids.contiguous()
    T = ids.numel()
    if not (0 < T <= buf["t_max"]) or E != buf["E"]:
        raise RuntimeError("split_align buffers too small")
    if not ids.is_cuda:
        raise ValueError("the split alignment needs GPU tensors")
    emap = None
    if expert_map is not None:
        emap = expert_map.to(torch.int32).contiguous()
        if emap.numel() < E or emap.device != ids.device:
            raise RuntimeError("expert_map needs E entries on the ids' device")
    s, e, ntpp = buf["s"], buf["e"], buf["ntpp"]
    numels = buf["numels"]
    with torch.cuda.device(ids.device):
        status = _native.load().moe_split_align(
            ids.data_ptr(), T, int(E), 0 if emap is None else emap.data_ptr(),
            buf["tab"].data_ptr(), buf["tab"].size(0) - 1,
            s[0].data_ptr(), s[1].data_ptr(), s[2].data_ptr(), s[3].data_ptr(),
            numels[0].data_ptr(),
            e[0].data_ptr(), e[1].data_ptr(), e[2].data_ptr(), e[3].data_ptr(),
            numels[1].data_ptr(), ntpp.data_ptr(),
            torch.cuda.current_stream(ids.device).cuda_stream)
    _native.check(status)
    return [(bs, s[k], e[k], ntpp[k:k + 1]) for k, bs in enumerate(SIZES)]
