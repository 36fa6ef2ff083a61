"""Synthetic PLE rows as the reference's decoder test makes them
(tests/models/qwen4_exp/test_exl3_ple_decode.py:33-38, :128-153): layouts
(bits per channel, channels, head vocabulary sizes), ids covering every head
row, padding rows past the table, negative and out-of-range ids, and random
packed words everywhere (a decoder must not read masked rows)."""

from __future__ import annotations

import numpy as np

LAYOUTS = [(6, 160, (97, 40, 13)), (3, 32, (5, 9)), (5, 16, (3, 3, 3, 3))]
NAN_SCALE = 0x7E00


def synthetic(bits: int, dim: int, sizes, seed: int, extra_ids=()):
    rng = np.random.default_rng(seed)
    offsets = [sum(sizes[:i]) for i in range(len(sizes))]
    end = sum(sizes)
    rows = end + 5  # head padding rows
    ids = [*range(rows), -1, -(1 << 40), rows, rows + 1000, *rng.integers(0, end, 8).tolist(),
           *extra_ids]
    words = 1 + dim * bits // 16
    packed = rng.integers(-(1 << 15), 1 << 15, (len(ids), words), dtype=np.int16)
    magnitude = rng.uniform(0.05, 2.0, len(ids)) * rng.choice((-1, 1), len(ids))
    packed[:, 0] = magnitude.astype(np.float16).view(np.int16)
    bias = rng.normal(0, 0.5, (len(sizes), dim)).astype(np.float16)
    return packed, ids, bias, offsets, list(sizes), rows
