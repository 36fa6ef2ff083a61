"""CPU oracle of the EXL3 PLE row decoder (test infrastructure only: used by
tests/ as the checker, never by the library).

A NumPy restatement of the reference's selected-row decoder,
csrc/exl3/ple.cu:49-147 (ple_decode_kernel) with its host masks, as the
reference's own test states the format
(tests/models/qwen4_exp/test_exl3_ple_decode.py:1-12, :43-80):

  * a row is one FP16 scale word, then a little-endian ring of dim * bits
    bits (ring bit p is bit p % 16 of ring word p // 16);
  * channel c's 16-bit state takes bit m from ring bit
    ((c - m // bits) mod dim) * bits + m % bits;
  * codebook: p = state * 0x83DCD12D mod 2^32, t = byte sum of p, value =
    RN16(RN32(RN32(1024 + t) * fp16(0x1EEE)) + fp16(0xC931)) (the FP32
    product is exact, the FP32 sum rounds once, then FP16);
  * out = RN_bf16(RN32(RN32(value * scale) + head_bias[head][c])) for a row
    whose id is owned (owner_lo <= id < owner_hi) and inside the vocabulary
    of the last head starting at or before it; every other row is 0.

Pinned by tests/test_oracle_ple.py: a per-bit pure-Python loop on small
rows, the codebook of every byte sum against the dense mul1 codebook of the
C oracle and an FP64 single rounding, the reference test's FP64 bound, and
the masks' closed forms (owner shards sum to the full row, a NaN scale
poisons only owned rows).
"""

from __future__ import annotations

import numpy as np

MUL1 = 0x83DCD12D
K_INV = np.float32(np.array([0x1EEE], np.uint16).view(np.float16)[0])
K_BIAS = np.float32(np.array([0xC931], np.uint16).view(np.float16)[0])


def states(packed: np.ndarray, bits: int, dim: int) -> np.ndarray:
    """uint32 [rows, dim] trellis states of the rows' rings."""
    words = packed.view(np.uint16)[:, 1:].astype(np.uint64)
    ring = ((words[:, :, None] >> np.arange(16, dtype=np.uint64)) & np.uint64(1)).reshape(len(packed), -1)
    channels = np.arange(dim)
    state = np.zeros((len(packed), dim), np.uint64)
    for m in range(16):
        source = ((channels - m // bits) % dim) * bits + m % bits
        state |= ring[:, source] << np.uint64(m)
    return state.astype(np.uint32)


def codebook(state: np.ndarray) -> np.ndarray:
    """float16 values of states (the decoder's FP32 steps)."""
    p = (state.astype(np.uint64) * np.uint64(MUL1)) & np.uint64(0xFFFFFFFF)
    t = sum((p >> np.uint64(s)) & np.uint64(255) for s in (0, 8, 16, 24))
    v = (1024 + t).astype(np.float32) * K_INV  # exact: 11 x 11 significant bits
    return (v + K_BIAS).astype(np.float32).astype(np.float16)


def owned_heads(ids, offsets, sizes, owner_lo: int, owner_hi: int) -> np.ndarray:
    """Head index of each row (-1: masked), ple.cu:51-75 and its owner test."""
    ids = np.asarray(ids, np.int64)
    offsets = np.asarray(offsets, np.int64)
    sizes = np.asarray(sizes, np.int64)
    head = np.searchsorted(offsets, ids, side="right") - 1
    clipped = np.clip(head, 0, len(offsets) - 1)
    ok = ((ids >= 0) & (ids >= owner_lo) & (ids < owner_hi) & (head >= 0)
          & (offsets[clipped] >= 0) & (sizes[clipped] > 0) & (ids - offsets[clipped] >= 0)
          & (ids - offsets[clipped] < sizes[clipped]))
    return np.where(ok, clipped, -1)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even BF16 bit patterns (NaN kept quiet)."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
    r = np.where(nan, (u >> np.uint64(16)) | np.uint64(0x40), r)
    return r.astype(np.uint16)


def decode(packed, ids, bias, offsets, sizes, owner_lo: int, owner_hi: int, bits: int) -> np.ndarray:
    """BF16 bit patterns [rows, dim] of ple_decode_out."""
    packed = np.ascontiguousarray(packed, np.int16)
    bias = np.asarray(bias, np.float16)
    dim = bias.shape[1]
    head = owned_heads(ids, offsets, sizes, owner_lo, owner_hi)
    value = codebook(states(packed, bits, dim)).astype(np.float32)
    scale = packed[:, 0].view(np.float16).astype(np.float32)[:, None]
    with np.errstate(invalid="ignore", over="ignore"):
        out = (value * scale).astype(np.float32) + bias[np.maximum(head, 0)].astype(np.float32)
    bits_out = f32_to_bf16_bits(out.astype(np.float32))
    bits_out[head < 0] = 0
    return bits_out
