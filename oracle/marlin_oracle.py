"""NumPy bindings of the CPU Marlin int4 MoE oracle in marlin_oracle.c.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the checker;
the product path (vllm-cmp170hx_amd/) never does.

Arrays follow the reference operators' layouts (decode_orig.cu:10-19):
  w13  int32 [E, K/16, 4N]   s13  act [E, K/128, 2N]   (gate | up columns)
  w2   int32 [E, N/16, 2K]   s2   act [E, N/128, K]
  x / out act [M, K]; act = bf16 (uint16 bit patterns) or fp16.
Dtype codes: 0 = bf16, 1 = fp16 (the C-ABI's codes).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_marlin.so")
_lib = None

BF16, FP16 = 0, 1


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        c = ctypes
        _lib = c.CDLL(_LIB_PATH)
        P, I64 = c.c_void_p, c.c_int64
        _lib.oracle_marlin_unpack.restype = None
        _lib.oracle_marlin_unpack.argtypes = [P, I64, I64, P]
        _lib.oracle_marlin_pack.restype = None
        _lib.oracle_marlin_pack.argtypes = [P, I64, I64, P]
        _lib.oracle_marlin_scale_pos.restype = I64
        _lib.oracle_marlin_scale_pos.argtypes = [I64]
        _lib.oracle_marlin_dequant.restype = None
        _lib.oracle_marlin_dequant.argtypes = [P, P, I64, I64, c.c_int, P]
        _lib.oracle_marlin_moe.restype = c.c_int
        _lib.oracle_marlin_moe.argtypes = [P, c.c_int, I64, I64, I64, P, P, I64, I64, P, P, P, P,
                                           c.c_float, P, P, P]
        _lib.oracle_moe_align.restype = c.c_int
        _lib.oracle_moe_align.argtypes = [P, I64, I64, I64, P, P, I64, P, I64, P]
    return _lib


def _ptr(a) -> int:
    return 0 if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def unpack(w: np.ndarray, K: int, N: int) -> np.ndarray:
    """q uint8 [K, N] (values 0..15) of one packed matrix int32 [K/16, 2N]."""
    w = _c(w, np.int32)
    q = np.empty((K, N), np.uint8)
    lib().oracle_marlin_unpack(_ptr(w), K, N, _ptr(q))
    return q


def pack(q: np.ndarray) -> np.ndarray:
    """int32 [K/16, 2N] of q uint8 [K, N]."""
    q = _c(q, np.uint8)
    K, N = q.shape
    w = np.empty((K // 16, 2 * N), np.int32)
    lib().oracle_marlin_pack(_ptr(q), K, N, _ptr(w))
    return w


def scale_positions(N: int) -> np.ndarray:
    """Stored position of each logical column of a scale row."""
    return np.array([lib().oracle_marlin_scale_pos(c) for c in range(N)], np.int64)


def dequant(w: np.ndarray, s: np.ndarray, K: int, N: int, dtype: int) -> np.ndarray:
    """W [K, N] in the activation dtype (uint16 bit patterns)."""
    w, s = _c(w, np.int32), _c(s, np.uint16)
    out = np.empty((K, N), np.uint16)
    lib().oracle_marlin_dequant(_ptr(w), _ptr(s), K, N, dtype, _ptr(out))
    return out


def moe(x, dtype, ids, weights, w13, s13, w2, s2, limit=float("inf"), want_intermediate=False):
    """The fused MoE forward (align, w13, activation, w2 x router weight,
    slot-order sum).  x, s13, s2: uint16 bit patterns of the act dtype."""
    x, ids = _c(x, np.uint16), _c(ids, np.int32)
    weights = _c(weights, np.float32)
    w13, w2 = _c(w13, np.int32), _c(w2, np.int32)
    s13, s2 = _c(s13, np.uint16), _c(s2, np.uint16)
    M, K = x.shape
    E, topk = w13.shape[0], ids.shape[1]
    N = w2.shape[1] * 16
    out = np.empty((M, K), np.uint16)
    h1 = np.zeros((M * topk, 2 * N), np.uint16) if want_intermediate else None
    h = np.zeros((M * topk, N), np.uint16) if want_intermediate else None
    rc = lib().oracle_marlin_moe(_ptr(x), dtype, M, K, N, _ptr(ids), _ptr(weights), topk, E,
                                 _ptr(w13), _ptr(s13), _ptr(w2), _ptr(s2), float(limit),
                                 _ptr(out), _ptr(h1), _ptr(h))
    if rc != 0:
        raise MemoryError("oracle marlin moe failed")
    return (out, h1, h) if want_intermediate else out


def align_sizes(numel: int, num_experts: int, block_size: int) -> tuple[int, int]:
    """(sorted size, block count) as moe_align_block_size sizes its outputs."""
    max_pad = numel + num_experts * (block_size - 1)
    if numel < num_experts:
        max_pad = min(numel * block_size, max_pad)
    return max_pad, (max_pad + block_size - 1) // block_size


def align(ids: np.ndarray, num_experts: int, block_size: int, expert_map=None):
    """(sorted_ids, expert_ids, ntpp) of the deterministic alignment."""
    ids = _c(ids, np.int32).reshape(-1)
    size, blocks = align_sizes(ids.size, num_experts, block_size)
    sorted_ids = np.empty(size, np.int32)
    expert_ids = np.empty(blocks, np.int32)
    ntpp = np.empty(1, np.int32)
    emap = None if expert_map is None else _c(expert_map, np.int32)
    rc = lib().oracle_moe_align(_ptr(ids), ids.size, num_experts, block_size, _ptr(emap),
                                _ptr(sorted_ids), size, _ptr(expert_ids), blocks, _ptr(ntpp))
    if rc != 0:
        raise ValueError("padded total exceeds the sorted size")
    return sorted_ids, expert_ids, ntpp
