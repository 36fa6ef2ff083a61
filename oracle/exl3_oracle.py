"""NumPy bindings of the CPU oracle in exl3_oracle.c.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the checker;
the product path (vllm-cmp170hx_amd/) never does.

Arrays follow the reference operators' layouts:
  trellis  int16  [padded_in/16, padded_out/16, 8*bits_x2]
  suh/svh  fp16   [padded_in] / [padded_out]
  x / out  bf16 (as uint16 bit patterns), fp16 or fp32, row-major
Dtype codes: 0 = bf16, 1 = fp16, 2 = fp32 (the same codes as the C-ABI).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_exl3.so")
_lib = None

BF16, FP16, FP32 = 0, 1, 2


def build() -> str:
    """Compiles the oracle library with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        c = ctypes
        _lib.oracle_f32_to_f16.restype = c.c_uint16
        _lib.oracle_f32_to_f16.argtypes = [c.c_float]
        _lib.oracle_f16_to_f32.restype = c.c_float
        _lib.oracle_f16_to_f32.argtypes = [c.c_uint16]
        _lib.oracle_f32_to_bf16.restype = c.c_uint16
        _lib.oracle_f32_to_bf16.argtypes = [c.c_float]
        _lib.oracle_bf16_to_f32.restype = c.c_float
        _lib.oracle_bf16_to_f32.argtypes = [c.c_uint16]
        _lib.oracle_exl3_state.restype = c.c_uint32
        _lib.oracle_exl3_state.argtypes = [c.c_void_p, c.c_int, c.c_int]
        _lib.oracle_exl3_codebook.restype = c.c_uint16
        _lib.oracle_exl3_codebook.argtypes = [c.c_uint32, c.c_int]
        _lib.oracle_exl3_lane_row.restype = c.c_int
        _lib.oracle_exl3_lane_row.argtypes = [c.c_int]
        _lib.oracle_exl3_lane_col.restype = c.c_int
        _lib.oracle_exl3_lane_col.argtypes = [c.c_int]
        _lib.oracle_exl3_decode.restype = None
        _lib.oracle_exl3_decode.argtypes = [c.c_void_p, c.c_int64, c.c_int64, c.c_int,
                                            c.c_int, c.c_void_p]
        _lib.oracle_exl3_h128.restype = None
        _lib.oracle_exl3_h128.argtypes = [c.c_void_p]
        _lib.oracle_exl3_linear_out.restype = c.c_int
        _lib.oracle_exl3_linear_out.argtypes = [
            c.c_void_p, c.c_int, c.c_int64, c.c_int64, c.c_void_p, c.c_void_p, c.c_void_p,
            c.c_int64, c.c_int64, c.c_int, c.c_int, c.c_int64, c.c_void_p, c.c_int, c.c_void_p]
        _lib.oracle_exl3_moe_out.restype = c.c_int
        _lib.oracle_exl3_moe_out.argtypes = [
            c.c_void_p, c.c_int, c.c_int64, c.c_int64, c.c_void_p, c.c_void_p, c.c_int64,
            c.c_void_p, c.c_void_p, c.c_int64, c.c_void_p, c.c_int64, c.c_int64, c.c_float,
            c.c_void_p, c.c_int]
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- scalar formats ----------------------------------------------------------

def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even FP32 -> BF16, as uint16 bit patterns."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def act_to_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == BF16:
        return bf16_bits_to_f32(a)
    return np.asarray(a).astype(np.float32)


# ---- EXL3 format -------------------------------------------------------------

def state(tile: np.ndarray, bits_x2: int, index: int) -> int:
    tile = np.ascontiguousarray(tile, dtype=np.int16)
    return int(lib().oracle_exl3_state(_ptr(tile), bits_x2, index))


def codebook(state_value: int, codebook_id: int) -> np.float16:
    bits = lib().oracle_exl3_codebook(state_value, codebook_id)
    return np.array(bits, np.uint16).view(np.float16)[()]


def decode(trellis: np.ndarray, bits_x2: int, codebook_id: int) -> np.ndarray:
    """Decoded FP16 weights W [padded_in, padded_out] (rows = k, cols = n)."""
    trellis = np.ascontiguousarray(trellis, dtype=np.int16)
    tk, tn, words = trellis.shape
    assert words == 8 * bits_x2
    w = np.empty((16 * tk, 16 * tn), np.uint16)
    lib().oracle_exl3_decode(_ptr(trellis), tk, tn, bits_x2, codebook_id, _ptr(w))
    return w.view(np.float16)


def h128(v: np.ndarray) -> np.ndarray:
    """The reference's FP32 H128 butterfly, over the last axis (a multiple of 128)."""
    out = np.ascontiguousarray(v, dtype=np.float32).copy()
    flat = out.reshape(-1, 128)
    for row in flat:
        lib().oracle_exl3_h128(row.ctypes.data)
    return out


def linear_out(x: np.ndarray, x_dtype: int, trellis: np.ndarray, suh: np.ndarray,
               svh: np.ndarray, bits_x2: int, codebook_id: int, logical_out: int,
               out_dtype: int = BF16, want_core: bool = False):
    """The reference's bit-exact dense linear.  x: [rows, logical_in] (uint16
    BF16 bits, float16 or float32).  Returns out (uint16 bits for BF16,
    float16, float32) and, with want_core, the FP32 core rows [rows, padded_out]."""
    x = np.ascontiguousarray(x)
    trellis = np.ascontiguousarray(trellis, dtype=np.int16)
    suh = np.ascontiguousarray(suh, dtype=np.float16)
    svh = np.ascontiguousarray(svh, dtype=np.float16)
    rows, logical_in = x.shape
    pin, pout = trellis.shape[0] * 16, trellis.shape[1] * 16
    assert suh.size == pin and svh.size == pout
    out = np.empty((rows, logical_out),
                   {BF16: np.uint16, FP16: np.float16, FP32: np.float32}[out_dtype])
    core = np.empty((rows, pout), np.float32) if want_core else None
    rc = lib().oracle_exl3_linear_out(
        _ptr(x), x_dtype, rows, logical_in, _ptr(trellis), _ptr(suh), _ptr(svh), pin, pout,
        bits_x2, codebook_id, logical_out, _ptr(out), out_dtype,
        _ptr(core) if want_core else None)
    if rc != 0:
        raise MemoryError("oracle linear_out failed")
    return (out, core) if want_core else out


class MoELayer:
    """Host copies of a layer's local experts: gate/up/down per expert, each
    (trellis, suh, svh, bits_x2, codebook), with the packed_ptrs / packed_meta
    tables the reference operator takes (host addresses here)."""

    def __init__(self, experts):
        self.experts = [[(np.ascontiguousarray(t, np.int16), np.ascontiguousarray(u, np.float16),
                          np.ascontiguousarray(v, np.float16), int(b), int(c))
                         for (t, u, v, b, c) in projections] for projections in experts]
        e = len(self.experts)
        self.ptrs = np.zeros((max(e, 1), 3, 3), np.int64)
        self.meta = np.zeros((max(e, 1), 3, 4), np.int64)
        for i, projections in enumerate(self.experts):
            for p, (t, u, v, b, c) in enumerate(projections):
                self.ptrs[i, p] = [t.ctypes.data, u.ctypes.data, v.ctypes.data]
                self.meta[i, p] = [t.shape[0] * 16, t.shape[1] * 16, b, c]


def moe_out(x: np.ndarray, x_dtype: int, topk_ids: np.ndarray, topk_weights: np.ndarray,
            layer: MoELayer, expert_map: np.ndarray, intermediate: int,
            swiglu_limit: float = 0.0, out_dtype: int = BF16) -> np.ndarray:
    """The reference's MoE operator (moe_out_reference) on the host."""
    x = np.ascontiguousarray(x)
    ids = np.ascontiguousarray(topk_ids, dtype=np.int64)
    w = np.ascontiguousarray(topk_weights, dtype=np.float32)
    emap = np.ascontiguousarray(expert_map, dtype=np.int64)
    rows, hidden = x.shape
    out = np.empty((rows, hidden), {BF16: np.uint16, FP16: np.float16, FP32: np.float32}[out_dtype])
    rc = lib().oracle_exl3_moe_out(
        _ptr(x), x_dtype, rows, hidden, _ptr(ids), _ptr(w), ids.shape[1],
        _ptr(layer.ptrs), _ptr(layer.meta), len(layer.experts), _ptr(emap), emap.size,
        intermediate, float(swiglu_limit), _ptr(out), out_dtype)
    if rc != 0:
        raise MemoryError("oracle moe_out failed")
    return out
