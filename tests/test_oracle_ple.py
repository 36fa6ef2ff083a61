"""Pins the PLE oracle (oracle/ple_oracle.py) on the CPU.

  * the ring mapping: a per-bit pure-Python loop over the format statement
    (state bit m <- ring bit ((c - m // bits) mod dim) * bits + m % bits,
    ring bit p = bit p % 16 of word p // 16) on small rows;
  * the codebook of every 16-bit state: the decoder's FP32 steps equal one
    FP64 rounding to FP16 and the dense EXL3 mul1 codebook (an FP16 FMA) of
    the C oracle, so the FP32 sum never double-rounds;
  * the outputs within BF16 rounding of an FP64 evaluation, the reference
    test's bound (test_exl3_ple_decode.py:103-112);
  * masks: owner shards sum to the full rows, a NaN scale gives NaN only on
    owned rows, masked rows are exactly zero.
"""

import numpy as np
import pytest

from oracle import exl3_oracle as X
from oracle import ple_oracle as P
from tests.ple_cases import LAYOUTS, NAN_SCALE, synthetic


def _loop_states(packed, bits, dim):
    out = np.zeros((len(packed), dim), np.uint32)
    for r, row in enumerate(packed.view(np.uint16)):
        for c in range(dim):
            s = 0
            for m in range(16):
                back = m // bits
                src = c - back if c >= back else dim - (back - c)
                bit = src * bits + m % bits
                s |= ((int(row[1 + bit // 16]) >> (bit % 16)) & 1) << m
            out[r, c] = s
    return out


@pytest.mark.parametrize("bits,dim,sizes", LAYOUTS + [(16, 4, (2,)), (1, 32, (4,)), (8, 6, (3,))])
def test_states_match_per_bit_loop(bits, dim, sizes):
    packed, *_ = synthetic(bits, dim, sizes, seed=bits + dim)
    assert np.array_equal(P.states(packed[:12], bits, dim), _loop_states(packed[:12], bits, dim))


def test_codebook_every_state():
    states = np.arange(65536, dtype=np.uint32)
    mine = P.codebook(states).view(np.uint16)
    dense = np.array([X.lib().oracle_exl3_codebook(int(s), 2) for s in states], np.uint16)
    assert np.array_equal(mine, dense)
    p = (states.astype(np.uint64) * np.uint64(P.MUL1)) & np.uint64(0xFFFFFFFF)
    t = sum((p >> np.uint64(s)) & np.uint64(255) for s in (0, 8, 16, 24)).astype(np.float64)
    once = ((1024.0 + t) * float(P.K_INV) + float(P.K_BIAS)).astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, once)
    assert float(P.codebook(np.array([0], np.uint32))[0]) == -3.453125


@pytest.mark.parametrize("bits,dim,sizes", LAYOUTS)
@pytest.mark.parametrize("owner", ["all", "lower", "upper"])
def test_decode_within_bf16_of_fp64(bits, dim, sizes, owner):
    packed, ids, bias, offsets, sizes, rows = synthetic(bits, dim, sizes, seed=bits)
    middle = sizes[0] + 1
    lo, hi = {"all": (0, rows), "lower": (0, middle), "upper": (middle, rows)}[owner]
    out = X.bf16_bits_to_f32(P.decode(packed, ids, bias, offsets, sizes, lo, hi, bits)).astype(np.float64)
    head = P.owned_heads(ids, offsets, sizes, lo, hi)
    valid = head >= 0
    assert valid.any() and not valid.all()
    assert np.all(out[~valid] == 0.0)
    code = P.codebook(P.states(packed, bits, dim)).astype(np.float64)
    scale = packed[:, 0].view(np.float16).astype(np.float64)[:, None]
    row_bias = bias[np.maximum(head, 0)].astype(np.float64)
    ref = code * scale + row_bias
    terms = np.abs(code * scale) + np.abs(row_bias)
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -22 * terms + 1e-30
    assert np.all(np.abs(out - ref)[valid] <= bound[valid])


@pytest.mark.parametrize("bits,dim,sizes", LAYOUTS)
def test_owner_shards_and_nan_scale(bits, dim, sizes):
    packed, ids, bias, offsets, sizes, rows = synthetic(bits, dim, sizes, seed=7)
    middle = rows // 2
    f = lambda lo, hi, p=packed: X.bf16_bits_to_f32(P.decode(p, ids, bias, offsets, sizes, lo, hi, bits))
    assert np.array_equal(f(0, middle) + f(middle, rows), f(0, rows))
    poisoned = packed.copy()
    poisoned[:, 0] = NAN_SCALE
    out = f(0, sizes[0], poisoned)
    owned = np.array([0 <= i < sizes[0] for i in ids])
    assert np.isnan(out[owned]).all() and np.all(out[~owned] == 0.0)
