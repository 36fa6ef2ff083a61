"""Seeded synthetic EXL3 matrices and helpers shared by the tests.

Data as the reference's tests and the benchmark configurations make them:
uniform int16 trellis words, suh / svh fp16 sign-times-scale vectors,
activations ~N(0, 1).
"""

from __future__ import annotations

import numpy as np

# Every format the reference accepts (csrc/exl3/gemm.cu:17-20).
FORMATS = [(b, 1) for b in range(2, 17, 2)] + [(b, 2) for b in (2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16)]


def random_matrix(rng: np.random.Generator, padded_in: int, padded_out: int, bits_x2: int,
                  scales: str = "sign"):
    """trellis int16 [K/16, N/16, 8*bits_x2], suh fp16 [K], svh fp16 [N].

    scales="sign": +-1 times N(1, 0.05) (the benchmark data);
    scales="test": suh ~ N(0, 1), svh ~ 0.05 N(0, 1) (the reference's tests,
    test_exl3_kernels.py:174-180)."""
    trellis = rng.integers(-(2 ** 15), 2 ** 15, (padded_in // 16, padded_out // 16, 8 * bits_x2),
                           dtype=np.int64).astype(np.int16)
    if scales == "sign":
        suh = (rng.choice([-1.0, 1.0], padded_in) * rng.normal(1.0, 0.05, padded_in)).astype(np.float16)
        svh = (rng.choice([-1.0, 1.0], padded_out) * rng.normal(1.0, 0.05, padded_out)).astype(np.float16)
    else:
        suh = rng.standard_normal(padded_in).astype(np.float16)
        svh = (rng.standard_normal(padded_out) * 0.05).astype(np.float16)
    return trellis, suh, svh


def bf16_bits(a: np.ndarray) -> np.ndarray:
    from oracle.exl3_oracle import f32_to_bf16_bits
    return f32_to_bf16_bits(a)


def random_acts(rng: np.random.Generator, rows: int, cols: int, dtype: str):
    """Activations ~N(0,1): (array for the oracle, dtype code, numpy view).
    BF16 is carried as uint16 bit patterns."""
    v = rng.standard_normal((rows, cols)).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits(v), 0
    return v.astype(np.float16), 1
