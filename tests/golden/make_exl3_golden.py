"""Writes tests/golden/exl3_golden.npz: small EXL3 fixtures (one 128 x 128
matrix per format listed) with their exact decoded FP16 weights and the
BF16 outputs of the reference's dense linear, both computed by the NumPy
statement of the format and of the linear's FP32 steps in tests/exl3_spec.py
(the reference test's specification restated, with an exactly rounded FMA
chain), not by the C oracle they pin.  The reference ships no numeric
goldens for this path; rerun to regenerate:

    python tests/golden/make_exl3_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.exl3_spec import f32_to_bf16_bits, spec_linear_bf16, spec_weight  # noqa: E402

FORMATS = [(8, 2), (4, 1), (6, 2), (3, 2), (16, 1), (2, 2)]


def main() -> None:
    arrays = {}
    for bits_x2, codebook in FORMATS:
        rng = np.random.default_rng(4242 + 10 * bits_x2 + codebook)
        name = f"b{bits_x2}c{codebook}"
        trellis = rng.integers(-(2 ** 15), 2 ** 15, (8, 8, 8 * bits_x2)).astype(np.int16)
        suh = rng.standard_normal(128).astype(np.float16)
        svh = (rng.standard_normal(128) * 0.05).astype(np.float16)
        x = f32_to_bf16_bits(rng.standard_normal((2, 120)).astype(np.float32))
        logical_out = 100
        arrays[name + "_format"] = np.array([bits_x2, codebook], np.int64)
        arrays[name + "_trellis"] = trellis
        arrays[name + "_suh"] = suh
        arrays[name + "_svh"] = svh
        arrays[name + "_x"] = x
        arrays[name + "_logical_out"] = np.array(logical_out, np.int64)
        arrays[name + "_weight"] = spec_weight(trellis, bits_x2, codebook).view(np.uint16)
        arrays[name + "_out"] = spec_linear_bf16(x, trellis, suh, svh, bits_x2, codebook, logical_out)
    np.savez_compressed(os.path.join(HERE, "exl3_golden.npz"), **arrays)


if __name__ == "__main__":
    main()
