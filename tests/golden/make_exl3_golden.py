"""Writes tests/golden/exl3_golden.npz: small EXL3 fixtures (one 128x128
matrix per format listed) with their exact decoded FP16 weights and the
bit-exact BF16 outputs of the reference's dense linear, computed by the CPU
oracle (itself pinned by tests/test_oracle_exl3.py against an independent
NumPy statement of the format).  The reference ships no numeric goldens for
this path, so these are generated here; rerun to regenerate:

    python tests/golden/make_exl3_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import exl3_oracle as O  # noqa: E402

FORMATS = [(8, 2), (4, 1), (6, 2), (3, 2), (16, 1), (2, 2)]


def main() -> None:
    arrays = {}
    for bits_x2, codebook in FORMATS:
        rng = np.random.default_rng(4242 + 10 * bits_x2 + codebook)
        name = f"b{bits_x2}c{codebook}"
        trellis = rng.integers(-(2 ** 15), 2 ** 15, (8, 8, 8 * bits_x2)).astype(np.int16)
        suh = rng.standard_normal(128).astype(np.float16)
        svh = (rng.standard_normal(128) * 0.05).astype(np.float16)
        x = O.f32_to_bf16_bits(rng.standard_normal((2, 120)).astype(np.float32))
        logical_out = 100
        arrays[name + "_format"] = np.array([bits_x2, codebook], np.int64)
        arrays[name + "_trellis"] = trellis
        arrays[name + "_suh"] = suh
        arrays[name + "_svh"] = svh
        arrays[name + "_x"] = x
        arrays[name + "_logical_out"] = np.array(logical_out, np.int64)
        arrays[name + "_weight"] = O.decode(trellis, bits_x2, codebook).view(np.uint16)
        arrays[name + "_out"] = O.linear_out(x, O.BF16, trellis, suh, svh, bits_x2, codebook,
                                             logical_out)
    np.savez_compressed(os.path.join(HERE, "exl3_golden.npz"), **arrays)


if __name__ == "__main__":
    main()
