"""Synthetic EXL3 checkpoints for the ingestion tests (safetensors files
written with the safetensors library)."""

import json
import struct

import numpy as np
import torch
from safetensors.torch import save_file

MUL1, MCG = 0x83DCD12D, 0xCBAC1FED


def marker(value):
    return torch.tensor(struct.unpack("<i", struct.pack("<I", value))[0], dtype=torch.int32)


def matrix_tensors(rng, prefix, k, n, bits_x2, codebook):
    trellis = torch.from_numpy(rng.integers(-(2 ** 15), 2 ** 15, (k // 16, n // 16, 8 * bits_x2),
                                            dtype=np.int64).astype(np.int16))
    suh = torch.from_numpy(rng.standard_normal(k).astype(np.float16))
    svh = torch.from_numpy((0.05 * rng.standard_normal(n)).astype(np.float16))
    out = {f"{prefix}.trellis": trellis, f"{prefix}.suh": suh, f"{prefix}.svh": svh}
    out[f"{prefix}.{'mul1' if codebook == 2 else 'mcg'}"] = marker(MUL1 if codebook == 2 else MCG)
    return out


def write(directory, files, index=None):
    """files: {filename: {name: tensor}}; index: {name: filename} or None."""
    for fname, tensors in files.items():
        save_file({k: v.contiguous() for k, v in tensors.items()}, str(directory / fname))
    if index is not None:
        (directory / "model.safetensors.index.json").write_text(json.dumps({"weight_map": index}))
