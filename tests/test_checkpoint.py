"""EXL3 checkpoint ingestion on the CPU (vllm_mi355x/kernels/exl3/checkpoint.py,
the on-disk rules of vllm_sm80/kernels/exl3/utils.py:183-288 and
quant.py:382-466): header inventory, matrix validation and its refusals,
H128-block shards, loading, on synthetic checkpoints written with the
safetensors library."""

import json
import struct

import numpy as np
import pytest
import torch

from tests.checkpoint_cases import MCG, MUL1, marker, matrix_tensors, write
from vllm_mi355x.kernels.exl3 import checkpoint as C


@pytest.fixture()
def ckpt(tmp_path):
    rng = np.random.default_rng(0)
    a = matrix_tensors(rng, "model.layers.0.mlp.up_proj", 256, 384, 8, 2)
    b = matrix_tensors(rng, "model.layers.0.self_attn.o_proj", 384, 256, 4, 1)
    a["model.norm.weight"] = torch.ones(256, dtype=torch.bfloat16)
    write(tmp_path, {"model-00001.safetensors": a, "model-00002.safetensors": b})
    return tmp_path, {**a, **b}


def test_manifest_inventory(ckpt):
    path, tensors = ckpt
    m = C.Exl3Manifest(path)
    assert set(m.tensors) == set(tensors)
    up = m.matrices["model.layers.0.mlp.up_proj"]
    assert (up.padded_in, up.padded_out, up.bits_x2, up.codebook, up.marker) == (256, 384, 8, 2, "mul1")
    o = m.matrices["model.layers.0.self_attn.o_proj"]
    assert (o.padded_in, o.padded_out, o.bits_x2, o.codebook) == (384, 256, 4, 1)
    assert set(m.matrices) == {"model.layers.0.mlp.up_proj", "model.layers.0.self_attn.o_proj"}


def test_load_whole_and_sharded(ckpt):
    path, tensors = ckpt
    m = C.Exl3Manifest(path)
    p = "model.layers.0.mlp.up_proj"
    w = C.load_matrix(m, p, 250, 380)
    assert torch.equal(w.trellis, tensors[f"{p}.trellis"])
    assert torch.equal(w.suh, tensors[f"{p}.suh"]) and torch.equal(w.svh, tensors[f"{p}.svh"])
    # a shard: input blocks [128, 256), output blocks [0, 128) and [256, 384)
    s = C.Exl3PackedWeight(m.matrices[p], 128, 256, slice(128, 256), [slice(0, 128), slice(256, 384)])
    s.load(m)
    t = tensors[f"{p}.trellis"]
    assert torch.equal(s.trellis, torch.cat([t[8:16, 0:8], t[8:16, 16:24]], 1))
    assert torch.equal(s.suh, tensors[f"{p}.suh"][128:256])
    assert torch.equal(s.svh, torch.cat([tensors[f"{p}.svh"][0:128], tensors[f"{p}.svh"][256:384]]))
    with pytest.raises(ValueError, match="not whole H128 blocks"):
        C.Exl3PackedWeight(m.matrices[p], 64, 128, slice(0, 64), [slice(0, 128)])
    with pytest.raises(ValueError, match="does not pad to the stored"):
        m.matrices[p].validate_logical(100, 380)


def test_shard_slices():
    assert C.aligned_shard(1024, 1024, 1, 4) == slice(256, 512)
    assert C.aligned_shard(1000, 1024, 0, 1) == slice(0, 1024)
    with pytest.raises(ValueError):
        C.aligned_shard(1024, 1024, 0, 3)
    # 5 blocks over 2 ranks: chunk 0 takes 3, chunk 1 takes 2; rotation swaps
    assert C.block_shard(640, 640, 0, 2) == slice(0, 384)
    assert C.block_shard(640, 640, 1, 2) == slice(384, 640)
    assert C.block_shard(640, 640, 0, 2, rotation=1) == slice(384, 640)


@pytest.mark.parametrize("case,message", [
    ("multiplier", "holds multiplier"), ("both_markers", "exactly one codebook marker"),
    ("no_marker", "exactly one codebook marker"), ("orphan", "without a trellis"),
    ("trellis_dtype", "must be int16"), ("geometry", "not whole H128 blocks of whole"),
    ("svh_shape", "svh must be fp16"), ("rate", "not a rate of codebook"),
    ("dense_conflict", "both a dense .weight"), ("duplicate", "appears in both"),
    ("index_conflict", "which does not hold it")])
def test_refusals(tmp_path, case, message):
    rng = np.random.default_rng(1)
    p = "layer.proj"
    t = matrix_tensors(rng, p, 128, 128, 4, 2)
    files = {"a.safetensors": t}
    index = None
    if case == "multiplier":
        t[f"{p}.mul1"] = marker(MCG)
    elif case == "both_markers":
        t[f"{p}.mcg"] = marker(MCG)
    elif case == "no_marker":
        del t[f"{p}.mul1"]
    elif case == "orphan":
        t["other.suh"] = torch.zeros(128, dtype=torch.float16)
    elif case == "trellis_dtype":
        t[f"{p}.trellis"] = t[f"{p}.trellis"].to(torch.int32)
    elif case == "geometry":
        t[f"{p}.trellis"] = t[f"{p}.trellis"][:4]
        t[f"{p}.suh"] = t[f"{p}.suh"][:64]
    elif case == "svh_shape":
        t[f"{p}.svh"] = t[f"{p}.svh"][:64]
    elif case == "rate":
        t[f"{p}.trellis"] = torch.zeros(8, 8, 8 * 3, dtype=torch.int16)
        t[f"{p}.mcg"] = marker(MCG)
        del t[f"{p}.mul1"]
    elif case == "dense_conflict":
        t[f"{p}.weight"] = torch.zeros(128, 128, dtype=torch.float16)
    elif case == "duplicate":
        files["b.safetensors"] = {f"{p}.suh": t[f"{p}.suh"].clone()}
    elif case == "index_conflict":
        index = {name: "b.safetensors" for name in t}
    write(tmp_path, files, index)
    with pytest.raises(ValueError, match=message):
        C.Exl3Manifest(tmp_path)


def test_header_extent_checks(tmp_path):
    rng = np.random.default_rng(2)
    write(tmp_path, {"a.safetensors": matrix_tensors(rng, "x.proj", 128, 128, 4, 2)})
    raw = (tmp_path / "a.safetensors").read_bytes()
    (n,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + n])
    name = "x.proj.svh"
    header[name]["data_offsets"][1] += 2  # claims more bytes than its shape
    body = json.dumps(header).encode()
    (tmp_path / "a.safetensors").write_bytes(struct.pack("<Q", len(body)) + body + raw[8 + n:])
    with pytest.raises(ValueError, match="spans bytes|overlaps|gap"):
        C.read_headers(tmp_path / "a.safetensors")
    (tmp_path / "a.safetensors").write_bytes(raw + b"\0\0\0\0")
    with pytest.raises(ValueError, match="belong to no tensor"):
        C.read_headers(tmp_path / "a.safetensors")
    with pytest.raises(ValueError, match="no \\*.safetensors files"):
        C.Exl3Manifest(tmp_path / "nothing")


def test_hybrid_selection_by_index(tmp_path):
    rng = np.random.default_rng(3)
    t = matrix_tensors(rng, "m.proj", 128, 128, 4, 2)
    extra = {"skip.me": torch.zeros(4, dtype=torch.float32)}
    write(tmp_path, {"a.safetensors": t, "b.safetensors": extra},
          index={name: "a.safetensors" for name in t})
    m = C.Exl3Manifest(tmp_path, select_by_index=True)
    assert m.unselected == 1 and "skip.me" not in m.tensors
    assert "m.proj" in m.matrices
