"""EXL3 checkpoint ingestion end to end on the GPU: experts written to a
safetensors checkpoint, inventoried and loaded by
vllm_mi355x/kernels/exl3/checkpoint.py, turned into the packed_ptrs /
packed_meta tables (reference quant.py:1105-1134) and run through moe_out_v2
and exl3_linear_out against the oracle on the same arrays."""

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as O
from tests.checkpoint_cases import write
from tests.exl3_cases import random_acts, random_matrix
from tests.test_gpu_exl3_linear import _assert_fp32_close, _out_np
from tests.test_gpu_exl3_moe import GEMV_ABS_RMS, _acts, _assert_moe_close, _dev, _oracle_f32

pytestmark = pytest.mark.gpu


def _marker(codebook):
    from tests.checkpoint_cases import MCG, MUL1, marker
    return marker(MUL1 if codebook == 2 else MCG)


def test_checkpoint_experts_through_moe_v2(device, tmp_path):
    from vllm_mi355x.kernels.exl3 import checkpoint as C
    from vllm_mi355x.kernels.exl3 import ops
    ops.ensure_extension()
    print("checkpoint -> moe_out_v2, 4 experts 256/128 3-bit", flush=True)
    rng = np.random.default_rng(44)
    experts, hidden, inter, bits_x2, topk, rows = 4, 256, 128, 6, 2, 6
    host, tensors = [], {}
    for e in range(experts):
        projections = []
        for name, (k, n) in (("gate_proj", (hidden, inter)), ("up_proj", (hidden, inter)),
                             ("down_proj", (inter, hidden))):
            t, u, v = random_matrix(rng, k, n, bits_x2, scales="sign")
            prefix = f"model.layers.3.mlp.experts.{e}.{name}"
            tensors[f"{prefix}.trellis"] = torch.from_numpy(t.view(np.int16))
            tensors[f"{prefix}.suh"] = torch.from_numpy(u.view(np.float16))
            tensors[f"{prefix}.svh"] = torch.from_numpy(v.view(np.float16))
            tensors[f"{prefix}.mul1"] = _marker(2)
            projections.append((t, u, v, bits_x2, 2))
        host.append(projections)
    write(tmp_path, {"model.safetensors": tensors})
    manifest = C.Exl3Manifest(tmp_path)
    loaded = [[C.load_matrix(manifest, f"model.layers.3.mlp.experts.{e}.{name}", k, n, device)
               for name, (k, n) in (("gate_proj", (hidden, inter)), ("up_proj", (hidden, inter)),
                                    ("down_proj", (inter, hidden)))] for e in range(experts)]
    ptrs, meta = C.expert_tables(loaded, device)
    assert meta[0].tolist() == [[hidden, inter, bits_x2, 2], [hidden, inter, bits_x2, 2],
                                [inter, hidden, bits_x2, 2]]
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    emap = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, "bf16", device)
    size = ops.moe_workspace_size(rows, hidden, inter, topk, experts)
    ws = torch.empty(size, dtype=torch.float32, device=device)
    out = torch.empty_like(x)
    ops.moe_out_v2(x, _dev(ids, device), _dev(weights, device), ptrs, meta, _dev(emap, device), inter,
                   bits_x2, out, ws)
    torch.cuda.synchronize()
    expected = O.moe_out(x_host, code, ids, weights, O.MoELayer(host), emap, inter, out_dtype=code)
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), "checkpoint experts", GEMV_ABS_RMS)


def test_checkpoint_linear(device, tmp_path):
    from vllm_mi355x.kernels.exl3 import checkpoint as C
    from vllm_mi355x.kernels.exl3 import ops
    ops.ensure_extension()
    rng = np.random.default_rng(45)
    k, n = 512, 384
    t, u, v = random_matrix(rng, k, n, 8, scales="test")
    p = "model.layers.0.self_attn.q_proj"
    write(tmp_path, {"m.safetensors": {f"{p}.trellis": torch.from_numpy(t.view(np.int16)),
                                       f"{p}.suh": torch.from_numpy(u.view(np.float16)),
                                       f"{p}.svh": torch.from_numpy(v.view(np.float16)),
                                       f"{p}.mcg": _marker(1)}})
    w = C.load_matrix(C.Exl3Manifest(tmp_path), p, k, n, device)
    x, code = random_acts(rng, 3, k, "bf16")
    xt = torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16)
    out = torch.empty(3, n, dtype=torch.float32, device=device)
    ws = torch.empty(ops.linear_workspace_size(3, k, n), dtype=torch.float32, device=device)
    ops.linear_out(xt, w.trellis, w.suh, w.svh, w.matrix.bits_x2, w.matrix.codebook, k, n, out, ws)
    torch.cuda.synchronize()
    want = O.linear_out(x, code, t, u, v, 8, 1, n, O.FP32)
    _assert_fp32_close(out.cpu().numpy(), want, "checkpoint linear")
