"""The benchmark workloads at their full sizes on the GPU, checked against the
CPU oracle on sampled rows / tokens (rows and tokens are independent, so a
sample pins the path at the full grid) and by size-independent properties.

  * EXL3 prefill, 8192 x 28672, 4 bits, M = 2048 and 8192: sampled rows
    against the oracle (the many-row path's FP16-operand bar of
    test_gpu_exl3_linear: 2^-8 rms(ref) + 2^-10 |ref| max-abs, 2^-10
    rms(ref) rms).
  * EXL3 3-bit MoE, 256 routed + 1 shared experts, 7168 / 2048, top-8 from
    Zipf(1.1)-skewed logits, 2048 tokens: a token's output depends only on
    its own row and routes (bitwise under a token permutation; routed alone,
    where its experts take the small-M GEMV, to the MoE bar), two calls
    agree bitwise, and sampled tokens whose routes are set to three routed
    experts plus the shared one match the oracle (bar of
    test_gpu_exl3_moe).  Scales are the reference's test scales (suh ~
    N(0, 1), svh ~ 0.05 N(0, 1)): the +-1 x N(1, 0.05) scales of the
    benchmark description overflow FP16 in the down projection of random
    weights.
  * Marlin int4 MoE, 128 experts, 2048 / 768, top-8, T = 1, 64 and 256:
    sampled tokens against the oracle (bar of test_gpu_marlin_moe).
"""

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as O
from oracle import marlin_oracle as M
from tests.exl3_cases import random_acts, random_matrix
from tests.test_gpu_exl3_linear import _assert_fp32_close, _dev, _out_np, _run_linear
from tests.test_gpu_exl3_moe import _assert_moe_close, _oracle_f32, _run
from tests.test_gpu_marlin_moe import Layer as MarlinLayer
from tests.test_gpu_marlin_moe import assert_close, dev, dev_act, from_f32, host_bits, routing

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from vllm_mi355x.kernels.exl3 import ops as exl3_ops
    exl3_ops.ensure_extension()
    return exl3_ops


@pytest.fixture(scope="module")
def prefill_matrix():
    rng = np.random.default_rng(8192)
    return random_matrix(rng, 8192, 28672, 8)


@pytest.mark.parametrize("rows", [2048, 8192])
def test_prefill_full_shape_sampled_rows(ops, device, prefill_matrix, rows):
    print(f"prefill 8192x28672 4-bit M={rows}", flush=True)
    trellis, suh, svh = prefill_matrix
    rng = np.random.default_rng(rows)
    x, code = random_acts(rng, rows, 8192, "fp16")
    got = _out_np(_run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, 28672, torch.float32))
    assert np.isfinite(got).all()
    sample = [0, rows - 1]
    want = O.linear_out(x[sample], code, trellis, suh, svh, 8, 2, 28672, O.FP32)
    _assert_fp32_close(got[sample], want, f"prefill M={rows}")


# ---- EXL3 3-bit MoE layer at 2048 tokens --------------------------------------------

class _Full:
    """Expert tables of a layer generated on the device (257 x 3 matrices)."""


def _full_layer(device, experts, hidden, intermediate, bits_x2, seed):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    layer = _Full()
    layer.keep, ptrs, meta = [], [], []
    for _ in range(experts):
        p, m = [], []
        for kk, nn in ((hidden, intermediate), (hidden, intermediate), (intermediate, hidden)):
            t = torch.randint(-(2 ** 15), 2 ** 15, (kk // 16, nn // 16, 8 * bits_x2), dtype=torch.int16,
                              device=device, generator=gen)
            u = torch.randn(kk, device=device, generator=gen).half()
            v = (0.05 * torch.randn(nn, device=device, generator=gen)).half()
            layer.keep.append((t, u, v))
            p.append([t.data_ptr(), u.data_ptr(), v.data_ptr()])
            m.append([kk, nn, bits_x2, 2])
        ptrs.append(p)
        meta.append(m)
    layer.ptrs = torch.tensor(ptrs, dtype=torch.int64, device=device)
    layer.meta = torch.tensor(meta, dtype=torch.int64, device=device)
    return layer


def test_moe_full_layer_2048_tokens(ops, device):
    print("moe_v2 full layer 257 x 7168/2048 3-bit, 2048 tokens", flush=True)
    hidden, intermediate, routed, topk, rows, bits_x2 = 7168, 2048, 256, 8, 2048, 6
    layer = _full_layer(device, routed + 1, hidden, intermediate, bits_x2, 2048)
    gen = torch.Generator(device=device)
    gen.manual_seed(2049)
    ranks = torch.randperm(routed, generator=torch.Generator().manual_seed(2050)).float() + 1.0
    logits = torch.randn(rows, routed, generator=gen, device=device) + (-1.1 * torch.log(ranks)).to(device)
    tw, ti = torch.topk(torch.softmax(logits, -1), topk, dim=-1)
    tw = tw / tw.sum(-1, keepdim=True)
    ids = torch.cat([ti.int(), torch.full((rows, 1), routed, dtype=torch.int32, device=device)], 1)
    weights = torch.cat([tw.float(), torch.ones(rows, 1, device=device)], 1)
    # sampled tokens: three routed experts and the shared one (the other
    # slots masked), so the oracle needs four experts
    sampled = {5: (3, 17, 200), 1000: (3, 90, 255), 2047: (17, 42, 128)}
    for t, experts in sampled.items():
        ids[t] = torch.tensor(list(experts) + [-1] * (topk - 3) + [routed], dtype=torch.int32)
    ids, weights = ids.contiguous(), weights.contiguous()
    emap = torch.arange(routed + 1, dtype=torch.int32, device=device)
    x = torch.randn(rows, hidden, generator=gen, device=device).half()

    def call(xx, ii, ww):
        return _run(ops, xx, ii.contiguous(), ww.contiguous(), layer, emap, intermediate,
                    bits_x2=bits_x2, poison=False)

    out = call(x, ids, weights)
    assert torch.isfinite(out.float()).all() and out.float().abs().max() > 0
    assert torch.equal(out.view(torch.int16), call(x, ids, weights).view(torch.int16))
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(2051)).to(device)
    permuted = call(x[perm], ids[perm], weights[perm])
    assert torch.equal(permuted.view(torch.int16), out[perm].view(torch.int16))
    # routed alone, a token's experts run on the small-M GEMV (another FP32
    # summation order than the tile GEMM the full call uses): the MoE bar
    for r in (0, 1000):
        alone = call(x[r:r + 1], ids[r:r + 1], weights[r:r + 1])
        _assert_moe_close(_out_np(alone), _out_np(out[r:r + 1]).astype(np.float64), f"token {r}")

    # the oracle on the sampled tokens, with the four experts they use
    used = sorted({e for experts in sampled.values() for e in experts} | {routed})
    host = []
    for e in used:
        host.append([(t.cpu().numpy(), u.cpu().numpy(), v.cpu().numpy(), bits_x2, 2)
                     for t, u, v in layer.keep[3 * e:3 * e + 3]])
    oracle_layer = O.MoELayer(host)
    oracle_map = np.full(routed + 1, -1, np.int64)
    oracle_map[used] = np.arange(len(used))
    rows_s = sorted(sampled)
    x_host = x[rows_s].cpu().numpy()
    expected = O.moe_out(x_host, O.FP16, ids[rows_s].cpu().numpy().astype(np.int64),
                         weights[rows_s].cpu().numpy(), oracle_layer, oracle_map, intermediate,
                         out_dtype=O.FP16)
    _assert_moe_close(_out_np(out[rows_s]), _oracle_f32(expected, O.FP16), "2048-token layer")


# ---- moe_out_prefill's served configuration ---------------------------------------

@pytest.fixture(scope="module")
def prefill_moe_layer(device):
    return _full_layer(device, 256, 2560, 640, 10, 2560)


@pytest.mark.parametrize("rows", [65, 512, 3460])
def test_moe_prefill_served_config(ops, device, prefill_moe_layer, rows):
    """The one configuration the reference's moe_out_prefill serves: hidden
    2560, intermediate 640, every routed matrix bits_x2 10 mul1, 65 to 3460
    rows, 256 local experts, top-10 (csrc/exl3/moe_prefill.h:9-14,
    vllm_sm80/kernels/exl3/ops.py:75-80), through
    torch.ops._exl3_C.moe_out_prefill.  At 3460 rows most experts run on the
    tile GEMM, at 65 on the small-M GEMV.  Three sampled tokens (routed to
    three experts each, the other slots masked) against the oracle; the
    call is deterministic and each token's result does not depend on the
    other rows (a token routed alone runs on the GEMV: the MoE bar)."""
    print(f"moe_out_prefill 256 x 2560/640 bits_x2 10 top-10 rows={rows}", flush=True)
    hidden, intermediate, experts, topk = 2560, 640, 256, 10
    layer = prefill_moe_layer
    gen = torch.Generator(device=device)
    gen.manual_seed(rows)
    logits = torch.randn(rows, experts, generator=gen, device=device)
    tw, ti = torch.topk(torch.softmax(logits, -1), topk, dim=-1)
    tw = tw / tw.sum(-1, keepdim=True)
    ids, weights = ti.int(), tw.float()
    sampled = {0: (3, 17, 200), rows // 2: (5, 90, 255), rows - 1: (17, 42, 128)}
    for t, chosen in sampled.items():
        ids[t] = torch.tensor(list(chosen) + [-1] * (topk - 3), dtype=torch.int32)
    ids, weights = ids.contiguous(), weights.contiguous()
    emap = torch.arange(experts, dtype=torch.int32, device=device)
    x = torch.randn(rows, hidden, generator=gen, device=device).bfloat16()
    size = ops.moe_workspace_size(rows, hidden, intermediate, topk, experts)

    def call(xx, ii, ww):
        out = torch.full_like(xx, float("nan"))
        ws = torch.empty(size, dtype=torch.float32, device=device)
        torch.ops._exl3_C.moe_out_prefill(xx, ii, ww, layer.ptrs, layer.meta, emap, intermediate,
                                          out, ws)
        torch.cuda.synchronize()
        return out

    out = call(x, ids, weights)
    assert torch.isfinite(out.float()).all() and out.float().abs().max() > 0
    assert torch.equal(out.view(torch.int16), call(x, ids, weights).view(torch.int16))
    r = rows // 3
    alone = call(x[r:r + 1], ids[r:r + 1], weights[r:r + 1])
    _assert_moe_close(_out_np(alone), _out_np(out[r:r + 1]).astype(np.float64), f"token {r}")
    used = sorted({e for chosen in sampled.values() for e in chosen})
    host = []
    for e in used:
        host.append([(t.cpu().numpy(), u.cpu().numpy(), v.cpu().numpy(), 10, 2)
                     for t, u, v in layer.keep[3 * e:3 * e + 3]])
    oracle_map = np.full(experts, -1, np.int64)
    oracle_map[used] = np.arange(len(used))
    rows_s = sorted(sampled)
    xs = x[rows_s].view(torch.int16).cpu().numpy().view(np.uint16)
    expected = O.moe_out(xs, O.BF16, ids[rows_s].cpu().numpy().astype(np.int64),
                         weights[rows_s].cpu().numpy(), O.MoELayer(host), oracle_map, intermediate,
                         out_dtype=O.BF16)
    _assert_moe_close(_out_np(out[rows_s]), _oracle_f32(expected, O.BF16), f"rows={rows}")


# ---- Marlin int4 MoE at the full expert shape ---------------------------------------

@pytest.fixture(scope="module")
def marlin_layer(device):
    rng = np.random.default_rng(128)
    return MarlinLayer(rng, 128, 2048, 768, M.FP16, device)


@pytest.mark.parametrize("T", [1, 64, 256])
def test_marlin_full_shape_sampled_tokens(device, marlin_layer, T):
    from vllm_mi355x.kernels.marlin_moe import fused
    print(f"marlin 128x2048/768 top-8 T={T}", flush=True)
    rng = np.random.default_rng(1000 + T)
    ids, w = routing(rng, T, 128, 8)
    x = from_f32(rng.standard_normal((T, 2048)), M.FP16)
    out = fused.fused_marlin_moe(dev_act(x, M.FP16, device), marlin_layer.w1, marlin_layer.w2,
                                 marlin_layer.s1, marlin_layer.s2, dev(w, device), dev(ids, device))
    torch.cuda.synchronize()
    got = host_bits(out)
    sample = sorted({0, T // 2, T - 1})
    expected = M.moe(x[sample], M.FP16, ids[sample], w[sample], *marlin_layer.host)
    assert_close(got[sample], expected, M.FP16, f"C4 T={T}")
