"""The device router with alignment (moe_route) against the router oracle
and the alignment oracle.

Logits: against the FP64 product of the bf16 inputs, within the FP32
summation bound (2^-20 sum |x| |w| per logit).  Selection and weights: the
oracle routes the device's own logits (weights within 1e-5 relative: FP32
scores and sums in another order); a row may differ only where its
chosen k-th and best unchosen keys are within 4 FP32 ulps (the device's
tanhf / expf against NumPy's).  Alignment: bit-exact against the alignment
oracle on the device's ids.  Padding rows route to -1."""

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as X
from oracle import marlin_oracle as M
from oracle import route_oracle as R

pytestmark = pytest.mark.gpu


def _bf16(rng, shape, scale=1.0):
    bits = X.f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))
    return bits, X.bf16_bits_to_f32(bits)


@pytest.mark.parametrize("M_,E,K,topk,bs,scoring", [
    (1, 288, 4096, 8, 8, "sigmoid"), (4, 288, 4096, 8, 8, "sigmoid"), (64, 288, 4096, 8, 16, "sigmoid"),
    (33, 128, 2048, 8, 8, "softmax"), (300, 64, 1024, 6, 32, "softmax"), (7, 257, 7168, 8, 8, "sigmoid"),
    (2048, 288, 4096, 8, 16, "sigmoid"), (8, 256, 1024, 8, 8, "sigmoid"), (100, 512, 1024, 8, 16, "sigmoid"),
    (5, 1024, 1024, 8, 16, "softmax"), (3, 40, 512, 4, 8, "softmax")])
def test_route_matches_oracle(device, M_, E, K, topk, bs, scoring):
    from vllm_mi355x.kernels.moe import route
    print(f"moe_route M={M_} E={E} K={K} topk={topk} bs={bs} {scoring}", flush=True)
    rng = np.random.default_rng(M_ * 7 + E)
    xb, xf = _bf16(rng, (M_, K))
    wb, wf = _bf16(rng, (E, K), 0.02)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    pad = np.zeros(M_, np.uint8)
    if M_ > 2:
        pad[[1, M_ - 1]] = 1
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    x = to(xb.view(np.int16)).view(torch.bfloat16)
    w = to(wb.view(np.int16)).view(torch.bfloat16)
    logits, tw, tid, sorted_ids, eids, ntpp = route.moe_route(
        x, w, to(bias) if scoring == "sigmoid" else None, topk=topk, block_size=bs, num_experts=E,
        routed_scaling_factor=2.5, is_padding=to(pad).bool(), scoring=scoring)
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    want = R.logits_fp64(xf, wf)
    bound = 2.0 ** -20 * (np.abs(xf).astype(np.float64) @ np.abs(wf).astype(np.float64).T) + 1e-30
    assert (np.abs(lg - want) <= bound).all(), "logits"
    ids, wts, gaps = R.route(lg, topk, sigmoid=scoring == "sigmoid", bias=bias, scale=2.5)
    got_ids = tid.cpu().numpy()
    got_w = tw.cpu().numpy()
    for m in range(M_):
        if pad[m]:
            assert (got_ids[m] == -1).all()
            continue
        if not np.array_equal(got_ids[m], ids[m]):
            assert gaps[m] <= 4 * np.spacing(np.float32(abs(lg[m]).max() + 2)), f"row {m}"
            continue
        assert np.allclose(got_w[m], wts[m], rtol=1e-5, atol=0), f"row {m} weights"
    es, eeids, entpp = M.align(got_ids, E, bs)
    assert int(ntpp.item()) == int(entpp[0])
    assert np.array_equal(sorted_ids.cpu().numpy(), es)
    assert np.array_equal(eids.cpu().numpy(), eeids)


def test_route_is_deterministic_and_takes_out(device):
    from vllm_mi355x.kernels.moe import route
    from vllm_mi355x.kernels.moe.align import align_sizes
    rng = np.random.default_rng(3)
    M_, E, K = 16, 288, 4096
    xb, _ = _bf16(rng, (M_, K))
    wb, _ = _bf16(rng, (E, K), 0.02)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    x = to(xb.view(np.int16)).view(torch.bfloat16)
    w = to(wb.view(np.int16)).view(torch.bfloat16)
    bias = to(np.zeros(E, np.float32))
    first = [t.clone() for t in route.moe_route(x, w, bias)]
    mnp, nblk = align_sizes(M_ * 8, E, 8)
    out = (torch.empty(M_, E, device=device), torch.empty(M_, 8, device=device),
           torch.empty(M_, 8, dtype=torch.int32, device=device),
           torch.empty(mnp, dtype=torch.int32, device=device),
           torch.empty(nblk, dtype=torch.int32, device=device),
           torch.empty(1, dtype=torch.int32, device=device))
    second = route.moe_route(x, w, bias, out=out)
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    assert second[0].data_ptr() == out[0].data_ptr()


def test_route_rows_independent_of_the_call(device):
    """Each row's logits, weights and ids depend on that row alone: the first
    64 rows of a 300-row call (router GEMV on 64 x 64 tiles) equal, bitwise,
    a call of those 64 rows (16 x 16 tiles; the selection runs one wavefront
    a row over as many workgroups as the rows need), and the alignment
    equals the alignment oracle on the ids."""
    from vllm_mi355x.kernels.moe import route
    rng = np.random.default_rng(11)
    M_, E, K, topk, bs = 300, 288, 4096, 8, 16
    xb, _ = _bf16(rng, (M_, K))
    wb, _ = _bf16(rng, (E, K), 0.02)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    x = to(xb.view(np.int16)).view(torch.bfloat16)
    w = to(wb.view(np.int16)).view(torch.bfloat16)
    lg_all, tw_all, tid_all, sorted_ids, eids, ntpp = route.moe_route(x, w, to(bias), topk=topk,
                                                                       block_size=bs, num_experts=E)
    lg_64, tw_64, tid_64, _, _, _ = route.moe_route(x[:64].contiguous(), w, to(bias), topk=topk,
                                                    block_size=bs, num_experts=E)
    torch.cuda.synchronize()
    assert torch.equal(lg_all[:64].view(torch.int32), lg_64.view(torch.int32))
    assert torch.equal(tid_all[:64], tid_64)
    assert torch.equal(tw_all[:64].view(torch.int32), tw_64.view(torch.int32))
    es, eeids, entpp = M.align(tid_all.cpu().numpy(), E, bs)
    assert int(ntpp.item()) == int(entpp[0])
    assert np.array_equal(sorted_ids.cpu().numpy(), es)
    assert np.array_equal(eids.cpu().numpy(), eeids)
