"""Marlin-format int4 fused MoE on the GPU, through the C-ABI (the Python
bindings of vllm_mi355x.kernels.marlin_moe / .moe and the _ampere_marlin_C
operators), against the CPU oracle (oracle/marlin_oracle.c).

Bars:
  * dequantized weights (the GEMM's own operand path): bit-exact;
  * alignment (sorted ids, expert per block, padded total): bit-exact;
  * moe_sum: bit-exact (the same FP32 additions in the same slot order);
  * the fused MoE: the oracle sums each output sequentially in FP32, the GPU
    on the matrix cores in another order; both round the same sums at the
    same points (w13 rows, SiLU, h, w2 rows, router product, final sum), so
    an intermediate next to a rounding boundary may round the other way:
    |err| <= ulp |ref| + 2^-8 rms(ref) and rms(err) <= 2^-9 rms(ref), ulp =
    2^-7 (BF16) or 2^-10 (FP16).  A wrong nibble, scale, row or slot is off
    by O(rms).
"""

import math

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as X
from oracle import marlin_oracle as M

pytestmark = pytest.mark.gpu

TORCH_DTYPE = {M.BF16: torch.bfloat16, M.FP16: torch.float16}


@pytest.fixture(scope="module")
def mm():
    from vllm_mi355x.kernels import marlin_moe, moe
    from vllm_mi355x.kernels.marlin_moe import extension
    extension.require_extension()
    return marlin_moe, moe


def to_f32(bits, dtype):
    return X.bf16_bits_to_f32(bits) if dtype == M.BF16 else bits.view(np.float16).astype(np.float32)


def from_f32(v, dtype):
    v = np.asarray(v, np.float32)
    return X.f32_to_bf16_bits(v) if dtype == M.BF16 else v.astype(np.float16).view(np.uint16)


def dev_act(bits, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(
        TORCH_DTYPE[dtype])


def host_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def random_words(rng, *shape):
    return rng.integers(-(2 ** 31), 2 ** 31, shape, dtype=np.int64).astype(np.int32)


def random_scales(rng, shape, dtype, sigma=0.02):
    return from_f32(np.abs(rng.normal(0.0, sigma, shape)).astype(np.float32), dtype)


class Layer:
    def __init__(self, rng, E, K, N, dtype, device):
        self.host = (random_words(rng, E, K // 16, 4 * N), random_scales(rng, (E, K // 128, 2 * N), dtype),
                     random_words(rng, E, N // 16, 2 * K), random_scales(rng, (E, N // 128, K), dtype))
        w13, s13, w2, s2 = self.host
        self.w1, self.w2 = dev(w13, device), dev(w2, device)
        self.s1, self.s2 = dev_act(s13, dtype, device), dev_act(s2, dtype, device)


def routing(rng, T, E, topk, skew=None):
    if skew is None:
        ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)])
    else:
        p = 1.0 / np.arange(1, E + 1) ** skew
        p /= p.sum()
        ids = np.stack([rng.choice(E, topk, replace=False, p=p) for _ in range(T)])
    return ids.astype(np.int32), rng.random((T, topk)).astype(np.float32)


def assert_close(actual_bits, expected_bits, dtype, name):
    a = to_f32(actual_bits, dtype).astype(np.float64)
    e = to_f32(expected_bits, dtype).astype(np.float64)
    rms = float(np.sqrt(np.mean(e ** 2)))
    err = np.abs(a - e)
    ulp = 2.0 ** (-7 if dtype == M.BF16 else -10)
    bound = ulp * np.abs(e) + 2.0 ** -8 * rms
    worst = int(np.argmax(err - bound))
    assert np.isfinite(a).all(), f"{name}: non-finite"
    assert (err <= bound).all(), f"{name}: err {err.flat[worst]:.3g} > {bound.flat[worst]:.3g} (rms {rms:.3g})"
    assert np.sqrt(np.mean(err ** 2)) <= 2.0 ** -9 * rms, f"{name}: rms error"


# ---- dequant, align, sum ------------------------------------------------------------

@pytest.mark.parametrize("dtype", [M.BF16, M.FP16])
@pytest.mark.parametrize("K,N", [(128, 64), (256, 320), (2048, 1536)])
def test_dequant_bit_exact(mm, device, dtype, K, N):
    print(f"dequant dtype={dtype} K={K} N={N}", flush=True)
    rng = np.random.default_rng(K + N + dtype)
    w = random_words(rng, K // 16, 2 * N)
    s = random_scales(rng, (K // 128, N), dtype, sigma=0.5)
    got = host_bits(mm[0].marlin_dequant(dev(w, device), dev_act(s, dtype, device)))
    assert np.array_equal(got, M.dequant(w, s, K, N, dtype))


@pytest.mark.parametrize("T,E,topk,bs", [(1, 8, 2, 8), (5, 16, 4, 16), (64, 128, 8, 8),
                                         (300, 128, 8, 64), (3, 288, 8, 48), (2000, 64, 6, 32),
                                         (0, 8, 2, 8), (1024, 128, 8, 64), (1025, 128, 8, 64),
                                         (256, 128, 8, 32), (1000, 64, 8, 16), (700, 400, 2, 8)])
def test_align_matches_oracle(mm, device, T, E, topk, bs):
    print(f"align T={T} E={E} topk={topk} bs={bs}", flush=True)
    rng = np.random.default_rng(T + E)
    ids = np.array([rng.permutation(E)[:topk] for _ in range(T)], np.int32).reshape(T, topk)
    s, eids, ntpp = mm[1].align(dev(ids, device), E, bs)
    es, eeids, entpp = M.align(ids, E, bs)
    assert int(ntpp.item()) == int(entpp[0])
    assert np.array_equal(s.cpu().numpy(), es)
    assert np.array_equal(eids.cpu().numpy(), eeids)


def test_align_expert_map_and_invalid_ids(mm, device):
    rng = np.random.default_rng(5)
    E = 8
    ids = rng.integers(-1, E + 1, (20, 3)).astype(np.int32)
    emap = np.array([-1, 0, 1, -1, 2, 3, -1, 4], np.int32)
    s, eids, ntpp = mm[1].align(dev(ids, device), E, 8, expert_map=dev(emap, device))
    es, eeids, entpp = M.align(ids, E, 8, expert_map=emap)
    assert int(ntpp.item()) == int(entpp[0])
    assert np.array_equal(s.cpu().numpy(), es) and np.array_equal(eids.cpu().numpy(), eeids)


@pytest.mark.parametrize("dtype", [M.BF16, M.FP16])
def test_moe_sum_bit_exact(mm, device, dtype):
    rng = np.random.default_rng(dtype)
    T, topk, H = 7, 8, 1000
    v = from_f32(rng.standard_normal((T, topk, H)), dtype)
    got = host_bits(mm[1].moe_sum(dev_act(v, dtype, device)))
    acc = np.zeros((T, H), np.float32)
    for k in range(topk):
        acc = (acc + to_f32(v[:, k], dtype)).astype(np.float32)
    assert np.array_equal(got, from_f32(acc, dtype))
    # slots outside [0, experts) add nothing
    ids = rng.integers(-1, 5, (T, topk)).astype(np.int32)
    got = host_bits(mm[1].moe_sum(dev_act(v, dtype, device), topk_ids=dev(ids, device),
                                  num_experts=4))
    acc = np.zeros((T, H), np.float32)
    for k in range(topk):
        keep = ((ids[:, k] >= 0) & (ids[:, k] < 4))[:, None]
        acc = np.where(keep, acc + to_f32(v[:, k], dtype), acc).astype(np.float32)
    assert np.array_equal(got, from_f32(acc, dtype))


# ---- fused MoE --------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,limit", [(M.BF16, 10.0), (M.FP16, None), (M.BF16, 0.02)])
@pytest.mark.parametrize("T,bs", [(1, None), (5, 8), (5, 16), (33, 32), (33, 48), (40, 64)])
def test_fused_matches_oracle(mm, device, dtype, limit, T, bs):
    print(f"fused dtype={dtype} limit={limit} T={T} bs={bs}", flush=True)
    rng = np.random.default_rng(T * 10 + dtype)
    E, K, N, topk = 8, 256, 128, 4
    layer = Layer(rng, E, K, N, dtype, device)
    ids, w = routing(rng, T, E, topk, skew=1.1)
    x = from_f32(rng.standard_normal((T, K)), dtype)
    out = mm[0].fused_marlin_moe(dev_act(x, dtype, device), layer.w1, layer.w2, layer.s1, layer.s2,
                                 dev(w, device), dev(ids, device), clamp_limit=limit,
                                 block_size=bs)
    torch.cuda.synchronize()
    expected = M.moe(x, dtype, ids, w, *layer.host,
                     limit=math.inf if limit is None else limit)
    assert_close(host_bits(out), expected, dtype, f"T={T} bs={bs}")


def test_fused_at_c4_shape(mm, device):
    """128 experts, hidden 2048, intermediate 768, top-8, fp16, 16 tokens."""
    print("fused C4 shape T=16", flush=True)
    rng = np.random.default_rng(4)
    E, K, N, topk, T = 128, 2048, 768, 8, 16
    layer = Layer(rng, E, K, N, M.FP16, device)
    ids, w = routing(rng, T, E, topk)
    x = from_f32(rng.standard_normal((T, K)), M.FP16)
    out = mm[0].fused_marlin_moe(dev_act(x, M.FP16, device), layer.w1, layer.w2, layer.s1,
                                 layer.s2, dev(w, device), dev(ids, device))
    torch.cuda.synchronize()
    expected = M.moe(x, M.FP16, ids, w, *layer.host)
    assert_close(host_bits(out), expected, M.FP16, "C4 T=16")


def test_fused_block_sizes_and_splits_agree(mm, device):
    """T=256 at the C4 expert count: every block size and K split gives the
    same outputs to the MoE bar (the per-token arithmetic differs only in the
    w13 summation order), and bit-identical ones where that order is the
    same: blocks of 48 and 64 tokens (one wavefront runs all of K)."""
    rng = np.random.default_rng(8)
    E, K, N, topk, T = 128, 512, 256, 8, 256
    layer = Layer(rng, E, K, N, M.BF16, device)
    ids, w = routing(rng, T, E, topk)
    x = dev_act(from_f32(rng.standard_normal((T, K)), M.BF16), M.BF16, device)
    args = (x, layer.w1, layer.w2, layer.s1, layer.s2, dev(w, device), dev(ids, device))
    runs = {(bs, ks): host_bits(mm[0].fused_marlin_moe(*args, block_size=bs, ksplit=ks))
            for bs, ks in ((64, 1), (48, 1), (8, 1), (16, 1), (32, 1), (16, 2), (64, 4))}
    base = runs[(64, 1)]
    for key, got in runs.items():
        assert_close(got, base, M.BF16, f"bs, ks = {key}")
    assert np.array_equal(runs[(48, 1)], base)


def test_fused_zero_weights_masked_slots_and_empty(mm, device):
    rng = np.random.default_rng(9)
    E, K, N, topk, T = 4, 128, 128, 2, 6
    layer = Layer(rng, E, K, N, M.BF16, device)
    x = dev_act(from_f32(rng.standard_normal((T, K)), M.BF16), M.BF16, device)
    w = torch.ones(T, topk, device=device)
    # every slot routed nowhere (id -1 or >= E): exact zeros
    ids = torch.tensor([[-1, E]] * T, dtype=torch.int32, device=device)
    out = mm[0].fused_marlin_moe(x, layer.w1, layer.w2, layer.s1, layer.s2, w, ids)
    assert torch.equal(out, torch.zeros_like(out))
    # q = 8 everywhere: zero weights, exact zeros
    zero = torch.full_like(layer.w1, np.uint32(0x88888888).view(np.int32).item())
    ids = torch.tensor([[0, 1]] * T, dtype=torch.int32, device=device)
    out = mm[0].fused_marlin_moe(x, zero, layer.w2, layer.s1, layer.s2, w, ids)
    assert torch.equal(out, torch.zeros_like(out))
    # no tokens
    out = mm[0].fused_marlin_moe(x[:0], layer.w1, layer.w2, layer.s1, layer.s2, w[:0], ids[:0])
    assert out.shape == (0, K)


def test_one_token_unrouted_writes_zeros(mm, device):
    """One token takes the identity-routed path, whose w2 launch also forms
    the top-k sum: a token none of whose slots is routed (ids outside the
    experts, or an expert map sending every chosen expert to -1) still gets
    its zero sum written, over whatever the output buffer held."""
    rng = np.random.default_rng(19)
    E, K, N, topk = 4, 256, 128, 3
    layer = Layer(rng, E, K, N, M.BF16, device)
    x = dev_act(from_f32(rng.standard_normal((1, K)), M.BF16), M.BF16, device)
    w = torch.ones(1, topk, device=device)
    nan = torch.full((1, K), float("nan"), dtype=x.dtype, device=device)
    ids = torch.tensor([[-1, E, E + 3]], dtype=torch.int32, device=device)
    out = mm[0].fused_marlin_moe(x, layer.w1, layer.w2, layer.s1, layer.s2, w, ids,
                                 output=nan.clone())
    assert torch.equal(out, torch.zeros_like(out))
    emap = torch.tensor([-1, -1, 0, 1, 2, 3, -1], dtype=torch.int32, device=device)
    ids = torch.tensor([[0, 1, 6]], dtype=torch.int32, device=device)
    out = mm[0].fused_marlin_moe(x, layer.w1, layer.w2, layer.s1, layer.s2, w, ids,
                                 expert_map=emap, output=nan.clone())
    assert torch.equal(out, torch.zeros_like(out))
    # one slot routed: the sum is that slot's row alone, and equals the
    # staged path's
    ids = torch.tensor([[-1, 2, E]], dtype=torch.int32, device=device)
    out = mm[0].fused_marlin_moe(x, layer.w1, layer.w2, layer.s1, layer.s2, w, ids,
                                 output=nan.clone())
    ref = mm[0].fused_marlin_moe(x, layer.w1, layer.w2, layer.s1, layer.s2, w, ids,
                                 path="staged")
    assert torch.equal(out, ref)


def test_fused_expert_map(mm, device):
    rng = np.random.default_rng(10)
    E_local, E_global, K, N, topk, T = 3, 6, 128, 128, 3, 9
    layer = Layer(rng, E_local, K, N, M.BF16, device)
    emap = np.array([-1, 0, -1, 1, 2, -1], np.int32)
    ids = rng.integers(0, E_global, (T, topk)).astype(np.int32)
    w = rng.random((T, topk)).astype(np.float32)
    x = from_f32(rng.standard_normal((T, K)), M.BF16)
    out = mm[0].fused_marlin_moe(dev_act(x, M.BF16, device), layer.w1, layer.w2, layer.s1,
                                 layer.s2, dev(w, device), dev(ids, device),
                                 expert_map=dev(emap, device))
    local = np.where(emap[ids] >= 0, emap[ids], -1).astype(np.int32)
    expected = M.moe(x, M.BF16, local, w, *layer.host)
    assert_close(host_bits(out), expected, M.BF16, "expert map")


# ---- the direct path (k-permuted activations, LDS weight ring, fused SwiGLU) ----------------

def permuted_k(k):
    w = k & 31
    return (k & ~31) + 8 * ((w >> 1) & 3) + 2 * (w >> 3) + (w & 1)


def test_permute_act_layout(mm, device):
    from vllm_mi355x.kernels.marlin_moe import _C
    rng = np.random.default_rng(21)
    x = torch.from_numpy(rng.integers(-2 ** 15, 2 ** 15, (7, 96), dtype=np.int64).astype(np.int16))
    x = x.to(device).view(torch.bfloat16)
    out = torch.zeros_like(x)
    _C.permute_act(x, out)
    torch.cuda.synchronize()
    perm = np.array([permuted_k(k) for k in range(96)])
    assert sorted(perm.tolist()) == list(range(96))
    want = np.zeros((7, 96), np.int16)
    want[:, perm] = x.view(torch.int16).cpu().numpy()
    assert np.array_equal(out.view(torch.int16).cpu().numpy(), want)


@pytest.mark.parametrize("T,E,topk,bs,K", [(1, 8, 2, 8, 32), (37, 16, 4, 16, 96), (300, 128, 8, 32, 2048)])
def test_align_permute_matches_separate_calls(mm, device, T, E, topk, bs, K):
    # one launch (alignment workgroup + permutation workgroups) == the two calls
    from vllm_mi355x.kernels.marlin_moe import _C
    import importlib
    A = importlib.import_module("vllm_mi355x.kernels.moe.align")  # the module, not its align()
    print(f"align_permute T={T} E={E} topk={topk} bs={bs} K={K}", flush=True)
    rng = np.random.default_rng(T + E)
    ids = torch.from_numpy(rng.integers(-1, E + 1, (T, topk), dtype=np.int64).astype(np.int32)).to(device)
    x = torch.from_numpy(rng.integers(-2 ** 15, 2 ** 15, (T, K), dtype=np.int64).astype(np.int16))
    x = x.to(device).view(torch.float16)
    size, blocks = A.align_sizes(ids.numel(), E, bs)
    got = [torch.full((size,), -7, dtype=torch.int32, device=device),
           torch.full((blocks,), -7, dtype=torch.int32, device=device),
           torch.zeros(1, dtype=torch.int32, device=device)]
    want = [t.clone() for t in got]
    xp_got = torch.zeros_like(x)
    xp_want = torch.zeros_like(x)
    _C.align_permute(ids, E, bs, *got, x, xp_got)
    A.kernel_moe_align_block_size(ids, E, bs, *want, None, None)
    _C.permute_act(x, xp_want)
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        assert torch.equal(g, w)
    assert torch.equal(xp_got.view(torch.int16), xp_want.view(torch.int16))


@pytest.mark.parametrize("dtype,limit", [(M.BF16, 10.0), (M.FP16, None), (M.BF16, 0.02)])
@pytest.mark.parametrize("T,bs", [(1, 8), (5, 16), (33, 32), (40, 8)])
def test_direct_path_matches_oracle(mm, device, dtype, limit, T, bs):
    print(f"direct dtype={dtype} limit={limit} T={T} bs={bs}", flush=True)
    rng = np.random.default_rng(T * 13 + dtype)
    E, K, N, topk = 8, 256, 128, 4
    layer = Layer(rng, E, K, N, dtype, device)
    ids, w = routing(rng, T, E, topk, skew=1.1)
    x = from_f32(rng.standard_normal((T, K)), dtype)
    out = mm[0].fused_marlin_moe(dev_act(x, dtype, device), layer.w1, layer.w2, layer.s1, layer.s2,
                                 dev(w, device), dev(ids, device), clamp_limit=limit,
                                 block_size=bs, path="direct")
    torch.cuda.synchronize()
    expected = M.moe(x, dtype, ids, w, *layer.host, limit=math.inf if limit is None else limit)
    assert_close(host_bits(out), expected, dtype, f"direct T={T} bs={bs}")


@pytest.mark.parametrize("dtype,bs", [(M.FP16, 32), (M.BF16, 16)])
def test_direct_and_staged_paths_bitwise_at_c4_shape(mm, device, dtype, bs):
    """128 experts, hidden 2048, intermediate 768, top-8, 256 tokens: the
    staged path runs four tiles per workgroup here, the same per-tile MFMA
    sequence as the direct path, so the fused outputs are equal bit for bit
    (the direct path's fused SwiGLU does marlin_moe_act's arithmetic); and
    the direct STORE / PARTIAL modes equal the staged ones."""
    from vllm_mi355x.kernels.marlin_moe import _C
    print(f"direct vs staged dtype={dtype} bs={bs}", flush=True)
    rng = np.random.default_rng(22 + bs)
    E, K, N, topk, T = 128, 2048, 768, 8, 256
    layer = Layer(rng, E, K, N, dtype, device)
    ids, w = routing(rng, T, E, topk)
    x = dev_act(from_f32(rng.standard_normal((T, K)), dtype), dtype, device)
    args = (x, layer.w1, layer.w2, layer.s1, layer.s2, dev(w, device), dev(ids, device))
    staged = mm[0].fused_marlin_moe(*args, block_size=bs, ksplit=1, path="staged", clamp_limit=7.0)
    direct = mm[0].fused_marlin_moe(*args, block_size=bs, path="direct", clamp_limit=7.0)
    torch.cuda.synchronize()
    assert torch.equal(staged.view(torch.int16), direct.view(torch.int16))
    # single GEMMs: w2 shape, STORE and PARTIAL
    slots = T * topk
    sorted_ids, expert_ids, ntpp = mm[1].align(dev(ids, device), E, bs)
    h = dev_act(from_f32(rng.standard_normal((slots, N)), dtype), dtype, device)
    hp = torch.empty_like(h)
    _C.permute_act(h, hp)
    o1 = torch.zeros(slots, K, dtype=h.dtype, device=device)
    o2 = torch.zeros_like(o1)
    _C.gemm(h, layer.w2, layer.s2, sorted_ids, expert_ids, ntpp, None, 1, slots, N, K, bs,
            _C.MODE_STORE, 1, out=o1)
    _C.gemm_direct(hp, layer.w2, layer.s2, sorted_ids, expert_ids, ntpp, None, 1, slots, N, K, bs,
                   _C.MODE_STORE, 1, out=o2)
    p1 = torch.zeros(slots * K, dtype=torch.float32, device=device)
    p2 = torch.zeros_like(p1)
    _C.gemm(h, layer.w2, layer.s2, sorted_ids, expert_ids, ntpp, None, 1, slots, N, K, bs,
            _C.MODE_PARTIAL, 1, part=p1)
    _C.gemm_direct(hp, layer.w2, layer.s2, sorted_ids, expert_ids, ntpp, None, 1, slots, N, K, bs,
                   _C.MODE_PARTIAL, 1, part=p2)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(p1, p2)


@pytest.mark.parametrize("dtype", [M.BF16, M.FP16])
def test_w13_act_bitwise_equals_partial_then_act(mm, device, dtype):
    """marlin_moe_w13_act (the w13 K-split GEMM whose SwiGLU is finished by
    the last wavefront of each (block, 64 gate columns) to arrive) equals
    marlin_moe_gemm(PARTIAL) then marlin_moe_act bit for bit: identity
    routing at one token (one slot routed to no local expert) and aligned
    blocks, K splits 1..8, one- and four-tile workgroups, calls of
    different sizes back to back (every call returns its arrival counters to
    zero), and four replays of a captured graph with eager work between."""
    from vllm_mi355x.kernels.marlin_moe import _C
    rng = np.random.default_rng(31 + dtype)
    E, K, N, topk = 128, 2048, 768, 8
    layer = Layer(rng, E, K, N, dtype, device)

    def case(T, bs, ks, limit):
        ids, _ = routing(rng, T, E, topk)
        if bs is None:
            ids[0, 3] = -1
        x = dev_act(from_f32(rng.standard_normal((T, K)), dtype), dtype, device)
        slots = T * topk
        ids_d = dev(ids, device).view(-1)
        if bs is None:
            routed = (None, ids_d, None, 16)
        else:
            routed = (*mm[1].align(dev(ids, device), E, bs), bs)
        sorted_ids, eids, ntpp, bsz = routed
        part1 = torch.zeros(ks * slots * 2 * N, dtype=torch.float32, device=device)
        part2 = torch.zeros_like(part1)
        h1 = torch.zeros(slots, N, dtype=TORCH_DTYPE[dtype], device=device)
        h2 = torch.zeros_like(h1)
        _C.gemm(x, layer.w1, layer.s1, sorted_ids, eids, ntpp, None, topk, slots, K, 2 * N, bsz,
                _C.MODE_PARTIAL, ks, part=part1)
        _C.act(part1, ids_d, ks, slots, N, limit, h1)

        def fused():
            _C.w13_act(x, layer.w1, layer.s1, sorted_ids, eids, ntpp, ids_d, topk, slots, K, 2 * N,
                       bsz, ks, limit, part2, h2)
        return h1, h2, fused

    cases = ((1, None, 4, math.inf), (1, None, 8, 7.0), (5, 16, 2, math.inf), (40, 8, 1, 0.5),
             (40, 32, 4, 7.0), (256, 16, 1, math.inf), (3, 8, 16, 7.0))
    for T, bs, ks, limit in cases:
        print(f"w13_act dtype={dtype} T={T} bs={bs} ks={ks} limit={limit}", flush=True)
        h1, h2, fused = case(T, bs, ks, limit)
        fused()
        torch.cuda.synchronize()
        assert torch.equal(h1.view(torch.int16), h2.view(torch.int16)), (T, bs, ks)
    print(f"w13_act graph dtype={dtype}", flush=True)
    h1, h2, fused = case(1, None, 4, 7.0)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fused()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused()
    for _ in range(4):
        h2.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(h1.view(torch.int16), h2.view(torch.int16))


@pytest.mark.parametrize("dtype", [M.BF16, M.FP16])
def test_w2_sum_bitwise_equals_topk_then_sum(mm, device, dtype):
    """marlin_moe_w2_sum (identity routing: the w2 slot rows, and the sum of
    a token's routed slots finished by the last of their wavefronts to
    arrive) equals marlin_moe_gemm(TOPK) then moe_sum bit for bit: one token
    of 8 slots (one routed to no local expert), three tokens of 4, one of 2,
    sizes back to back (every call returns its arrival counters to zero),
    and four replays of a captured graph with eager work between."""
    from vllm_mi355x.kernels.marlin_moe import _C
    rng = np.random.default_rng(47 + dtype)
    E, K, N = 128, 768, 2048  # w2: intermediate 768 in, hidden 2048 out

    w2 = dev(random_words(rng, E, K // 16, 2 * N), device)
    s2 = dev_act(random_scales(rng, (E, K // 128, N), dtype), dtype, device)

    def case(T, topk, drop):
        ids, tw = routing(rng, T, E, topk)
        if drop:
            ids[0, 1] = -1
        slots = T * topk
        ids_d, tw_d = dev(ids, device).view(-1), dev(tw, device).view(-1)
        h = dev_act(from_f32(rng.standard_normal((slots, K)), dtype), dtype, device)
        c3a = torch.zeros(slots, N, dtype=TORCH_DTYPE[dtype], device=device)
        c3b, outa = torch.zeros_like(c3a), torch.zeros(T, N, dtype=TORCH_DTYPE[dtype], device=device)
        outb = torch.zeros_like(outa)
        _C.gemm(h, w2, s2, None, ids_d, None, tw_d, 1, slots, K, N, 16, _C.MODE_TOPK, 1, out=c3a)
        mm[1].moe_sum(c3a.view(T, topk, N), outa, ids_d.view(T, topk), E)

        def fused():
            _C.w2_sum(h, w2, s2, ids_d, tw_d, topk, slots, K, N, 16, c3b, outb)
        return (c3a, outa), (c3b, outb), fused

    for T, topk, drop in ((1, 8, True), (3, 4, False), (1, 2, False), (1, 8, False)):
        print(f"w2_sum dtype={dtype} T={T} topk={topk} drop={drop}", flush=True)
        a, b, fused = case(T, topk, drop)
        fused()
        torch.cuda.synchronize()
        for x, y in zip(a, b):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16)), (T, topk)
    print(f"w2_sum graph dtype={dtype}", flush=True)
    a, b, fused = case(1, 8, True)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fused()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused()
    for _ in range(4):
        b[1].zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a[1].view(torch.int16), b[1].view(torch.int16))


# ---- the reference's operator sequence ----------------------------------------------------

def test_decode_ops_sequence_matches_fused(mm, device):
    """decode.run's sequence (decode.py:301-339) through torch.ops.
    _ampere_marlin_C: align (block 8) -> decode_gemm_orig (w13, rows 64) ->
    decode_act_orig -> decode_gemm_orig (w2) -> moe_sum.  Equal, bit for bit,
    to fused_marlin_moe with the same block size and K split."""
    ops = torch.ops._ampere_marlin_C
    rng = np.random.default_rng(11)
    E, K, N, topk, T = 16, 2048, 512, 8, 4
    layer = Layer(rng, E, K, N, M.BF16, device)
    ids, w = routing(rng, T, E, topk)
    x = dev_act(from_f32(rng.standard_normal((T, K)), M.BF16), M.BF16, device)
    ids_d, w_d = dev(ids, device), dev(w, device)
    slots = T * topk
    sorted_ids, expert_ids, ntpp = mm[1].align(ids_d, E, 8)
    part = torch.zeros(4 * slots * 2 * N, dtype=torch.float32, device=device)
    h = torch.zeros(slots * N, dtype=torch.bfloat16, device=device)
    c3 = torch.zeros(slots * K, dtype=torch.bfloat16, device=device)
    ctr = torch.zeros(2, dtype=torch.int32, device=device)
    ksplit = ops.decode_gemm_orig(x, layer.w1, layer.s1, sorted_ids, expert_ids, ntpp,
                                  w_d.view(-1), topk, slots, K, 2 * N, True, 64, 0, ctr, part)
    assert ksplit == K // 16 // 64
    ops.decode_act_orig(part, ids_d.view(-1), ksplit, slots, N, 10.0, h)
    ops.decode_gemm_orig(h.view(slots, N), layer.w2, layer.s2, sorted_ids, expert_ids, ntpp,
                         w_d.view(-1), topk, slots, N, K, False, N // 16, 0, ctr, c3)
    out = mm[1].moe_sum(c3.view(T, topk, K))
    assert torch.equal(ctr, torch.zeros_like(ctr))
    fused = mm[0].fused_marlin_moe(x, layer.w1, layer.w2, layer.s1, layer.s2, w_d, ids_d,
                                   clamp_limit=10.0, block_size=8, ksplit=ksplit)
    assert torch.equal(out.view(torch.int16), fused.view(torch.int16))


def test_prefill_tile_gemm_matches_oracle_rows(mm, device):
    """prefill.run's list GEMMs (prefill.py:430-446): w13 without, w2 with
    the router weight, through prefill_tile_gemm; rows checked against the
    oracle's intermediate rows."""
    ops = torch.ops._ampere_marlin_C
    rng = np.random.default_rng(12)
    E, K, N, topk, T, bs = 8, 256, 128, 4, 48, 64
    layer = Layer(rng, E, K, N, M.BF16, device)
    ids, w = routing(rng, T, E, topk, skew=1.1)
    xb = from_f32(rng.standard_normal((T, K)), M.BF16)
    x = dev_act(xb, M.BF16, device)
    sorted_ids, expert_ids, ntpp = mm[1].align(dev(ids, device), E, bs)
    slots = T * topk
    none = None
    c1 = ops.prefill_tile_gemm(x, none, layer.w1, none, layer.s1, none, none, none,
                               torch.zeros(8, dtype=torch.int32, device=device), sorted_ids,
                               expert_ids, ntpp, dev(w, device), bs, topk, False, 0, T, 2 * N, K,
                               False, True, False, -1, -1, -1,
                               torch.empty(1, device=device), none)
    _, h1, h = M.moe(xb, M.BF16, ids, w, *layer.host, limit=10.0, want_intermediate=True)
    assert_close(host_bits(c1), h1, M.BF16, "w13 rows")
    hd = dev_act(h, M.BF16, device)
    c3 = ops.prefill_tile_gemm(hd, none, layer.w2, none, layer.s2, none, none, none,
                               torch.zeros(8, dtype=torch.int32, device=device), sorted_ids,
                               expert_ids, ntpp, dev(w, device), bs, 1, True, 0, slots, K, N,
                               False, True, False, -1, -1, -1, torch.empty(1, device=device), none)
    # expected w2 rows from the oracle's h: RN(RN(h @ W2) * RN(w))
    w2f = [to_f32(M.dequant(layer.host[2][e], layer.host[3][e], N, K, M.BF16), M.BF16)
           for e in range(E)]
    hf = to_f32(h, M.BF16).astype(np.float64)
    rows = np.empty((slots, K), np.uint16)
    for sl in range(slots):
        y = from_f32((hf[sl] @ w2f[ids.flat[sl]]).astype(np.float32), M.BF16)
        rw = to_f32(from_f32(np.float32(w.flat[sl]), M.BF16), M.BF16)
        rows[sl] = from_f32(to_f32(y, M.BF16) * rw, M.BF16)
    assert_close(host_bits(c3), rows, M.BF16, "w2 rows")
