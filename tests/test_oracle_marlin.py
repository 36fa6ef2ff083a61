"""Pins the CPU Marlin int4 MoE oracle (oracle/marlin_oracle.c) on the CPU.

What pins what:
  * the packed layout, restated independently from two sources the reference
    itself relies on: the PTX ISA's register table of the mma.m16n8k16 A
    fragment (rows = output columns n, columns = k) and the reference decode
    kernel's use of each nibble (decode_orig.cu:56-62, :238-249: deq2 takes
    bits [0,4) and [16,20); the four A registers are deq2(q), deq2(q >> 8),
    deq2(q >> 4), deq2(q >> 12)) with its tile addressing (:142-146, :196-198);
  * the scale permutation, restated from the decode kernel's scale reads
    (:165-167, :242-243: lane g reads stored positions 8g..8g+7 of a 64-column
    chunk, pair j = columns (16j + g, 16j + g + 8));
  * pack / unpack round trips; all-0x88888888 words (q = 8) dequantize to
    zero, so the MoE output is exactly zero;
  * the dequant against NumPy's own float16 rounding and a BF16 rounding of
    the exact product;
  * the fused MoE against an FP64 restatement of the reference test's
    reference_fp64 (test_ampere_pp_marlin_prefill.py:353-370), with the
    oracle's rounded weights (structure: routing, rounding points, slot
    order) and with unrounded weights (the reference test's own bar);
  * the alignment against a NumPy restatement of moe_align_reference.py's
    rank-by-ascending-index rule and the invariants of its output.
"""

import numpy as np
import pytest

from oracle import exl3_oracle as X
from oracle import marlin_oracle as M

# ---- independent restatements ------------------------------------------------

# PTX m16n8k16 .f16/.bf16 A fragment: register element a_i of lane
# (groupID g = lane / 4, threadID_in_group c = lane % 4) -> (row, col).
_A_FRAGMENT = [(0, 0), (0, 1), (8, 0), (8, 1), (0, 8), (0, 9), (8, 8), (8, 9)]
# nibble at bit 4i feeds A element: deq2(q) -> a0 (bit 0), a1 (bit 16);
# deq2(q >> 8) -> a2 (bit 8), a3 (bit 24); deq2(q >> 4) -> a4 (bit 4),
# a5 (bit 20); deq2(q >> 12) -> a6 (bit 12), a7 (bit 28).
_NIBBLE_TO_A = {0: 0, 4: 1, 2: 2, 6: 3, 1: 4, 5: 5, 3: 6, 7: 7}


def spec_unpack(w: np.ndarray, K: int, N: int) -> np.ndarray:
    q = np.empty((K, N), np.uint8)
    words = w.astype(np.uint32).reshape(K // 16, N // 64, 32, 4)
    for lane in range(32):
        g, c = lane // 4, lane % 4
        for nib in range(8):
            dn, dk = _A_FRAGMENT[_NIBBLE_TO_A[nib]]
            vals = (words[:, :, lane, :] >> (4 * nib)) & 15  # [K/16, N/64, 4 (j)]
            for j in range(4):
                q[dk + 2 * c::16, 0:N][:, (np.arange(N // 64) * 64 + 16 * j + g + dn)] = vals[:, :, j]
    return q


def spec_scale_positions(N: int) -> np.ndarray:
    pos = np.empty(N, np.int64)
    for chunk in range(N // 64):
        for g in range(8):
            for j in range(4):
                pos[64 * chunk + 16 * j + g] = 64 * chunk + 8 * g + 2 * j
                pos[64 * chunk + 16 * j + g + 8] = 64 * chunk + 8 * g + 2 * j + 1
    return pos


def to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    return X.bf16_bits_to_f32(bits) if dtype == M.BF16 else bits.view(np.float16).astype(np.float32)


def from_f32(v: np.ndarray, dtype: int) -> np.ndarray:
    v = np.asarray(v, np.float32)
    return X.f32_to_bf16_bits(v) if dtype == M.BF16 else v.astype(np.float16).view(np.uint16)


def rnd(v, dtype):
    return to_f32(from_f32(v, dtype), dtype).astype(np.float64)


def random_words(rng, *shape):
    return rng.integers(-(2 ** 31), 2 ** 31, shape, dtype=np.int64).astype(np.int32)


def random_scales(rng, shape, dtype, sigma=0.02):
    return from_f32(np.abs(rng.normal(0.0, sigma, shape)).astype(np.float32), dtype)


def make_layer(rng, E, K, N, dtype):
    """Random experts: uniform nibbles, |N(0, 0.02)| group scales."""
    return (random_words(rng, E, K // 16, 4 * N), random_scales(rng, (E, K // 128, 2 * N), dtype),
            random_words(rng, E, N // 16, 2 * K), random_scales(rng, (E, N // 128, K), dtype))


# ---- layout --------------------------------------------------------------------

@pytest.mark.parametrize("K,N", [(16, 64), (128, 192), (256, 512)])
def test_unpack_matches_fragment_spec(K, N):
    rng = np.random.default_rng(K + N)
    w = random_words(rng, K // 16, 2 * N)
    assert np.array_equal(M.unpack(w, K, N), spec_unpack(w, K, N))
    assert np.array_equal(M.pack(M.unpack(w, K, N)), w)


def test_single_nibble_positions():
    # one set nibble per word position lands on one (k, n)
    K, N = 16, 64
    for lane in (0, 5, 31):
        for j in range(4):
            for nib in range(8):
                w = np.zeros((1, 2 * N), np.int32)
                w[0, lane * 4 + j] = np.int32(np.uint32(9 << (4 * nib)).view(np.int32))
                q = M.unpack(w, K, N)
                k, n = np.argwhere(q == 9)[0]
                dn, dk = _A_FRAGMENT[_NIBBLE_TO_A[nib]]
                assert (k, n) == (2 * (lane % 4) + dk, 16 * j + lane // 4 + dn)
                assert np.count_nonzero(q) == 1


def test_scale_positions_match_kernel_reads():
    assert np.array_equal(M.scale_positions(256), spec_scale_positions(256))
    assert sorted(M.scale_positions(256).tolist()) == list(range(256))


@pytest.mark.parametrize("dtype", [M.BF16, M.FP16])
def test_dequant_rounds_the_exact_product_once(dtype):
    rng = np.random.default_rng(dtype)
    K, N = 256, 128
    w = random_words(rng, K // 16, 2 * N)
    s = random_scales(rng, (K // 128, N), dtype, sigma=0.7)
    q = spec_unpack(w, K, N).astype(np.float64)
    logical = to_f32(s, dtype)[:, M.scale_positions(N)].astype(np.float64)
    exact = (q - 8.0) * np.repeat(logical, 128, axis=0)
    expected = from_f32(exact.astype(np.float32), dtype)  # exact in float32, one rounding
    assert np.array_equal(M.dequant(w, s, K, N, dtype), expected)


def test_all_eights_dequantize_to_zero():
    rng = np.random.default_rng(0)
    K, N = 256, 128
    w = np.full((K // 16, 2 * N), np.uint32(0x88888888).view(np.int32), np.int32)
    s = random_scales(rng, (K // 128, N), M.BF16)
    assert not to_f32(M.dequant(w, s, K, N, M.BF16), M.BF16).any()


# ---- fused MoE -------------------------------------------------------------------

def spec_moe(x, dtype, ids, weights, layer, limit, rounded_weights):
    """FP64 over the dequantized weights with the bf16/fp16 rounding points
    of the reference test's reference_fp64; returns the FP64 sum before the
    final rounding."""
    w13, s13, w2, s2 = layer
    E, topk = w13.shape[0], ids.shape[1]
    Mtok, K = x.shape
    N = w2.shape[1] * 16
    xf = to_f32(x, dtype).astype(np.float64)
    acc = np.zeros((Mtok, K))
    for e in np.unique(ids):
        if not 0 <= e < E:
            continue
        if rounded_weights:
            d13 = to_f32(M.dequant(w13[e], s13[e], K, 2 * N, dtype), dtype).astype(np.float64)
            d2 = to_f32(M.dequant(w2[e], s2[e], N, K, dtype), dtype).astype(np.float64)
        else:
            def deq(w, s, k, n):
                q = M.unpack(w, k, n).astype(np.float64) - 8.0
                return q * np.repeat(to_f32(s, dtype)[:, M.scale_positions(n)], 128, axis=0)
            d13, d2 = deq(w13[e], s13[e], K, 2 * N), deq(w2[e], s2[e], N, K)
        r, slot = np.nonzero(ids == e)
        h1 = rnd(xf[r] @ d13, dtype)
        gate = np.minimum(h1[:, :N], limit)
        up = np.clip(h1[:, N:], -limit, limit)
        h = rnd(rnd(gate / (1.0 + np.exp(-gate)), dtype) * up, dtype)
        y = rnd(h @ d2, dtype)
        np.add.at(acc, r, rnd(y * rnd(weights[r, slot], dtype)[:, None], dtype))
    return acc


@pytest.mark.parametrize("dtype,limit", [(M.BF16, 10.0), (M.FP16, float("inf")), (M.BF16, 0.05)])
def test_moe_matches_fp64(dtype, limit):
    rng = np.random.default_rng(int(dtype) + 7)
    E, K, N, topk, T = 6, 256, 128, 3, 5
    layer = make_layer(rng, E, K, N, dtype)
    x = from_f32(rng.standard_normal((T, K)), dtype)
    ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int32)
    ids[0, 1] = -1  # a masked slot contributes nothing
    weights = rng.random((T, topk)).astype(np.float32)
    out = to_f32(M.moe(x, dtype, ids, weights, *layer, limit=limit), dtype).astype(np.float64)
    exact = spec_moe(x, dtype, ids, weights, layer, limit, rounded_weights=True)
    scale = float(np.sqrt(np.mean(exact ** 2)))
    assert scale > 0
    # same weights and rounding points, other summation order: one output
    # ulp, a few ulps of the intermediate rows' rounding flips
    err = np.abs(out - exact)
    ulp = 2.0 ** (-7 if dtype == M.BF16 else -10)
    assert (err <= ulp * np.abs(exact) + 2.0 ** -8 * scale).all()
    assert np.sqrt(np.mean(err ** 2)) <= 2.0 ** -9 * scale
    # the reference test's unrounded FP64 weights: the weight rounding alone
    # moves single outputs by a few percent (its own checks are error ratios
    # against the incumbent), so only the RMS is bounded here
    loose = spec_moe(x, dtype, ids, weights, layer, limit, rounded_weights=False)
    err = np.abs(out - loose)
    assert np.sqrt(np.mean(err ** 2)) <= 2.0 ** -6 * scale


def test_moe_zero_weights_give_exact_zero():
    rng = np.random.default_rng(1)
    E, K, N, topk, T = 3, 128, 128, 2, 3
    w13, s13, w2, s2 = make_layer(rng, E, K, N, M.BF16)
    w13[:] = np.uint32(0x88888888).view(np.int32)
    x = from_f32(rng.standard_normal((T, K)), M.BF16)
    ids = np.array([[0, 1], [2, 0], [1, 2]], np.int32)
    out = M.moe(x, M.BF16, ids, np.ones((T, topk), np.float32), w13, s13, w2, s2)
    assert not to_f32(out, M.BF16).any()


def test_moe_intermediates_follow_the_rounding_points():
    rng = np.random.default_rng(2)
    E, K, N, topk, T = 2, 128, 128, 2, 2
    layer = make_layer(rng, E, K, N, M.BF16)
    x = from_f32(rng.standard_normal((T, K)), M.BF16)
    ids = np.array([[0, 1], [1, 0]], np.int32)
    w = np.array([[0.25, 0.75], [0.5, 0.5]], np.float32)
    out, h1, h = M.moe(x, M.BF16, ids, w, *layer, limit=10.0, want_intermediate=True)
    g = to_f32(h1[:, :N], M.BF16)
    u = to_f32(h1[:, N:], M.BF16)
    gc = np.minimum(g, np.float32(10.0))
    uc = np.clip(u, np.float32(-10.0), np.float32(10.0))
    silu = rnd(gc / (np.float32(1.0) + np.exp(-gc)), M.BF16).astype(np.float32)
    expect = from_f32(silu * uc, M.BF16)
    # SiLU's exp may differ by an ulp from NumPy's: allow one bf16 ulp
    diff = np.abs(to_f32(h, M.BF16) - to_f32(expect, M.BF16))
    assert (diff <= 2.0 ** -7 * np.abs(to_f32(expect, M.BF16)) + 1e-30).all()


# ---- alignment -----------------------------------------------------------------------

def spec_align(ids, E, bs, expert_map=None):
    flat = ids.reshape(-1).astype(np.int64)
    numel = flat.size
    size, blocks = M.align_sizes(numel, E, bs)
    ok = (flat >= 0) & (flat < E)
    e = flat.copy()
    if expert_map is not None:
        e = np.where(ok, expert_map[np.where(ok, flat, 0)], -1)
        ok &= e >= 0
    counts = np.array([np.count_nonzero(ok & (e == x)) for x in range(E)])
    padded = (counts + bs - 1) // bs * bs
    excl = np.cumsum(padded) - padded
    sorted_ids = np.full(size, numel, np.int32)
    for x in range(E):
        rows = np.nonzero(ok & (e == x))[0]  # ascending flat index
        sorted_ids[excl[x]:excl[x] + rows.size] = rows
    ntpp = int(padded.sum())
    b = np.arange(blocks)
    owner = ((excl // bs)[None, :] <= b[:, None]).sum(1) - 1
    expert_ids = np.where(b < ntpp // bs, owner, -1).astype(np.int32)
    return sorted_ids, expert_ids, ntpp


@pytest.mark.parametrize("T,E,topk,bs", [(1, 8, 2, 8), (5, 16, 4, 16), (64, 128, 8, 8),
                                         (300, 128, 8, 64), (3, 288, 8, 48)])
def test_align_matches_spec(T, E, topk, bs):
    rng = np.random.default_rng(T * E)
    ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int32)
    s, eids, ntpp = M.align(ids, E, bs)
    es, eeids, entpp = spec_align(ids, E, bs)
    assert ntpp[0] == entpp and np.array_equal(s, es) and np.array_equal(eids, eeids)
    # invariants: every routed row once, blocks of one expert, padding = numel
    valid = s[s < ids.size]
    assert np.array_equal(np.sort(valid), np.arange(ids.size))
    for blk in range(ntpp[0] // bs):
        rows = s[blk * bs:(blk + 1) * bs]
        rows = rows[rows < ids.size]
        assert (ids.reshape(-1)[rows] == eids[blk]).all()
        assert np.all(np.diff(rows) > 0)


def test_align_with_expert_map_and_invalid_ids():
    rng = np.random.default_rng(5)
    E = 8
    ids = rng.integers(-1, E + 1, (20, 3)).astype(np.int32)
    emap = np.array([-1, 0, 1, -1, 2, 3, -1, 4], np.int32)
    s, eids, ntpp = M.align(ids, E, 8, expert_map=emap)
    es, eeids, entpp = spec_align(ids, E, 8, expert_map=emap)
    assert ntpp[0] == entpp and np.array_equal(s, es) and np.array_equal(eids, eeids)


def test_torch_cpu_path_matches_the_oracle_layout():
    """oracle/marlin_torch_ref.py (the bench's CPU baseline) dequantizes to
    the unrounded (q - 8) s of the pinned layout, and its MoE is the FP64
    restatement above with unrounded weights."""
    import torch
    from oracle import marlin_torch_ref as R
    rng = np.random.default_rng(21)
    E, K, N, topk, T = 3, 256, 128, 2, 4
    layer = make_layer(rng, E, K, N, M.BF16)
    w13, s13, w2, s2 = layer
    q = M.unpack(w13[1], K, 2 * N).astype(np.float64) - 8.0
    sc = to_f32(s13[1], M.BF16)[:, M.scale_positions(2 * N)].astype(np.float64)
    expect = q * np.repeat(sc, 128, axis=0)
    s13_t = torch.from_numpy(s13.view(np.int16)).view(torch.bfloat16)
    got = R.dequant_fp64(torch.from_numpy(w13[1]), s13_t[1], K, 2 * N).numpy()
    assert np.array_equal(got, expect)
    x = from_f32(rng.standard_normal((T, K)), M.BF16)
    ids = np.array([[0, 2], [1, 0], [2, 1], [0, 1]], np.int32)
    w = rng.random((T, topk)).astype(np.float32)
    s2_t = torch.from_numpy(s2.view(np.int16)).view(torch.bfloat16)
    x_t = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    got = R.moe_fp64(x_t, torch.from_numpy(ids), torch.from_numpy(w), torch.from_numpy(w13),
                     torch.from_numpy(w2), s13_t, s2_t, clamp=10.0).numpy()
    want = spec_moe(x, M.BF16, ids, w, layer, 10.0, rounded_weights=False)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
