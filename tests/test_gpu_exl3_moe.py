"""EXL3 routed-expert MoE on the GPU (moe_out / moe_out_v2 through the
_exl3_C operators and the C-ABI) against the CPU oracle's restatement of the
reference's moe_out_reference (csrc/exl3/reference.cu:371-448).

Bar: the oracle computes the reference's FP32 chain per assignment; the GPU
runs the expert GEMVs on the matrix cores with the activations split into
FP16 high/low parts and sums in another order, so the gate/up/down results
carry a few FP32 roundings of difference that then pass through SiLU, the
down projection and the routed sum.  Outputs (BF16 / FP16) must agree to
|err| <= 2^-7 |ref| + 2^-13 rms(ref) (2^-10 rms(ref) where a reaching
SwiGLU clamp exposes the absolute error of large gate sums), and
rms(err) <= 2^-10 rms(ref): one output ulp for values next to a rounding
boundary plus a small absolute term; a wrong decode, index, route or scale
is off by O(rms).  moe_out and moe_out_v2 run the same arithmetic
in the same order and must agree bitwise.

Cases follow the reference's tests: expert maps with masked, padding and
out-of-range ids (test_exl3_kernels.py:242-278), every mul1 rate of the
fixed-rate variant, the SwiGLU clamp at the DeepSeek routed-expert shape
(test_exl3_moe_swiglu_clamp.py:51-86), empty and fully masked routes, and
the operator's error checks; at the benchmark's expert geometry (7168 /
2048, 3 bits) against the oracle, and the whole 257-expert layer by
properties that hold at any size (row independence, token order,
determinism).
"""

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as O
from tests.exl3_cases import random_acts, random_matrix

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from vllm_mi355x.kernels.exl3 import ops as exl3_ops
    exl3_ops.ensure_extension()
    return exl3_ops


def _dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _out_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return O.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.float().cpu().numpy()


def _oracle_f32(out, code):
    return O.bf16_bits_to_f32(out) if code == O.BF16 else out.astype(np.float32)


# Absolute part of the MoE bar, in units of rms(ref).  Both expert kernels
# (the small-M GEMV and the many-row tile GEMM) carry ~22-bit activations
# (FP16 high + low parts): 2^-13, and an rms error within 2^-10 rms(ref).
# Under exl3_set_tile_precision(1) (an opt-in below the reference's
# precision) the tile GEMM rounds each rotated input once to FP16, about
# 2^-11 rms(ref) of error through the three projections, which also moves
# bf16 outputs across rounding boundaries (one bf16 ulp, 2^-8 relative, for
# about one output in 16): 2^-8 (max-abs), and an rms error within 2^-8
# rms(ref).
GEMV_ABS_RMS = 2.0 ** -13
FP16_ABS_RMS = 2.0 ** -8


def _assert_moe_close(actual, expected, name, abs_rms=GEMV_ABS_RMS, rms_bar=None):
    expected = expected.astype(np.float64)
    rms = float(np.sqrt(np.mean(expected ** 2)))
    err = np.abs(actual.astype(np.float64) - expected)
    bound = 2.0 ** -7 * np.abs(expected) + abs_rms * rms
    worst = int(np.argmax(err - bound))
    assert np.isfinite(actual).all(), f"{name}: non-finite output"
    assert (err <= bound).all(), (
        f"{name}: err {err.flat[worst]:.3g} > {bound.flat[worst]:.3g} (rms {rms:.3g})")
    if rms_bar is None:
        rms_bar = 2.0 ** -8 if abs_rms >= FP16_ABS_RMS else 2.0 ** -10
    assert np.sqrt(np.mean(err ** 2)) <= rms_bar * rms, f"{name}: rms error"


class Layer:
    """Random local experts (gate, up, down) on the host and the device, with
    the packed_ptrs / packed_meta tables (reference quant.py:1105-1134)."""

    def __init__(self, rng, experts, hidden, intermediate, formats, device, scales="test"):
        hpad, ipad = -(-hidden // 128) * 128, -(-intermediate // 128) * 128
        self.host = []
        for e in range(experts):
            projections = []
            for p, (k, n) in enumerate(((hpad, ipad), (hpad, ipad), (ipad, hpad))):
                bits_x2, codebook = formats[(e + p) % len(formats)]
                t, u, v = random_matrix(rng, k, n, bits_x2, scales=scales)
                projections.append((t, u, v, bits_x2, codebook))
            self.host.append(projections)
        self.oracle = O.MoELayer(self.host)
        self.keep = []
        ptrs, meta = [], []
        for projections in self.host:
            ptrs.append([])
            meta.append([])
            for t, u, v, bits_x2, codebook in projections:
                tensors = [_dev(a, device) for a in (t, u, v)]
                self.keep.append(tensors)
                ptrs[-1].append([a.data_ptr() for a in tensors])
                meta[-1].append([u.size, v.size, bits_x2, codebook])
        self.ptrs = torch.tensor(ptrs, dtype=torch.int64, device=device).reshape(experts, 3, 3)
        self.meta = torch.tensor(meta, dtype=torch.int64, device=device).reshape(experts, 3, 4)


def _run(ops, x, ids, weights, layer, expert_map, intermediate, limit=0.0, bits_x2=None,
         poison=True):
    rows, hidden = x.shape
    size = ops.moe_workspace_size(rows, hidden, intermediate, ids.shape[1], layer.ptrs.shape[0])
    workspace = torch.empty(max(size, 1), dtype=torch.float32, device=x.device)
    if poison:
        workspace.fill_(float("nan"))
    out = torch.full_like(x, float("nan"))
    if bits_x2 is None:
        ops.moe_out(x, ids, weights, layer.ptrs, layer.meta, expert_map, intermediate, out,
                    workspace, swiglu_limit=limit)
    else:
        ops.moe_out_v2(x, ids, weights, layer.ptrs, layer.meta, expert_map, intermediate, bits_x2,
                       out, workspace, swiglu_limit=limit)
    torch.cuda.synchronize()
    return out


def _acts(rng, rows, hidden, dtype, device, scale=1.0):
    a, code = random_acts(rng, rows, hidden, dtype)
    if scale != 1.0:
        v = (O.bf16_bits_to_f32(a) if code == O.BF16 else a.astype(np.float32)) * scale
        a = O.f32_to_bf16_bits(v) if code == O.BF16 else v.astype(np.float16)
    t = _dev(a, device)
    return a, code, (t.view(torch.bfloat16) if code == O.BF16 else t)


@pytest.mark.parametrize("rows", [1, 5, 33])
@pytest.mark.parametrize("id_dtype", [torch.int64, torch.int32])
def test_moe_matches_oracle_with_expert_map_and_masked_routes(ops, device, rows, id_dtype):
    print(f"moe mixed formats rows={rows} ids={id_dtype}", flush=True)
    rng = np.random.default_rng(rows)
    hidden, intermediate, local, global_experts, topk = 256, 200, 4, 8, 3
    layer = Layer(rng, local, hidden, intermediate, [(10, 2), (7, 2), (6, 1), (16, 2)], device)
    # global experts 1, 3, 4, 6 are local; the rest belong to another rank
    expert_map = np.full(global_experts, -1, np.int64)
    expert_map[[1, 3, 4, 6]] = np.arange(4)
    ids = rng.integers(-1, global_experts + 1, (rows, topk))
    ids[0] = [3, -1, global_experts]  # local, padding, out of range
    weights = rng.uniform(0.05, 0.5, (rows, topk)).astype(np.float32)
    x_host, code, x = _acts(rng, rows, hidden, "bf16", device)
    out = _run(ops, x, _dev(ids, device).to(id_dtype), _dev(weights, device), layer,
               _dev(expert_map, device).to(id_dtype), intermediate)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate)
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), f"moe rows={rows}", GEMV_ABS_RMS)


@pytest.mark.parametrize("bits_x2", [2, 3, 4, 5, 6, 7, 8, 10, 16])
@pytest.mark.parametrize("rows,dtype", [(1, "bf16"), (9, "fp16"), (40, "bf16")])
def test_moe_v2_fixed_rate_matches_oracle_and_moe_out(ops, device, bits_x2, rows, dtype):
    """moe_out_v2 at a layer rate (2..8: the fixed-rate kernels; 10 and 16,
    as the reference's (2560, 640, 10) v2 layer: the run-time-rate kernel)
    against the oracle and bitwise against moe_out."""
    print(f"moe_v2 bits_x2={bits_x2} rows={rows} {dtype}", flush=True)
    rng = np.random.default_rng(1000 * bits_x2 + rows)
    hidden, intermediate, experts, topk = 384, 256, 6, 4
    layer = Layer(rng, experts, hidden, intermediate, [(bits_x2, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, dtype, device)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    fixed = _run(ops, x, *args, bits_x2=bits_x2)
    generic = _run(ops, x, *args)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate,
                         out_dtype=code)
    _assert_moe_close(_out_np(fixed), _oracle_f32(expected, code), f"v2 bits_x2={bits_x2}", GEMV_ABS_RMS)
    assert torch.equal(fixed.view(torch.int16), generic.view(torch.int16))


def test_moe_skewed_routes_many_tasks(ops, device):
    """Routes concentrated on a few experts: experts with many 8-row tasks,
    experts with none, and a task table longer than the expert count."""
    print("moe skewed", flush=True)
    rng = np.random.default_rng(7)
    hidden, intermediate, experts, topk, rows = 256, 384, 16, 4, 48
    layer = Layer(rng, experts, hidden, intermediate, [(4, 2)], device, scales="sign")
    p = 1.0 / np.arange(1, experts + 1) ** 1.1
    p /= p.sum()
    ids = np.stack([rng.choice(experts, topk, replace=False, p=p) for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, "bf16", device)
    out = _run(ops, x, _dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device),
               intermediate, bits_x2=4)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate)
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), "moe skewed")


def test_moe_swiglu_clamp_at_routed_expert_shape(ops, device):
    """hidden 5120, intermediate 2304, 3 bpw mul1 (reference
    test_exl3_moe_swiglu_clamp.py): the clamp matches the oracle, a limit
    no activation reaches equals no limit, a reaching limit changes it."""
    print("moe swiglu clamp 5120x2304", flush=True)
    rng = np.random.default_rng(0)
    hidden, intermediate, experts, topk, rows = 5120, 2304, 4, 2, 4
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)]).astype(np.int32)
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int32)
    x_host, code, x = _acts(rng, rows, hidden, "bf16", device, scale=4.0)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    results = {}
    for limit in (0.0, 0.5, 1e30):
        results[limit] = _run(ops, x, *args, limit=limit, bits_x2=6)
    # A reaching clamp keeps only gate values near zero, whose absolute FP32
    # error is that of the large pre-clamp sums (|g| ~ 300 here, summed in
    # another order by the oracle's sequential chain): fp16-scale bar,
    # 2^-10 rms(ref), there.
    for limit, abs_rms in ((0.0, GEMV_ABS_RMS), (0.5, 2.0 ** -10)):
        expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate,
                             swiglu_limit=limit)
        _assert_moe_close(_out_np(results[limit]), _oracle_f32(expected, code), f"limit {limit}",
                          abs_rms)
    assert torch.equal(results[1e30], results[0.0])
    assert not torch.equal(results[0.5], results[0.0])


def test_moe_deterministic_and_workspace_independent(ops, device):
    rng = np.random.default_rng(11)
    hidden, intermediate, experts, topk, rows = 512, 256, 8, 4, 24
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2), (4, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    _, _, x = _acts(rng, rows, hidden, "bf16", device)
    args = (_dev(ids, device), _dev(weights, device), layer,
            torch.arange(experts, device=device), intermediate)
    first = _run(ops, x, *args, poison=True)
    second = _run(ops, x, *args, poison=False)
    third = _run(ops, x, *args, poison=True)
    assert torch.equal(first.view(torch.int16), second.view(torch.int16))
    assert torch.equal(first.view(torch.int16), third.view(torch.int16))


def test_moe_input_at_two_byte_offset(ops, device):
    """The forming reads x rows with 16-byte loads at any alignment: x at a
    2-byte offset (a view into a larger buffer) gives the aligned call's
    outputs bitwise, on the GEMV path and with the forming one wavefront a
    row (8192 or more routed slots)."""
    rng = np.random.default_rng(17)
    hidden, intermediate, experts, topk = 512, 256, 8, 8
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device, scales="sign")
    for rows in (24, 1100):
        ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
        weights = rng.random((rows, topk)).astype(np.float32)
        _, _, x = _acts(rng, rows, hidden, "bf16", device)
        flat = torch.zeros(rows * hidden + 1, dtype=x.dtype, device=device)
        x_odd = flat[1:].view(rows, hidden)
        x_odd.copy_(x)
        assert x_odd.data_ptr() % 16 == 2
        args = (_dev(ids, device), _dev(weights, device), layer,
                torch.arange(experts, device=device), intermediate)
        aligned = _run(ops, x, *args, bits_x2=6)
        shifted = _run(ops, x_odd, *args, bits_x2=6)
        assert torch.isfinite(aligned.float()).all()
        assert torch.equal(aligned.view(torch.int16), shifted.view(torch.int16)), f"rows={rows}"


def test_moe_fully_masked_and_empty(ops, device):
    rng = np.random.default_rng(3)
    hidden, intermediate, experts, topk, rows = 256, 128, 2, 2, 5
    layer = Layer(rng, experts, hidden, intermediate, [(4, 2)], device)
    _, _, x = _acts(rng, rows, hidden, "bf16", device)
    weights = torch.rand(rows, topk, device=device)
    emap = torch.arange(experts, device=device)
    # every route masked or remote
    ids = torch.tensor([[-1, 2]] * rows, device=device)
    out = _run(ops, x, ids, weights, layer, emap, intermediate)
    assert torch.equal(out, torch.zeros_like(out))
    # no local experts at all
    empty = Layer(rng, 0, hidden, intermediate, [(4, 2)], device)
    empty.ptrs = torch.zeros(0, 3, 3, dtype=torch.int64, device=device)
    empty.meta = torch.zeros(0, 3, 4, dtype=torch.int64, device=device)
    out = _run(ops, x, torch.zeros(rows, topk, dtype=torch.int64, device=device), weights, empty,
               torch.full((experts,), -1, device=device), intermediate)
    assert torch.equal(out, torch.zeros_like(out))
    # zero rows: nothing to do
    out = _run(ops, x[:0], ids[:0], weights[:0], layer, emap, intermediate)
    assert out.shape == (0, hidden)


def test_moe_expert_geometry_mismatch_gives_nan_rows(ops, device):
    """An expert whose metadata disagrees with the layer's padded sizes is
    never read out of bounds: tokens routed to it come out NaN."""
    rng = np.random.default_rng(5)
    hidden, intermediate, experts, topk, rows = 256, 128, 3, 1, 6
    layer = Layer(rng, experts, hidden, intermediate, [(4, 2)], device)
    layer.meta[1, 0, 0] = 128  # gate claims 128 input rows
    ids = torch.tensor([[0], [1], [2], [1], [0], [2]], device=device)
    _, _, x = _acts(rng, rows, hidden, "bf16", device)
    out = _run(ops, x, ids, torch.ones(rows, topk, device=device), layer,
               torch.arange(experts, device=device), intermediate).float()
    bad = (ids[:, 0] == 1)
    assert torch.isnan(out[bad]).all()
    assert torch.isfinite(out[~bad]).all()


def test_moe_v2_full_expert_geometry_matches_oracle(ops, device):
    """The routed-expert geometry of the 3-bit MoE decode workload (hidden
    7168, intermediate 2048, mul1): four local experts, the last taken by
    every token as a shared expert with weight 1, with the reference's test
    scales (svh ~ 0.05 N(0, 1): the +-1 benchmark scales overflow FP16 in the
    down projection of random weights).  moe_out_v2 against the oracle, and
    moe_out bitwise."""
    print("moe_v2 full expert geometry 7168/2048 3-bit", flush=True)
    rng = np.random.default_rng(7168)
    hidden, intermediate, experts, rows = 7168, 2048, 4, 4
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device)
    routed = np.stack([rng.permutation(experts - 1)[:2] for _ in range(rows)])
    ids = np.concatenate([routed, np.full((rows, 1), experts - 1)], 1)
    weights = np.concatenate([rng.random((rows, 2)), np.ones((rows, 1))], 1).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, "fp16", device)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    fixed = _run(ops, x, *args, bits_x2=6)
    generic = _run(ops, x, *args)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate,
                         out_dtype=code)
    _assert_moe_close(_out_np(fixed), _oracle_f32(expected, code), "full expert geometry")
    assert torch.equal(fixed.view(torch.int16), generic.view(torch.int16))


def test_moe_v2_full_layer_row_independent_and_deterministic(ops, device):
    """The whole 3-bit MoE layer of the decode workload (256 routed experts +
    1 shared, hidden 7168, intermediate 2048, top-8 from Zipf(1.1)-skewed
    logits, 64 tokens), checked by properties that hold at any size: a
    token's output depends only on its own row and routes (the rows of a
    task are independent MFMA columns, each with its own scale), so
    reordering the tokens reorders the outputs bitwise and a token routed
    alone gets the same bits; two calls agree bitwise; every output is
    finite and nonzero somewhere."""
    print("moe_v2 full layer 257 x 7168/2048 3-bit, 64 tokens", flush=True)
    hidden, intermediate, experts, topk, rows, bits_x2 = 7168, 2048, 256, 8, 64, 6
    gen = torch.Generator(device=device)
    gen.manual_seed(64)
    keep, ptrs, meta = [], [], []
    for _ in range(experts + 1):
        p, m = [], []
        for kk, nn in ((hidden, intermediate), (hidden, intermediate), (intermediate, hidden)):
            t = torch.randint(-(2 ** 15), 2 ** 15, (kk // 16, nn // 16, 8 * bits_x2), dtype=torch.int16,
                              device=device, generator=gen)
            # the reference's test scales (the +-1 benchmark scales overflow
            # FP16 in the down projection of random weights)
            u = torch.randn(kk, device=device, generator=gen).half()
            v = (0.05 * torch.randn(nn, device=device, generator=gen)).half()
            keep += [t, u, v]
            p.append([t.data_ptr(), u.data_ptr(), v.data_ptr()])
            m.append([kk, nn, bits_x2, 2])
        ptrs.append(p)
        meta.append(m)

    class Full:
        pass

    Full.ptrs = torch.tensor(ptrs, dtype=torch.int64, device=device)
    Full.meta = torch.tensor(meta, dtype=torch.int64, device=device)
    ranks = torch.randperm(experts, generator=torch.Generator().manual_seed(65)).float() + 1.0
    logits = torch.randn(rows, experts, generator=gen, device=device) + (-1.1 * torch.log(ranks)).to(device)
    tw, ti = torch.topk(torch.softmax(logits, -1), topk, dim=-1)
    tw = tw / tw.sum(-1, keepdim=True)
    ids = torch.cat([ti.int(), torch.full((rows, 1), experts, dtype=torch.int32, device=device)], 1)
    weights = torch.cat([tw.float(), torch.ones(rows, 1, device=device)], 1).contiguous()
    emap = torch.arange(experts + 1, dtype=torch.int32, device=device)
    x = torch.randn(rows, hidden, generator=gen, device=device).half()

    def call(xx, ii, ww):
        return _run(ops, xx, ii.contiguous(), ww.contiguous(), Full, emap, intermediate, bits_x2=bits_x2,
                    poison=False)

    out = call(x, ids, weights)
    assert torch.isfinite(out.float()).all() and out.float().abs().max() > 0
    assert torch.equal(out.view(torch.int16), call(x, ids, weights).view(torch.int16))
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(66)).to(device)
    permuted = call(x[perm], ids[perm], weights[perm])
    assert torch.equal(permuted.view(torch.int16), out[perm].view(torch.int16))
    # routed alone, a token's experts run on the small-M GEMV, whose FP32
    # summation order differs from the tile GEMM's (the shared expert has 64
    # rows here): the same value to the MoE bar
    for r in (0, 37):
        alone = call(x[r:r + 1], ids[r:r + 1], weights[r:r + 1])
        _assert_moe_close(_out_np(alone), _out_np(out[r:r + 1]).astype(np.float64), f"token {r}")
    del keep


@pytest.fixture()
def tile_rows():
    from vllm_mi355x import _native
    lib = _native.load()

    def force(rows):
        _native.check(lib.exl3_set_moe_tile_rows(rows))

    yield force
    _native.check(lib.exl3_set_moe_tile_rows(0))


@pytest.fixture()
def tile_fp16():
    """exl3_set_tile_precision: True = the tile GEMM on FP16 high parts
    alone; reset to the default (high and low parts) after the test."""
    from vllm_mi355x import _native
    lib = _native.load()

    def set_(on):
        _native.check(lib.exl3_set_tile_precision(int(on)))

    yield set_
    _native.check(lib.exl3_set_tile_precision(0))


@pytest.mark.parametrize("bits_x2", [2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16])
@pytest.mark.parametrize("rows,dtype", [(5, "bf16"), (40, "fp16"), (96, "bf16"), (120, "fp16")])
def test_moe_tile_path_matches_oracle_and_gemv(ops, device, tile_rows, bits_x2, rows, dtype):
    """Every expert on the many-row tile GEMM (threshold forced to 1 row),
    at every mul1 rate: against the oracle, and against the small-M GEMV
    path to the same bar (the two sum in different FP32 orders).  Experts
    of ~3, ~27, ~64 and ~80 routed rows: the task loops of 2, 4, 5, 6 and 8
    row blocks."""
    print(f"moe tile path bits_x2={bits_x2} rows={rows} {dtype}", flush=True)
    rng = np.random.default_rng(3000 * bits_x2 + rows)
    hidden, intermediate, experts, topk = 384, 256 + 128, 6, 4
    layer = Layer(rng, experts, hidden, intermediate, [(bits_x2, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    ids[0, -1] = -1  # a masked route
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, dtype, device)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    tile_rows(1)
    tiled = _run(ops, x, *args, bits_x2=bits_x2)
    again = _run(ops, x, *args, bits_x2=bits_x2)
    tile_rows(1 << 30)
    gemv = _run(ops, x, *args, bits_x2=bits_x2)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate,
                         out_dtype=code)
    _assert_moe_close(_out_np(tiled), _oracle_f32(expected, code), f"tile bits_x2={bits_x2}")
    _assert_moe_close(_out_np(tiled), _out_np(gemv).astype(np.float64), "tile vs gemv")
    assert torch.equal(tiled.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("bits_x2", [3, 8, 10, 16])
def test_moe_tile_fp16_precision_opt_in(ops, device, tile_rows, tile_fp16, bits_x2):
    """exl3_set_tile_precision(1): the tile experts' rows on FP16 high parts
    alone, at the FP16-operand bar; the default afterwards meets the
    GEMV's bar again."""
    print(f"moe tile fp16 opt-in bits_x2={bits_x2}", flush=True)
    rng = np.random.default_rng(3500 + bits_x2)
    hidden, intermediate, experts, topk, rows = 384, 384, 6, 4, 40
    layer = Layer(rng, experts, hidden, intermediate, [(bits_x2, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, "bf16", device)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    expected = _oracle_f32(O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map,
                                     intermediate, out_dtype=code), code)
    tile_rows(1)
    tile_fp16(True)
    fp16 = _run(ops, x, *args, bits_x2=bits_x2)
    _assert_moe_close(_out_np(fp16), expected, f"fp16 tile bits_x2={bits_x2}", FP16_ABS_RMS)
    tile_fp16(False)
    hilo = _run(ops, x, *args, bits_x2=bits_x2)
    _assert_moe_close(_out_np(hilo), expected, f"hi/lo tile bits_x2={bits_x2}")


@pytest.mark.parametrize("path", ["gemv", "tile"])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_moe_ragged_logical_sizes_match_oracle(ops, device, tile_rows, path, dtype):
    """Logical hidden / intermediate sizes that end inside an 8-input chunk
    (300 and 250, padded to 384 and 256): the forming kernels read the last
    chunk of x, suh and the gate / up results one element at a time, and the
    padded inputs past the logical size form zero; on the GEMV path and on
    the tile path (whose down projection also has a partial 256-column
    tile), against the oracle."""
    print(f"moe ragged sizes path={path} {dtype}", flush=True)
    rng = np.random.default_rng(4242 if path == "gemv" else 4243)
    hidden, intermediate, experts, topk, rows = 300, 250, 5, 3, 40
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, dtype, device)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    tile_rows(1 if path == "tile" else 1 << 30)
    out = _run(ops, x, *args, bits_x2=6)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate,
                         out_dtype=code)
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), f"ragged {path}")


def test_moe_tile_path_clamp_geometry_and_alignment(ops, device, tile_rows, tile_fp16):
    """The tile path with the SwiGLU clamp, an expert of the wrong geometry
    (NaN rows, never read) and expert matrices at 2-byte offsets (routed to
    the GEMV, which reads any alignment)."""
    print("moe tile path clamp / geometry / alignment", flush=True)
    rng = np.random.default_rng(77)
    hidden, intermediate, experts, topk, rows = 512, 256, 4, 2, 48
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, "bf16", device, scale=4.0)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    tile_rows(1)
    out = _run(ops, x, *args, limit=0.5, bits_x2=6)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate,
                         swiglu_limit=0.5)
    # The clamp at 0.5 cuts gate / up sums of magnitude ~100 (inputs x4 over
    # 512 inputs); the sums' absolute error, which the clamp does not shrink
    # where it lets values through, is in units of that pre-clamp scale:
    # with high and low parts (~22 bits) a bar of 2^-10 rms(ref), as the
    # GEMV's clamp case; FP16 operands alone (the opt-in) leave ~2^-12 of
    # the pre-clamp magnitude: 2^-4 rms(ref) max-abs and 2^-6 rms(ref) rms
    # (an unclamped result is off by O(rms(ref))).
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), "tile clamp", 2.0 ** -10)
    tile_fp16(True)
    out = _run(ops, x, *args, limit=0.5, bits_x2=6)
    tile_fp16(False)
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), "fp16 tile clamp", 2.0 ** -4,
                      2.0 ** -6)
    # expert 2 at 2-byte offsets: GEMV tasks; the others stay on tiles
    ptrs = layer.ptrs.cpu().numpy()
    for p, (t, _, _, _, _) in enumerate(layer.host[2]):
        flat = torch.empty(t.size + 2, dtype=torch.int16, device=device)
        view = flat[1:1 + t.size].view(t.shape)
        view.copy_(_dev(t, device))
        layer.keep.append([flat])
        ptrs[2, p, 0] = view.data_ptr()
    layer.ptrs = torch.from_numpy(ptrs).to(device)
    out = _run(ops, x, *args, bits_x2=6)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate)
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), "tile + unaligned expert")
    # expert 1 claims another geometry: its tokens come out NaN
    layer.meta[1, 0, 0] = 128
    out = _run(ops, x, *args, bits_x2=6).float()
    bad = torch.from_numpy((ids == 1).any(1)).to(device)
    assert torch.isnan(out[bad]).all() and torch.isfinite(out[~bad]).all()


def test_moe_rejects_bad_arguments(ops, device):
    rng = np.random.default_rng(9)
    hidden, intermediate, experts, topk, rows = 256, 128, 2, 2, 3
    layer = Layer(rng, experts, hidden, intermediate, [(4, 2)], device)
    _, _, x = _acts(rng, rows, hidden, "bf16", device)
    ids = torch.zeros(rows, topk, dtype=torch.int64, device=device)
    weights = torch.ones(rows, topk, device=device)
    emap = torch.arange(experts, device=device)
    size = ops.moe_workspace_size(rows, hidden, intermediate, topk, experts)
    ws = torch.empty(size, dtype=torch.float32, device=device)
    out = torch.empty_like(x)
    with pytest.raises(RuntimeError, match="workspace"):
        ops.moe_out(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate, out, ws[:size - 1])
    with pytest.raises(RuntimeError, match="dtype"):
        ops.moe_out(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate,
                    torch.empty(rows, hidden, dtype=torch.float16, device=device), ws)
    with pytest.raises(RuntimeError, match="swiglu"):
        ops.moe_out(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate, out, ws,
                    swiglu_limit=-1.0)
    with pytest.raises(RuntimeError, match="geometry"):
        ops.moe_out(x, ids[:1], weights[:1], layer.ptrs, layer.meta, emap, intermediate, out, ws)
    with pytest.raises(RuntimeError, match="mul1"):
        ops.moe_out_v2(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate, 9, out, ws)
