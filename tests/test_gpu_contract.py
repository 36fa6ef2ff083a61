"""The drop-in contract on the GPU, beyond the per-kernel parity tests:

  * the CPU-plumbing linear (4096 x 4096, 4 bits, mul1, +-1 x N(1, 0.05)
    scales, M = 1) against the oracle;
  * every aliased _exl3_C schema (the reference's variants with one
    contract) called once, bitwise equal to the operator that serves it;
  * the small-M path's column ranges (a workspace sized for the automatic
    plan under a forced plan that needs more) and unaligned trellis bases at
    every block count, against the oracle and bitwise against one range;
  * two graphs captured on one stream and replayed concurrently on two
    streams (their arrival counters must not collide);
  * exl3_linear's row chunking, moe_sum_add (the shared-expert fold),
    moe_out_v2 at 5 bits (bits_x2 10, the reference's first served v2
    layer, 2560 / 640) and expert trellises at 2-byte offsets.

Bars as the kernel tests state them (test_gpu_exl3_linear.py,
test_gpu_exl3_moe.py); moe_sum_add is bit-exact against a NumPy statement
of its two roundings.
"""

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as O
from tests.exl3_cases import random_acts, random_matrix
from tests.test_gpu_exl3_linear import _assert_fp32_close, _assert_round_close, _dev, _out_np, \
    _run_linear, _to_torch_act
from tests.test_gpu_exl3_moe import Layer, _acts, _assert_moe_close, _oracle_f32, _run

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from vllm_mi355x.kernels.exl3 import ops as exl3_ops
    exl3_ops.ensure_extension()
    return exl3_ops


@pytest.fixture()
def native():
    from vllm_mi355x import _native
    lib = _native.load()
    yield _native, lib
    _native.check(lib.exl3_set_gemv_blocks(0))
    _native.check(lib.exl3_set_gemv_groups(0))
    _native.check(lib.exl3_set_gemv_finish(-1))


@pytest.mark.parametrize("x_dtype", ["fp16", "bf16"])
def test_cpu_plumbing_linear_4096(ops, device, x_dtype):
    print(f"C1 linear 4096x4096 4-bit M=1 {x_dtype}", flush=True)
    rng = np.random.default_rng(4096)
    trellis, suh, svh = random_matrix(rng, 4096, 4096, 8)
    x, code = random_acts(rng, 1, 4096, x_dtype)
    got = _run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, 4096, torch.float32)
    want = O.linear_out(x, code, trellis, suh, svh, 8, 2, 4096, O.FP32)
    _assert_fp32_close(_out_np(got), want, "C1")
    out_dtype = torch.float16 if x_dtype == "fp16" else torch.bfloat16
    got16 = _run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, 4096, out_dtype)
    want16 = O.linear_out(x, code, trellis, suh, svh, 8, 2, 4096, O.FP16 if x_dtype == "fp16" else O.BF16)
    want16 = want16.astype(np.float32) if x_dtype == "fp16" else O.bf16_bits_to_f32(want16)
    got16 = _out_np(got16)
    if x_dtype == "fp16":
        rms = float(np.sqrt(np.mean(want16.astype(np.float64) ** 2)))
        err = np.abs(got16.astype(np.float64) - want16)
        assert (err <= 2.0 ** -10 * np.abs(want16) + 2.0 ** -14 * rms).all(), "C1 fp16 out"
    else:
        _assert_round_close(got16, want16, "C1 bf16 out")


def test_every_linear_alias_matches_linear_out(ops, device):
    rng = np.random.default_rng(21)
    trellis, suh, svh = random_matrix(rng, 512, 384, 8, scales="test")
    for rows in (3, 40):
        print(f"linear aliases rows={rows}", flush=True)
        x, code = random_acts(rng, rows, 500, "bf16")
        args = (_to_torch_act(x, code, device), _dev(trellis, device), _dev(suh, device),
                _dev(svh, device), 8, 2, 500, 380)
        results = {}
        for name in ("linear_out", "linear_out_splitk", "linear_out_prefill"):
            out = torch.empty(rows, 380, dtype=torch.bfloat16, device=device)
            ws = torch.empty(ops.linear_workspace_size(rows, 512, 384), dtype=torch.float32, device=device)
            getattr(torch.ops._exl3_C, name)(*args, out, ws)
            results[name] = out
        torch.cuda.synchronize()
        for name, out in results.items():
            assert torch.equal(out, results["linear_out"]), name


def test_every_moe_alias_matches_its_operator(ops, device):
    print("moe aliases", flush=True)
    rng = np.random.default_rng(22)
    hidden, intermediate, experts, topk, rows = 256, 256, 4, 2, 5
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device, scales="sign")
    ids = torch.from_numpy(np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])).to(device)
    weights = torch.from_numpy(rng.random((rows, topk)).astype(np.float32)).to(device)
    emap = torch.arange(experts, device=device)
    _, _, x = _acts(rng, rows, hidden, "bf16", device)
    size = ops.moe_workspace_size(rows, hidden, intermediate, topk, experts)

    def call(name, *extra, limit=None):
        out = torch.full_like(x, float("nan"))
        ws = torch.empty(size, dtype=torch.float32, device=device)
        fn = getattr(torch.ops._exl3_C, name)
        tail = () if limit is None else (limit,)
        fn(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate, *extra, out, ws, *tail)
        torch.cuda.synchronize()
        return out.view(torch.int16)

    base = call("moe_out")
    assert torch.equal(call("moe_out_mixed"), base)
    v2 = call("moe_out_v2", 6)
    assert torch.equal(v2, base)
    for name in ("moe_out_v2_fold", "moe_out_prefill_v2", "moe_out_prefill_try", "moe_out_v2_mixed",
                 "moe_out_prefill_try_mixed"):
        assert torch.equal(call(name, 6), v2), name
    for name in ("moe_out_v2_try", "moe_out_v2_try_mixed"):
        assert torch.equal(call(name, 6, limit=0.0), v2), name
    # moe_out_prefill: moe_out's schema at the one rate the reference's
    # operator is built for (bits_x2 10, mul1); an expert of another format
    # gives NaN rows (the reference's kernel traps)
    assert torch.isnan(call("moe_out_prefill").view(x.dtype)).all()
    layer = Layer(rng, experts, hidden, intermediate, [(10, 2)], device, scales="sign")
    base = call("moe_out")
    assert torch.equal(call("moe_out_prefill"), base)
    assert torch.equal(call("moe_out_v2", 10), base)


def test_linear_column_ranges_match_one_range(ops, device, native):
    """A forced one-block plan at K = 8192 needs twice the automatic plan's
    K-split partials: with the workspace the size function gives, the call
    runs in column ranges; the sums are the same, so bitwise equal."""
    _native, lib = native
    print("linear column ranges", flush=True)
    rng = np.random.default_rng(23)
    k, n, rows = 8192, 384, 3
    trellis, suh, svh = random_matrix(rng, k, n, 8)
    x, code = random_acts(rng, rows, k, "fp16")
    args = (_to_torch_act(x, code, device), _dev(trellis, device), _dev(suh, device), _dev(svh, device),
            8, 2, k, n)
    _native.check(lib.exl3_set_gemv_blocks(1))
    size = ops.linear_workspace_size(rows, k, n)
    outs = []
    for elements in (size, 4 * size):
        out = torch.empty(rows, n, dtype=torch.float32, device=device)
        ops.linear_out(*args, out, torch.empty(elements, dtype=torch.float32, device=device))
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    want = O.linear_out(x, code, trellis, suh, svh, 8, 2, n, O.FP32)
    _assert_fp32_close(outs[0].cpu().numpy(), want, "column ranges")


@pytest.mark.parametrize("offset_bytes", [2, 4])
@pytest.mark.parametrize("blocks", [2, 4, 8])
@pytest.mark.parametrize("bits_x2,codebook", [(8, 2), (3, 2), (12, 1)])
def test_linear_unaligned_trellis_every_block_count(ops, device, native, offset_bytes, blocks, bits_x2,
                                                    codebook):
    _native, lib = native
    print(f"linear unaligned offset={offset_bytes} blocks={blocks} bits_x2={bits_x2}", flush=True)
    rng = np.random.default_rng(600 + offset_bytes + 10 * blocks + bits_x2)
    k, n = 2048, 256
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2, scales="test")
    x, code = random_acts(rng, 2, k, "bf16")
    flat = torch.empty(trellis.size + 8, dtype=torch.int16, device=device)
    view = flat[offset_bytes // 2:offset_bytes // 2 + trellis.size].view(trellis.shape)
    view.copy_(_dev(trellis, device))
    _native.check(lib.exl3_set_gemv_blocks(blocks))
    out = torch.empty(2, n, dtype=torch.float32, device=device)
    ws = torch.empty(ops.linear_workspace_size(2, k, n), dtype=torch.float32, device=device)
    ops.linear_out(_to_torch_act(x, code, device), view, _dev(suh, device), _dev(svh, device), bits_x2,
                   codebook, k, n, out, ws)
    torch.cuda.synchronize()
    want = O.linear_out(x, code, trellis, suh, svh, bits_x2, codebook, n, O.FP32)
    _assert_fp32_close(out.cpu().numpy(), want, f"offset={offset_bytes} blocks={blocks}")


def test_graphs_from_one_stream_replayed_concurrently(ops, device):
    """Two graphs captured on one stream hold their own arrival counters:
    replayed at the same time on two streams, each still matches its eager
    result (counters shared between them would mis-time the finish)."""
    print("graphs replayed concurrently", flush=True)
    k, n = 4096, 14336
    rng = np.random.default_rng(24)
    problems = []
    for _ in range(2):
        trellis, suh, svh = random_matrix(rng, k, n, 8)
        x, code = random_acts(rng, 1, k, "fp16")
        problems.append(dict(args=(_to_torch_act(x, code, device), _dev(trellis, device), _dev(suh, device),
                                   _dev(svh, device), 8, 2, k, n),
                             out=torch.empty(1, n, dtype=torch.float32, device=device),
                             ws=torch.empty(ops.linear_workspace_size(1, k, n), dtype=torch.float32,
                                            device=device)))
    eager = []
    for p in problems:
        ops.linear_out(*p["args"], p["out"], p["ws"])
        torch.cuda.synchronize()
        eager.append(p["out"].clone())
    capture = torch.cuda.Stream()
    graphs = []
    for p in problems:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(capture):
            with torch.cuda.graph(g, stream=capture):
                ops.linear_out(*p["args"], p["out"], p["ws"])
        graphs.append(g)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for it in range(20):
        for p in problems:
            p["out"].zero_()
        torch.cuda.synchronize()
        for g, s in zip(graphs, streams):
            with torch.cuda.stream(s):
                g.replay()
        torch.cuda.synchronize()
        for i, p in enumerate(problems):
            assert torch.equal(p["out"], eager[i]), f"replay {it}, graph {i}"


def test_exl3_linear_row_chunking(ops, device):
    print("exl3_linear row chunks", flush=True)
    rng = np.random.default_rng(25)
    k, n, rows = 1024, 768, 10
    trellis, suh, svh = random_matrix(rng, k, n, 8, scales="test")
    x, code = random_acts(rng, rows, k, "bf16")
    args = (_to_torch_act(x, code, device), _dev(trellis, device), _dev(suh, device), _dev(svh, device),
            8, 2, n)
    want = O.linear_out(x, code, trellis, suh, svh, 8, 2, n, O.FP32)
    for chunk in (3, 4, None):
        got = ops.exl3_linear(*args, row_chunk=chunk, out_dtype=torch.float32)
        torch.cuda.synchronize()
        _assert_fp32_close(got.cpu().numpy(), want, f"row_chunk={chunk}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("strided", [False, True])
def test_moe_sum_add_bit_exact(device, dtype, strided):
    from vllm_mi355x.kernels.moe import routing
    print(f"moe_sum_add {dtype} strided={strided}", flush=True)
    M, topk, H = 37, 8, 2048 + 64
    gen = torch.Generator(device=device)
    gen.manual_seed(26)
    inp = torch.randn(M, topk, H, generator=gen, device=device).to(dtype)
    big = torch.randn(M, H + 16, generator=gen, device=device).to(dtype)
    shared = big[:, 8:8 + H] if strided else big[:, :H].contiguous()
    got = routing.moe_sum_add(inp, shared)
    torch.cuda.synchronize()
    acc = torch.zeros(M, H, dtype=torch.float32, device=device)
    for k in range(topk):  # FP32 in slot order, rounded once
        acc = acc + inp[:, k].float()
    want = (acc.to(dtype).float() + shared.float()).to(dtype)
    assert torch.equal(got, want)


def test_moe_v2_rate_10_at_2560x640(ops, device):
    """moe_out_v2 at bits_x2 10 (reference ops.py:51: (2560, 640, 10, 256,
    512)), run by the run-time decode, against the oracle and moe_out."""
    print("moe_v2 bits_x2=10 2560/640", flush=True)
    rng = np.random.default_rng(27)
    hidden, intermediate, experts, topk, rows = 2560, 640, 4, 2, 6
    layer = Layer(rng, experts, hidden, intermediate, [(10, 2)], device, scales="sign")
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, "bf16", device)
    args = (_dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device), intermediate)
    v2 = _run(ops, x, *args, bits_x2=10)
    generic = _run(ops, x, *args)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate)
    _assert_moe_close(_out_np(v2), _oracle_f32(expected, code), "v2 bits_x2=10")
    assert torch.equal(v2.view(torch.int16), generic.view(torch.int16))
    # an expert of another rate under the layer's rate gives NaN rows
    layer.meta[1, :, 2] = 8
    bad = _run(ops, x, *args, bits_x2=10).float()
    routed_to_1 = torch.from_numpy((ids == 1).any(1)).to(device)
    assert torch.isnan(bad[routed_to_1]).all() and torch.isfinite(bad[~routed_to_1]).all()


@pytest.mark.parametrize("bits_x2", [6, None])
def test_moe_expert_trellis_at_2_byte_offsets(ops, device, bits_x2):
    """Every expert matrix two bytes past a 4-byte boundary: the halfword
    trellis loads of the fixed-rate GEMV and the run-time decode."""
    print(f"moe unaligned trellis bits_x2={bits_x2}", flush=True)
    rng = np.random.default_rng(28)
    hidden, intermediate, experts, topk, rows = 384, 256, 4, 2, 9
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device, scales="sign")
    ptrs = layer.ptrs.cpu().numpy()
    for e, projections in enumerate(layer.host):
        for p, (t, _, _, _, _) in enumerate(projections):
            flat = torch.empty(t.size + 2, dtype=torch.int16, device=device)
            view = flat[1:1 + t.size].view(t.shape)
            view.copy_(_dev(t, device))
            assert view.data_ptr() % 4 == 2
            layer.keep.append([flat])
            ptrs[e, p, 0] = view.data_ptr()
    layer.ptrs = torch.from_numpy(ptrs).to(device)
    ids = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    weights = rng.random((rows, topk)).astype(np.float32)
    expert_map = np.arange(experts, dtype=np.int64)
    x_host, code, x = _acts(rng, rows, hidden, "fp16", device)
    out = _run(ops, x, _dev(ids, device), _dev(weights, device), layer, _dev(expert_map, device),
               intermediate, bits_x2=bits_x2)
    expected = O.moe_out(x_host, code, ids, weights, layer.oracle, expert_map, intermediate,
                         out_dtype=code)
    _assert_moe_close(_out_np(out), _oracle_f32(expected, code), "unaligned expert trellis")


def test_moe_out_row_chunks_match_one_call(device):
    """ops.moe_out / moe_out_v2 in row chunks (forced small here; automatic
    above the 32-bit workspace offset limit) give the single call's outputs
    bitwise: the calls are small enough to stay on the GEMV, whose tokens
    are independent."""
    from vllm_mi355x.kernels.exl3 import ops
    ops.ensure_extension()
    rng = np.random.default_rng(81)
    hidden, intermediate, experts, topk, rows = 256, 128, 4, 2, 11
    layer = Layer(rng, experts, hidden, intermediate, [(6, 2)], device, scales="sign")
    ids = _dev(np.stack([rng.permutation(experts)[:topk] for _ in range(rows)]), device)
    weights = _dev(rng.random((rows, topk)).astype(np.float32), device)
    emap = _dev(np.arange(experts, dtype=np.int64), device)
    _, _, x = _acts(rng, rows, hidden, "bf16", device)
    ws = torch.empty(ops.moe_workspace_size(rows, hidden, intermediate, topk, experts),
                     dtype=torch.float32, device=device)
    for v2 in (False, True):
        outs = []
        for chunk in (None, 3):
            out = torch.empty_like(x)
            if v2:
                ops.moe_out_v2(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate, 6, out, ws,
                               row_chunk=chunk)
            else:
                ops.moe_out(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate, out, ws,
                            row_chunk=chunk)
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), f"v2={v2}"


def test_moe_route_over_many_workgroups_matches_row_chunks(device):
    """A call of 8192 or more routed slots groups its rows by expert over
    many workgroups (per-part counts and places, the tables from the summed
    histograms, then each slot to its row); its outputs equal, bitwise,
    those of the same call in row chunks of fewer slots, which the
    one-workgroup route groups.  moe_out's run-time-format GEMV keeps every
    token independent of the others."""
    from vllm_mi355x.kernels.exl3 import ops
    ops.ensure_extension()
    rng = np.random.default_rng(83)
    hidden, intermediate, experts, topk, rows = 256, 128, 16, 8, 2300
    chunk = 700
    assert rows * topk >= 8192 and chunk * topk < 8192
    layer = Layer(rng, experts, hidden, intermediate, [(4, 2)], device, scales="sign")
    ids_np = np.stack([rng.permutation(experts)[:topk] for _ in range(rows)])
    ids_np[::7, 3] = -1  # masked slots
    ids = _dev(ids_np, device)
    weights = _dev(rng.random((rows, topk)).astype(np.float32), device)
    emap_np = np.arange(experts, dtype=np.int64)
    emap_np[5] = -1  # a remote expert
    emap = _dev(emap_np, device)
    _, _, x = _acts(rng, rows, hidden, "bf16", device)
    ws = torch.empty(ops.moe_workspace_size(rows, hidden, intermediate, topk, experts),
                     dtype=torch.float32, device=device)
    outs = []
    for row_chunk in (None, chunk):
        out = torch.empty_like(x)
        ops.moe_out(x, ids, weights, layer.ptrs, layer.meta, emap, intermediate, out, ws,
                    row_chunk=row_chunk)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0].float()).all()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
