"""EXL3 dense path on the GPU, through the _exl3_C operators and the C-ABI,
against the CPU oracle (oracle/exl3_oracle.c, the reference's scalar
operators restated).

Bars:
  * decoded weights: bit-exact (every format, aligned and unaligned bases);
  * linear_out: the oracle computes the reference's exact FP32 chain; the
    GPU sums on the matrix cores in another order with the activations split
    into FP16 high/low parts (every kernel: the small-M GEMV, the many-row
    tile GEMM and the decode-to-LDS prefill GEMM), so FP32 outputs must
    agree to
    |err| <= 2^-14 * rms(ref) + 2^-16 * |ref| (a few FP32 roundings of a
    K-term sum; a wrong decode or index is off by O(rms)), and BF16 outputs
    within one BF16 ulp (a value next to a rounding boundary may round the
    other way): |err| <= 2^-7 |ref| + 2^-14 rms(ref).
"""

import os

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as O
from tests.exl3_cases import FORMATS, random_acts, random_matrix

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from vllm_mi355x.kernels.exl3 import ops as exl3_ops
    exl3_ops.ensure_extension()
    return exl3_ops


def _dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _to_torch_act(a: np.ndarray, code: int, device):
    t = _dev(a, device)
    return t.view(torch.bfloat16) if code == O.BF16 else t


def _out_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return O.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.float().cpu().numpy()


def _oracle_f32(out, code):
    return O.bf16_bits_to_f32(out) if code == O.BF16 else out.astype(np.float32)


def _assert_fp32_close(actual, expected, name):
    rms = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
    err = np.abs(actual.astype(np.float64) - expected)
    bound = 2.0 ** -14 * rms + 2.0 ** -16 * np.abs(expected)
    worst = int(np.argmax(err - bound))
    assert (err <= bound).all(), f"{name}: err {err.flat[worst]:.3g} > {bound.flat[worst]:.3g} (rms {rms:.3g})"


def _assert_fp16_operand_close(actual, expected, name):
    """The bar of the tile GEMM at FP16 precision (exl3_set_tile_precision(1),
    an opt-in below the reference's precision): each rotated input is
    rounded once to FP16 (relative error <= 2^-11) and the products are
    accumulated in FP32, so an output's error is a sum of K independent
    rounding terms, about 2^-12 rms(ref) in rms.  Bar: every output within
    2^-8 rms(ref) + 2^-10 |ref| (max-abs), and the rms error within 2^-10
    rms(ref)."""
    expected = expected.astype(np.float64)
    rms = float(np.sqrt(np.mean(expected ** 2)))
    err = np.abs(actual.astype(np.float64) - expected)
    bound = 2.0 ** -8 * rms + 2.0 ** -10 * np.abs(expected)
    worst = int(np.argmax(err - bound))
    assert np.isfinite(actual).all(), f"{name}: non-finite output"
    assert (err <= bound).all(), f"{name}: err {err.flat[worst]:.3g} > {bound.flat[worst]:.3g} (rms {rms:.3g})"
    assert np.sqrt(np.mean(err ** 2)) <= 2.0 ** -10 * rms, f"{name}: rms error"


def _assert_round_close(actual, expected, name):
    rms = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
    err = np.abs(actual.astype(np.float64) - expected)
    bound = 2.0 ** -7 * np.abs(expected) + 2.0 ** -14 * rms
    worst = int(np.argmax(err - bound))
    assert (err <= bound).all(), f"{name}: err {err.flat[worst]:.3g} > {bound.flat[worst]:.3g}"


@pytest.mark.parametrize("bits_x2,codebook", FORMATS)
@pytest.mark.parametrize("aligned", [True, False])
def test_decode_bit_exact(ops, device, bits_x2, codebook, aligned):
    print(f"decode bits_x2={bits_x2} codebook={codebook} aligned={aligned}", flush=True)
    rng = np.random.default_rng(100 * bits_x2 + codebook)
    trellis, _, _ = random_matrix(rng, 256, 384, bits_x2)
    expected = O.decode(trellis, bits_x2, codebook).view(np.uint16)
    t = _dev(trellis, device)
    if not aligned:
        # a base two bytes past a 4-byte boundary
        flat = torch.empty(trellis.size + 1, dtype=torch.int16, device=device)
        flat[1:] = t.reshape(-1)
        t = flat[1:].view(trellis.shape)
        assert t.data_ptr() % 4 == 2
    got = ops.decode(t, bits_x2, codebook).view(torch.int16).cpu().numpy().view(np.uint16)
    mismatch = np.argwhere(got != expected)
    assert mismatch.size == 0, f"{len(mismatch)} mismatches, first at {mismatch[0]}"


def _run_linear(ops, device, trellis, suh, svh, x, x_code, bits_x2, codebook, logical_out,
                out_dtype):
    rows = x.shape[0]
    out = torch.empty(rows, logical_out, dtype=out_dtype, device=device)
    ws = torch.empty(ops.linear_workspace_size(rows, suh.size, svh.size), dtype=torch.float32,
                     device=device)
    ops.linear_out(_to_torch_act(x, x_code, device), _dev(trellis, device), _dev(suh, device),
                   _dev(svh, device), bits_x2, codebook, x.shape[1], logical_out, out, ws)
    torch.cuda.synchronize()
    return out


def test_linear_zero_rows(ops, device):
    """An empty batch: linear_out returns with nothing to do, and the row
    chunking (the reference's exl3_linear, ops.py:1455-1486) gives a
    [0, logical_out] result."""
    rng = np.random.default_rng(5)
    trellis, suh, svh = random_matrix(rng, 256, 384, 8, scales="test")
    t, u, v = _dev(trellis, device), _dev(suh, device), _dev(svh, device)
    x = torch.empty(0, 250, dtype=torch.bfloat16, device=device)
    out = torch.empty(0, 300, dtype=torch.bfloat16, device=device)
    ws = torch.empty(ops.linear_workspace_size(1, 256, 384), dtype=torch.float32, device=device)
    ops.linear_out(x, t, u, v, 8, 2, 250, 300, out, ws)
    y = ops.exl3_linear(x, t, u, v, 8, 2, 300)
    torch.cuda.synchronize()
    assert y.shape == (0, 300) and y.dtype == torch.bfloat16


@pytest.mark.parametrize("bits_x2,codebook", FORMATS)
@pytest.mark.parametrize("rows", [1, 3, 8, 17])
def test_linear_matches_oracle(ops, device, bits_x2, codebook, rows):
    print(f"linear bits_x2={bits_x2} codebook={codebook} rows={rows}", flush=True)
    rng = np.random.default_rng(1000 * bits_x2 + 10 * codebook + rows)
    # logical sizes below the padded H128 blocks exercise both crops
    trellis, suh, svh = random_matrix(rng, 256, 384, bits_x2, scales="test")
    logical_in, logical_out = 250, 300
    x, code = random_acts(rng, rows, logical_in, "bf16")
    got = _run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, codebook, logical_out,
                      torch.float32)
    want = O.linear_out(x, code, trellis, suh, svh, bits_x2, codebook, logical_out, O.FP32)
    _assert_fp32_close(_out_np(got), want, f"bits_x2={bits_x2} cb={codebook} rows={rows}")
    got_bf = _run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, codebook, logical_out,
                         torch.bfloat16)
    want_bf = O.linear_out(x, code, trellis, suh, svh, bits_x2, codebook, logical_out, O.BF16)
    _assert_round_close(_out_np(got_bf), O.bf16_bits_to_f32(want_bf), "bf16 out")


@pytest.mark.parametrize("shape", [(4096, 14336), (14336, 4096)])
@pytest.mark.parametrize("bits_x2", [4, 6, 8])
@pytest.mark.parametrize("rows", [1, 4, 8])
def test_linear_benchmark_shapes(ops, device, shape, bits_x2, rows):
    """The GEMV benchmark shapes (fp16 activations, mul1, sign scales)."""
    print(f"linear shape={shape} bits_x2={bits_x2} rows={rows}", flush=True)
    k, n = shape
    rng = np.random.default_rng(7 * k + n + bits_x2 + rows)
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2)
    x, code = random_acts(rng, rows, k, "fp16")
    got = _run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, 2, n, torch.float32)
    want = O.linear_out(x, code, trellis, suh, svh, bits_x2, 2, n, O.FP32)
    _assert_fp32_close(_out_np(got), want, f"{shape} bits_x2={bits_x2} rows={rows}")


def test_linear_rejects_small_workspace(ops, device):
    rng = np.random.default_rng(0)
    trellis, suh, svh = random_matrix(rng, 128, 128, 8)
    x = torch.zeros(2, 128, dtype=torch.bfloat16, device=device)
    out = torch.empty(2, 128, dtype=torch.bfloat16, device=device)
    ws = torch.empty(ops.linear_workspace_size(2, 128, 128) - 1, dtype=torch.float32, device=device)
    with pytest.raises(RuntimeError, match="workspace is too small"):
        ops.linear_out(x, _dev(trellis, device), _dev(suh, device), _dev(svh, device), 8, 2, 128,
                       128, out, ws)


@pytest.mark.parametrize("rows", [1, 8])
def test_linear_repeated_calls_are_bitwise_identical(ops, device, rows):
    """Many calls, alternating two streams (two counter banks of the fused
    finish) and two output buffers: every result must be bitwise the first
    one, and match the oracle."""
    print(f"repeat rows={rows}", flush=True)
    k, n, bits_x2 = 4096, 14336, 8
    rng = np.random.default_rng(31 + rows)
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2)
    x, code = random_acts(rng, rows, k, "fp16")
    t, u, v = _dev(trellis, device), _dev(suh, device), _dev(svh, device)
    xt = _dev(x, device)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    wss = [torch.empty(ops.linear_workspace_size(rows, k, n), dtype=torch.float32, device=device)
           for _ in streams]
    outs = [torch.empty(rows, n, dtype=torch.float32, device=device) for _ in range(2)]
    first = None
    for it in range(60):
        i = it % 2
        with torch.cuda.stream(streams[i]):
            ops.linear_out(xt, t, u, v, bits_x2, 2, k, n, outs[i], wss[i])
        streams[i].synchronize()
        got = outs[i].clone()
        if first is None:
            first = got
        else:
            assert torch.equal(got, first), f"call {it} differs"
    want = O.linear_out(x, code, trellis, suh, svh, bits_x2, 2, n, O.FP32)
    _assert_fp32_close(first.cpu().numpy(), want, "repeated")


def test_linear_graph_replay_matches_eager(ops, device):
    k, n, bits_x2, rows = 2048, 4096, 8, 2
    rng = np.random.default_rng(77)
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2)
    x, _ = random_acts(rng, rows, k, "bf16")
    t, u, v = _dev(trellis, device), _dev(suh, device), _dev(svh, device)
    xt = _dev(x, device).view(torch.bfloat16)
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=device)
    ws = torch.empty(ops.linear_workspace_size(rows, k, n), dtype=torch.float32, device=device)
    ops.linear_out(xt, t, u, v, bits_x2, 2, k, n, out, ws)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            ops.linear_out(xt, t, u, v, bits_x2, 2, k, n, out, ws)
    torch.cuda.synchronize()
    for _ in range(5):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("shape,rows", [((4096, 14336), 1), ((14336, 4096), 1), ((4096, 14336), 8),
                                        ((256, 384), 3)])
def test_linear_fused_and_separate_finish_agree(ops, device, shape, rows):
    """The fused finish (last workgroup per column block) and the separate
    output kernel add the same values in the same order: bitwise equal."""
    from vllm_mi355x import _native
    print(f"finish modes shape={shape} rows={rows}", flush=True)
    k, n = shape
    rng = np.random.default_rng(k + rows)
    trellis, suh, svh = random_matrix(rng, k, n, 8)
    x, code = random_acts(rng, rows, k, "bf16")
    results = []
    lib = _native.load()
    try:
        for mode in (0, 1):
            _native.check(lib.exl3_set_gemv_finish(mode))
            results.append(_run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, n,
                                       torch.float32))
    finally:
        _native.check(lib.exl3_set_gemv_finish(-1))
    assert torch.equal(results[0], results[1])
    if k * n <= 4096 * 4096:
        want = O.linear_out(x, code, trellis, suh, svh, 8, 2, n, O.FP32)
        _assert_fp32_close(_out_np(results[0]), want, "finish modes")


@pytest.mark.parametrize("blocks,groups", [(1, 1), (2, 1), (4, 1), (8, 1), (1, 4), (2, 4), (4, 4)])
@pytest.mark.parametrize("bits_x2,codebook", [(8, 2), (4, 1), (3, 2), (2, 2), (10, 2), (16, 1)])
@pytest.mark.parametrize("rows", [1, 3, 6, 8])
def test_linear_workgroup_shapes_match_oracle(ops, device, blocks, groups, bits_x2, codebook, rows):
    """Every (blocks per group, groups per workgroup) shape of the small-M
    kernel, forced through the tuning switches: same bar as the automatic
    choice (a shape the rate cannot use falls back, and must still agree)."""
    from vllm_mi355x import _native
    print(f"linear shape blocks={blocks} groups={groups} bits_x2={bits_x2} rows={rows}", flush=True)
    rng = np.random.default_rng(100 * blocks + 10 * groups + bits_x2 + rows)
    trellis, suh, svh = random_matrix(rng, 2048, 384, bits_x2, scales="test")
    logical_in, logical_out = 2040, 380
    x, code = random_acts(rng, rows, logical_in, "fp16")
    lib = _native.load()
    try:
        _native.check(lib.exl3_set_gemv_blocks(blocks))
        _native.check(lib.exl3_set_gemv_groups(groups))
        got = _run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, codebook, logical_out,
                          torch.float32)
    finally:
        _native.check(lib.exl3_set_gemv_blocks(0))
        _native.check(lib.exl3_set_gemv_groups(0))
    want = O.linear_out(x, code, trellis, suh, svh, bits_x2, codebook, logical_out, O.FP32)
    _assert_fp32_close(_out_np(got), want, f"blocks={blocks} groups={groups} bits_x2={bits_x2}")


@pytest.mark.parametrize("rows", [5, 8])
@pytest.mark.parametrize("blocks", [2, 4])
def test_linear_row_form_equals_task_form(ops, device, rows, blocks):
    """The 8-row kernel forms its activations eight inputs a lane (16-byte
    loads) when logical_in is a multiple of 8 and x and suh are 16-byte
    aligned, and two inputs a lane per (block, row) otherwise.  The same
    inputs through both (logical_in 2040; 2041 with a zero last input; x at
    a 2-byte offset) give the same outputs, bitwise."""
    from vllm_mi355x import _native
    rng = np.random.default_rng(40 + rows + blocks)
    trellis, suh, svh = random_matrix(rng, 2048, 384, 8, scales="test")
    x, code = random_acts(rng, rows, 2040, "fp16")
    x_pad = np.concatenate([x, np.zeros((rows, 1), x.dtype)], 1)
    lib = _native.load()
    try:
        _native.check(lib.exl3_set_gemv_blocks(blocks))
        a = _run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, 380, torch.float32)
        b = _run_linear(ops, device, trellis, suh, svh, x_pad, code, 8, 2, 380, torch.float32)
        flat = torch.zeros(rows * 2040 + 1, dtype=torch.float16, device=device)
        x_odd = flat[1:].view(rows, 2040)
        x_odd.copy_(_to_torch_act(x, code, device))
        assert x_odd.data_ptr() % 16 == 2
        c = torch.empty(rows, 380, dtype=torch.float32, device=device)
        ws = torch.empty(ops.linear_workspace_size(rows, suh.size, svh.size), dtype=torch.float32,
                         device=device)
        ops.linear_out(x_odd, _dev(trellis, device), _dev(suh, device), _dev(svh, device), 8, 2, 2040, 380,
                       c, ws)
        torch.cuda.synchronize()
    finally:
        _native.check(lib.exl3_set_gemv_blocks(0))
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert torch.equal(a.view(torch.int32), c.view(torch.int32))
    want = O.linear_out(x, code, trellis, suh, svh, 8, 2, 380, O.FP32)
    _assert_fp32_close(_out_np(a), want, f"rows={rows} blocks={blocks}")


@pytest.mark.parametrize("offset_bytes", [2, 4, 8])
@pytest.mark.parametrize("bits_x2,codebook", [(8, 2), (3, 2), (12, 1)])
def test_linear_unaligned_trellis_matches_oracle(ops, device, offset_bytes, bits_x2, codebook):
    """Trellis bases that are not 16-byte aligned take the dword (4, 8) or
    halfword (2) load paths."""
    print(f"linear unaligned offset={offset_bytes} bits_x2={bits_x2}", flush=True)
    rng = np.random.default_rng(500 + offset_bytes + bits_x2)
    trellis, suh, svh = random_matrix(rng, 512, 256, bits_x2, scales="test")
    x, code = random_acts(rng, 2, 512, "bf16")
    flat = torch.empty(trellis.size + 8, dtype=torch.int16, device=device)
    shift = offset_bytes // 2
    view = flat[shift:shift + trellis.size].view(trellis.shape)
    view.copy_(_dev(trellis, device))
    out = torch.empty(2, 256, dtype=torch.float32, device=device)
    ws = torch.empty(ops.linear_workspace_size(2, 512, 256), dtype=torch.float32, device=device)
    ops.linear_out(_to_torch_act(x, code, device), view, _dev(suh, device), _dev(svh, device), bits_x2,
                   codebook, 512, 256, out, ws)
    torch.cuda.synchronize()
    want = O.linear_out(x, code, trellis, suh, svh, bits_x2, codebook, 256, O.FP32)
    _assert_fp32_close(out.cpu().numpy(), want, f"offset={offset_bytes}")


@pytest.mark.parametrize("rows", [9, 32, 33, 64, 300, 513])
@pytest.mark.parametrize("bits_x2,codebook", [(8, 2), (4, 1), (6, 2), (3, 2)])
def test_prefill_matches_oracle(ops, device, rows, bits_x2, codebook):
    """Rows past one small-M launch: up to 32 the small-M kernel in chunks
    of 8 rows, above that the large-M path (decode to LDS + MFMA, output
    transform in its epilogue); rows are independent, so the oracle checks a
    sample of them."""
    print(f"prefill rows={rows} bits_x2={bits_x2} cb={codebook}", flush=True)
    rng = np.random.default_rng(5000 + rows + bits_x2)
    k, n = 1024, 2048 + 128  # a partial 256-column tile too
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2, scales="test")
    logical_in, logical_out = k - 3, n - 5
    x, code = random_acts(rng, rows, logical_in, "bf16")
    got = _out_np(_run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, codebook,
                              logical_out, torch.float32))
    sample = sorted({0, 1, rows // 2, rows - 2, rows - 1})
    want = O.linear_out(x[sample], code, trellis, suh, svh, bits_x2, codebook, logical_out, O.FP32)
    _assert_fp32_close(got[sample], want, f"prefill rows={rows}")


@pytest.mark.parametrize("rows", [40, 300])
def test_prefill_16bit_outputs_are_the_rounded_fp32_outputs(ops, device, rows):
    """The many-row path computes each output in FP32 and rounds it once to
    the output dtype, storing eight columns together where the address
    allows and one at a time otherwise (a width of n - 5 leaves rows at
    every 16-byte phase and a partial last group): its BF16 / FP16 outputs
    are the round-to-nearest-even of its FP32 outputs, bit for bit."""
    print(f"prefill 16-bit outputs rows={rows}", flush=True)
    rng = np.random.default_rng(6100 + rows)
    k, n = 1024, 2048 + 128
    trellis, suh, svh = random_matrix(rng, k, n, 8, scales="test")
    logical_in, logical_out = k - 3, n - 5
    x, code = random_acts(rng, rows, logical_in, "fp16")
    f32 = _run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, logical_out,
                      torch.float32).cpu().numpy()
    assert np.isfinite(f32).all()
    f16 = _run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, logical_out, torch.float16)
    assert np.array_equal(f16.cpu().numpy().view(np.uint16), f32.astype(np.float16).view(np.uint16))
    bf = _run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, logical_out, torch.bfloat16)
    u = f32.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # RNE, finite values
    assert np.array_equal(bf.view(torch.int16).cpu().numpy().view(np.uint16), want)


def test_prefill_benchmark_shape(ops, device):
    """8192 x 28672 at 4 bits, 512 fp16 rows: sampled rows against the oracle."""
    print("prefill 8192x28672 M=512", flush=True)
    k, n, rows = 8192, 28672, 512
    rng = np.random.default_rng(99)
    trellis, suh, svh = random_matrix(rng, k, n, 8)
    x, code = random_acts(rng, rows, k, "fp16")
    got = _out_np(_run_linear(ops, device, trellis, suh, svh, x, code, 8, 2, n, torch.float32))
    sample = [0, 255, 511]
    want = O.linear_out(x[sample], code, trellis, suh, svh, 8, 2, n, O.FP32)
    _assert_fp32_close(got[sample], want, "prefill 8192x28672")


@pytest.fixture()
def prefill_switches():
    """exl3_set_prefill_kernel (0 automatic, 1 the decode-to-LDS prefill_gemm,
    2 the tile GEMM) and exl3_set_tile_precision (1: FP16 high parts alone),
    reset after the test."""
    from vllm_mi355x import _native
    lib = _native.load()

    def kernel(k):
        _native.check(lib.exl3_set_prefill_kernel(k))

    def fp16_only(on):
        _native.check(lib.exl3_set_tile_precision(int(on)))

    yield kernel, fp16_only
    _native.check(lib.exl3_set_prefill_kernel(0))
    _native.check(lib.exl3_set_tile_precision(0))


@pytest.mark.parametrize("rows", [33, 300, 513])
@pytest.mark.parametrize("bits_x2,codebook", [(10, 1), (10, 2), (12, 1), (12, 2), (14, 1), (14, 2),
                                              (16, 1), (16, 2), (3, 2), (8, 2)])
@pytest.mark.parametrize("kernel", [1, 2])
def test_prefill_kernels_every_rate_match_oracle(ops, device, prefill_switches, rows, bits_x2,
                                                 codebook, kernel):
    """Both many-row kernels at the rates above 4 bits per weight (the
    reference's real checkpoints hold mostly bits_x2 10 / 12 / 16 dense
    matrices) and two below, aligned trellis, ragged logical sizes and a
    partial 256-column tile: the decode-to-LDS prefill_gemm (kernel 1) and
    the register-decode tile GEMM (kernel 2), against the oracle on sampled
    rows at the FP32 bar."""
    print(f"prefill kernel={kernel} rows={rows} bits_x2={bits_x2} cb={codebook}", flush=True)
    set_kernel, _ = prefill_switches
    rng = np.random.default_rng(7000 + 100 * bits_x2 + 10 * codebook + rows)
    k, n = 512, 768 + 128
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2, scales="test")
    logical_in, logical_out = k - 5, n - 3
    x, code = random_acts(rng, rows, logical_in, "bf16")
    set_kernel(kernel)
    got = _out_np(_run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, codebook,
                              logical_out, torch.float32))
    sample = sorted({0, 1, rows // 2, rows - 2, rows - 1})
    want = O.linear_out(x[sample], code, trellis, suh, svh, bits_x2, codebook, logical_out, O.FP32)
    _assert_fp32_close(got[sample], want, f"kernel={kernel} rows={rows} bits_x2={bits_x2}")


@pytest.mark.parametrize("offset_bytes", [2, 4])
@pytest.mark.parametrize("bits_x2,codebook", [(10, 2), (12, 1), (14, 2), (16, 1), (16, 2), (8, 2)])
@pytest.mark.parametrize("rows", [33, 300, 513])
def test_prefill_unaligned_trellis_matches_oracle(ops, device, rows, offset_bytes, bits_x2,
                                                  codebook):
    """Many-row calls on trellis bases off a 16-byte boundary take the
    decode-to-LDS prefill_gemm (halfword loads at a 2-byte offset, words at
    a 4-byte one), against the oracle."""
    print(f"prefill unaligned offset={offset_bytes} rows={rows} bits_x2={bits_x2}", flush=True)
    rng = np.random.default_rng(7500 + offset_bytes + 10 * bits_x2 + rows)
    k, n = 512, 384
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2, scales="test")
    x, code = random_acts(rng, rows, k, "fp16")
    flat = torch.empty(trellis.size + 8, dtype=torch.int16, device=device)
    shift = offset_bytes // 2
    view = flat[shift:shift + trellis.size].view(trellis.shape)
    view.copy_(_dev(trellis, device))
    assert view.data_ptr() % 16 == offset_bytes
    out = torch.empty(rows, n, dtype=torch.float32, device=device)
    ws = torch.empty(ops.linear_workspace_size(rows, k, n), dtype=torch.float32, device=device)
    ops.linear_out(_to_torch_act(x, code, device), view, _dev(suh, device), _dev(svh, device),
                   bits_x2, codebook, k, n, out, ws)
    torch.cuda.synchronize()
    sample = sorted({0, rows // 3, rows - 1})
    want = O.linear_out(x[sample], code, trellis, suh, svh, bits_x2, codebook, n, O.FP32)
    _assert_fp32_close(out.cpu().numpy()[sample], want, f"offset={offset_bytes} bits_x2={bits_x2}")


@pytest.mark.parametrize("shape", [(4096, 1024), (5120, 512)])
@pytest.mark.parametrize("kernel", [0, 1])
def test_prefill_checkpoint_geometries_bits10(ops, device, prefill_switches, shape, kernel):
    """Two dense geometries of the reference's real checkpoint inventory
    (tests/models/deepseek_v41/sm80/fixtures/exl3_headers.json: a 4096 ->
    1024 slice and the 5120 -> 512 projection) at bits_x2 10, mul1, 300
    rows, on the automatic kernel and on prefill_gemm."""
    print(f"prefill checkpoint geometry {shape} kernel={kernel}", flush=True)
    set_kernel, _ = prefill_switches
    k, n = shape
    rng = np.random.default_rng(k + n)
    trellis, suh, svh = random_matrix(rng, k, n, 10, scales="test")
    x, code = random_acts(rng, 300, k, "bf16")
    set_kernel(kernel)
    got = _out_np(_run_linear(ops, device, trellis, suh, svh, x, code, 10, 2, n, torch.float32))
    sample = [0, 150, 299]
    want = O.linear_out(x[sample], code, trellis, suh, svh, 10, 2, n, O.FP32)
    _assert_fp32_close(got[sample], want, f"{shape} kernel={kernel}")


@pytest.mark.parametrize("bits_x2,codebook", [(8, 2), (4, 1), (3, 2), (10, 2), (16, 1)])
@pytest.mark.parametrize("rows", [40, 300])
def test_tile_fp16_precision_opt_in(ops, device, prefill_switches, bits_x2, codebook, rows):
    """exl3_set_tile_precision(1): the tile GEMM on the FP16 high parts alone
    (half the MFMAs), at the FP16-operand bar; the default afterwards is
    the FP32 bar again."""
    print(f"tile fp16 opt-in bits_x2={bits_x2} rows={rows}", flush=True)
    _, fp16_only = prefill_switches
    rng = np.random.default_rng(8100 + bits_x2 + rows)
    k, n = 1024, 768
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2, scales="test")
    x, code = random_acts(rng, rows, k, "fp16")
    sample = [0, rows // 2, rows - 1]
    want = O.linear_out(x[sample], code, trellis, suh, svh, bits_x2, codebook, n, O.FP32)
    fp16_only(True)
    got = _out_np(_run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, codebook, n,
                              torch.float32))
    _assert_fp16_operand_close(got[sample], want, f"fp16 bits_x2={bits_x2}")
    fp16_only(False)
    got = _out_np(_run_linear(ops, device, trellis, suh, svh, x, code, bits_x2, codebook, n,
                              torch.float32))
    _assert_fp32_close(got[sample], want, f"hi/lo bits_x2={bits_x2}")


def _graph_nodes(graph) -> int:
    import ctypes
    lib = ctypes.CDLL("libamdhip64.so")
    count = ctypes.c_size_t(0)
    rc = lib.hipGraphGetNodes(ctypes.c_void_p(graph.raw_cuda_graph()), None, ctypes.byref(count))
    assert rc == 0, f"hipGraphGetNodes failed ({rc})"
    return count.value


def test_many_captures_keep_the_fused_finish(ops, device):
    """Every graph captured on one stream shares that stream's arrival-counter
    range: after 220 captures the last graph still holds the one fused GEMV
    launch (no separate output kernel), no launch fell back, and every graph
    replays bitwise equal to the eager call."""
    from vllm_mi355x import _native
    print("220 graph captures on one stream", flush=True)
    lib = _native.load()
    k, n, bits_x2 = 1024, 2048, 8
    rng = np.random.default_rng(220)
    trellis, suh, svh = random_matrix(rng, k, n, bits_x2)
    x, _ = random_acts(rng, 1, k, "fp16")
    t, u, v = _dev(trellis, device), _dev(suh, device), _dev(svh, device)
    xt = _dev(x, device)
    out = torch.empty(1, n, dtype=torch.float32, device=device)
    ws = torch.empty(ops.linear_workspace_size(1, k, n), dtype=torch.float32, device=device)
    ops.linear_out(xt, t, u, v, bits_x2, 2, k, n, out, ws)
    torch.cuda.synchronize()
    eager = out.clone()
    before = lib.exl3_counter_fallbacks()
    stream = torch.cuda.Stream()
    graphs = []
    for _ in range(220):
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                ops.linear_out(xt, t, u, v, bits_x2, 2, k, n, out, ws)
        graph.instantiate()
        graphs.append(graph)
    torch.cuda.synchronize()
    assert lib.exl3_counter_fallbacks() == before
    assert _graph_nodes(graphs[-1]) == 1 and _graph_nodes(graphs[0]) == 1
    for graph in (graphs[0], graphs[-1], graphs[107]):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    del graphs
