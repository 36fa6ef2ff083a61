"""exl3_linear_out_scratch, the entry point that allocates nothing (its
scratch is a static device array of the library), through the C-ABI:
bitwise equal to exl3_linear_out (the same kernels and sums) on two calls in
a row, the second with a smaller input, at small-M and large-M sizes; a call
beyond the scratch is rejected with an error."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as O
from tests.exl3_cases import random_acts, random_matrix

pytestmark = pytest.mark.gpu


def _call_scratch(lib, x, trellis, suh, svh, bits_x2, n, out):
    return lib.exl3_linear_out_scratch(
        x.data_ptr(), 1, x.size(0), x.size(1), trellis.data_ptr(), *trellis.shape,
        suh.data_ptr(), suh.numel(), svh.data_ptr(), svh.numel(), bits_x2, 2, x.size(1), n,
        out.data_ptr(), 2, out.size(0), out.size(1), torch.cuda.current_stream().cuda_stream)


def _call_workspace(lib, x, trellis, suh, svh, bits_x2, n, out):
    ws = torch.empty(lib.exl3_linear_workspace_size(x.size(0), suh.numel(), svh.numel()),
                     dtype=torch.float32, device=x.device)
    return lib.exl3_linear_out(
        x.data_ptr(), 1, x.size(0), x.size(1), trellis.data_ptr(), *trellis.shape,
        suh.data_ptr(), suh.numel(), svh.data_ptr(), svh.numel(), bits_x2, 2, x.size(1), n,
        out.data_ptr(), 2, out.size(0), out.size(1), ws.data_ptr(), ws.numel(),
        torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("k,n,rows", [(4096, 14336, (8, 1)), (2048, 1024, (200, 40)), (1024, 512, (33, 3))])
def test_scratch_entry_matches_workspace_entry(device, k, n, rows):
    from vllm_mi355x import _native
    lib = _native.load()
    print(f"scratch entry {k}x{n} rows={rows}", flush=True)
    rng = np.random.default_rng(k + n)
    trellis, suh, svh = random_matrix(rng, k, n, 8)
    t = torch.from_numpy(trellis).to(device)
    u = torch.from_numpy(suh).to(device)
    v = torch.from_numpy(svh).to(device)
    for r in rows:  # two calls in a row, the second smaller
        x, _ = random_acts(rng, r, k, "fp16")
        xt = torch.from_numpy(x).to(device)
        got = torch.full((r, n), float("nan"), dtype=torch.float32, device=device)
        want = torch.empty(r, n, dtype=torch.float32, device=device)
        _native.check(_call_scratch(lib, xt, t, u, v, 8, n, got))
        _native.check(_call_workspace(lib, xt, t, u, v, 8, n, want))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"rows={r}"
        if r <= 8 and k * n <= 4096 * 14336:
            ref = O.linear_out(x[:1], 1, trellis, suh, svh, 8, 2, n, O.FP32)
            err = np.abs(got[:1].cpu().numpy().astype(np.float64) - ref)
            rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
            assert (err <= 2.0 ** -14 * rms + 2.0 ** -16 * np.abs(ref)).all()


def test_scratch_entry_rejects_rows_beyond_the_scratch(device):
    from vllm_mi355x import _native
    lib = _native.load()
    k, n = 8192, 256
    limit = lib.exl3_linear_scratch_rows(k, n)
    assert limit == (4 << 20) // (k + 1)
    rng = np.random.default_rng(1)
    trellis, suh, svh = random_matrix(rng, k, n, 8)
    t = torch.from_numpy(trellis).to(device)
    u = torch.from_numpy(suh).to(device)
    v = torch.from_numpy(svh).to(device)
    x = torch.zeros(limit + 1, k, dtype=torch.float16, device=device)
    out = torch.empty(limit + 1, n, dtype=torch.float32, device=device)
    assert _call_scratch(lib, x, t, u, v, 8, n, out) == 1
    assert b"static scratch" in lib.vllm_mi355x_last_error()
