"""ple_decode_out on the GPU against the PLE oracle (oracle/ple_oracle.py),
bit-exact: the decoder's arithmetic is fully IEEE-specified (FP32 product,
FP32 sum, FP16 and BF16 round-to-nearest, no contraction).  Cases follow the
reference's decoder test (tests/models/qwen4_exp/test_exl3_ple_decode.py):
three row layouts, owner shards, a NaN scale, and rows beyond one grid pass;
and more layouts: every chunk width, a long row, many heads.
"""

import numpy as np
import pytest
import torch

from oracle import ple_oracle as P
from tests.ple_cases import LAYOUTS, NAN_SCALE, synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from vllm_mi355x.kernels.exl3 import ops as exl3_ops
    exl3_ops.ensure_extension()
    return exl3_ops


def _decode(ops, device, packed, ids, bias, offsets, sizes, lo, hi, bits):
    out = torch.full((len(ids), bias.shape[1]), 123.0, dtype=torch.bfloat16, device=device)
    ops.ple_decode_out(torch.from_numpy(packed).to(device), torch.tensor(ids, dtype=torch.int64, device=device),
                       torch.from_numpy(bias).to(device), torch.tensor(offsets, dtype=torch.int64, device=device),
                       torch.tensor(sizes, dtype=torch.int64, device=device), lo, hi, bits, out)
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("bits,dim,sizes", LAYOUTS)
@pytest.mark.parametrize("owner", ["all", "lower", "upper"])
def test_ple_decode_bit_exact(ops, device, bits, dim, sizes, owner):
    print(f"ple bits={bits} dim={dim} owner={owner}", flush=True)
    packed, ids, bias, offsets, sizes, rows = synthetic(bits, dim, sizes, seed=bits)
    middle = sizes[0] + 1
    lo, hi = {"all": (0, rows), "lower": (0, middle), "upper": (middle, rows)}[owner]
    got = _decode(ops, device, packed, ids, bias, offsets, sizes, lo, hi, bits)
    assert np.array_equal(got, P.decode(packed, ids, bias, offsets, sizes, lo, hi, bits))


# every chunk count: 1-bit (16 chunks, the first 15 channels wrapping), 2-,
# 4-, 7-, 8-, 9-, 12- and 16-bit chunks, a 2560-channel row, 70 heads (one
# search round, then a direct count) with an empty head among them, and 5000
# heads (two rounds), a third of them empty
MORE_LAYOUTS = [(1, 16, (7, 5)), (2, 64, (20, 11)), (4, 256, (33,)), (7, 32, (12, 3)),
                (8, 96, (10, 10)), (9, 16, (4, 4)), (12, 4, (6,)), (16, 48, (9, 4, 6)),
                (6, 2560, (40, 9)), (5, 16, tuple([2] * 40 + [0] + [1] * 29)),
                (3, 16, tuple(([1, 2, 0] * 1700)[:5000]))]


@pytest.mark.parametrize("bits,dim,sizes", MORE_LAYOUTS)
def test_ple_decode_bit_exact_more_layouts(ops, device, bits, dim, sizes):
    print(f"ple bits={bits} dim={dim} heads={len(sizes)}", flush=True)
    packed, ids, bias, offsets, sizes, rows = synthetic(bits, dim, sizes, seed=100 + bits)
    got = _decode(ops, device, packed, ids, bias, offsets, sizes, 0, rows, bits)
    assert np.array_equal(got, P.decode(packed, ids, bias, offsets, sizes, 0, rows, bits))


@pytest.mark.parametrize("bits,dim,sizes", LAYOUTS)
def test_ple_decode_nan_scale_only_owned(ops, device, bits, dim, sizes):
    packed, ids, bias, offsets, sizes, rows = synthetic(bits, dim, sizes, seed=3)
    packed[:, 0] = NAN_SCALE
    got = _decode(ops, device, packed, ids, bias, offsets, sizes, 0, sizes[0], bits)
    owned = np.array([0 <= i < sizes[0] for i in ids])
    assert ((got[owned] & 0x7FFF) > 0x7F80).all()
    assert (got[~owned] == 0).all()


def test_ple_decode_rows_beyond_one_grid_pass(ops, device):
    packed, ids, bias, offsets, sizes, rows = synthetic(5, 16, (3, 3), seed=11)
    repeat = 70000 // len(ids) + 1
    packed, ids = np.tile(packed, (repeat, 1)), ids * repeat
    got = _decode(ops, device, packed, ids, bias, offsets, sizes, 0, rows, 5)
    assert np.array_equal(got, P.decode(packed, ids, bias, offsets, sizes, 0, rows, 5))


def test_ple_decode_rejects_bad_geometry(ops, device):
    packed, ids, bias, offsets, sizes, rows = synthetic(6, 160, (97, 40, 13), seed=1)
    with pytest.raises(RuntimeError, match="bits must be"):
        _decode(ops, device, packed, ids, bias, offsets, sizes, 0, rows, 17)
    with pytest.raises(RuntimeError, match="packed_rows must be"):
        _decode(ops, device, packed, ids, bias, offsets, sizes, 0, rows, 5)
    with pytest.raises(RuntimeError, match="owner range"):
        _decode(ops, device, packed, ids, bias, offsets, sizes, 5, 2, 6)
