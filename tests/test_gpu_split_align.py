"""Split-cover MoE alignment on the GPU (moe_split_align) and the Marlin MoE
over its block lists (fused_marlin_moe(path="split"), the reference's
prefill.run, vllm_sm80/kernels/marlin_moe/prefill.py:381-447).

The device lists equal the CPU layout model (oracle/split_align_oracle.py)
entry for entry; the split path matches the oracle's MoE on sampled tokens,
the single-list staged path to the MoE bar (lists of other block sizes sum
w13 in another order), and itself bitwise from run to run."""

import numpy as np
import pytest
import torch

from oracle import marlin_oracle as M
from oracle import split_align_oracle as SO
from tests.test_gpu_marlin_moe import Layer, assert_close, dev, dev_act, from_f32, host_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sa():
    from vllm_mi355x.kernels.marlin_moe import extension, split_align
    extension.require_extension()
    return split_align


def _skewed_ids(rng, T, E, topk, invalid=0):
    pop = rng.gamma(4.0, size=E)
    z = np.log(pop)[None, :] - np.log(-np.log(rng.uniform(1e-12, 1 - 1e-7, (T, E))))
    ids = np.argsort(-z, axis=1)[:, :topk].astype(np.int32)
    if invalid:
        flat = ids.reshape(-1)
        flat[rng.choice(flat.size, invalid, replace=False)] = -1
    return ids


@pytest.mark.parametrize("T,E,topk,invalid,mapped", [
    (1, 128, 8, 0, False), (5, 288, 8, 3, False), (100, 128, 8, 0, True),
    (2304, 288, 8, 17, False), (1282, 288, 8, 0, True), (64, 16, 4, 0, False)])
def test_device_lists_equal_the_model(sa, device, T, E, topk, invalid, mapped):
    print(f"split_align T={T} E={E} topk={topk} invalid={invalid} mapped={mapped}", flush=True)
    rng = np.random.default_rng(T + E)
    ids = _skewed_ids(rng, T, E, topk, invalid)
    emap = None
    if mapped:
        emap = np.arange(E, dtype=np.int32)
        emap[rng.choice(E, E // 8, replace=False)] = -1
    buf = sa.buffers(T * topk, E, device)
    lists = sa.split_align(dev(ids, device), E, buf,
                           expert_map=None if emap is None else dev(emap, device))
    torch.cuda.synchronize()
    model = SO.split_layout(ids.reshape(-1).tolist(), E, buf["tab"].cpu().numpy(), emap)
    for bs, sorted_ids, expert_ids, ntpp in lists:
        want_sorted, want_eids = model[bs]
        n = int(ntpp.item())
        assert n == len(want_sorted), f"bs={bs}: ntpp"
        assert sorted_ids[:n].cpu().numpy().tolist() == want_sorted, f"bs={bs}: sorted ids"
        eids = expert_ids.cpu().numpy()
        assert eids[:n // bs].tolist() == want_eids, f"bs={bs}: expert ids"
        assert (eids[n // bs:] == -1).all(), f"bs={bs}: blocks past the list"


def test_split_path_matches_oracle_and_staged(device):
    from vllm_mi355x.kernels.marlin_moe import extension, fused
    extension.require_extension()
    print("marlin split path E=64 512/256 top-8 T=300", flush=True)
    rng = np.random.default_rng(300)
    E, K, N, topk, T = 64, 512, 256, 8, 300
    layer = Layer(rng, E, K, N, M.BF16, device)
    ids = _skewed_ids(rng, T, E, topk)
    w = rng.random((T, topk)).astype(np.float32)
    x = from_f32(rng.standard_normal((T, K)), M.BF16)
    args = (dev_act(x, M.BF16, device), layer.w1, layer.w2, layer.s1, layer.s2, dev(w, device),
            dev(ids, device))
    ws = {}
    split = host_bits(fused.fused_marlin_moe(*args, path="split", ksplit=1, workspace=ws))
    again = host_bits(fused.fused_marlin_moe(*args, path="split", ksplit=1, workspace=ws))
    staged = host_bits(fused.fused_marlin_moe(*args, path="staged", block_size=64, ksplit=1))
    assert np.array_equal(split, again)
    assert_close(split, staged, M.BF16, "split vs staged")
    sample = [0, 1, 150, 299]
    expected = M.moe(x[sample], M.BF16, ids[sample], w[sample], *layer.host)
    assert_close(split[sample], expected, M.BF16, "split vs oracle")
