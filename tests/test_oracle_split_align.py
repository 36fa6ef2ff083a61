"""The split-cover alignment's host half and its model, on the CPU.

cover_table (the product's DP, vllm_mi355x/kernels/marlin_moe/split_align.py)
against exhaustive enumeration of covers; the layout model of
oracle/split_align_oracle.py against the contract's invariants
(vllm_sm80/kernels/marlin_moe/split_align.py:1-31)."""

import numpy as np
import pytest

from oracle import split_align_oracle as SO
from vllm_mi355x.kernels.marlin_moe import split_align as SA


def test_brute_cover_known_values():
    # one 16-row block; a 32 beats two 16s; a 64 beats 48 + 16
    assert SO.brute_cover_cost(1) == pytest.approx(14.1)
    assert SO.brute_cover_cost(17) == pytest.approx(20.3)
    assert SO.brute_cover_cost(64) == pytest.approx(33.3)
    assert SO.brute_cover_cost(65) == pytest.approx(min(33.3 + 14.1, 26.4 + 20.3))
    assert SO.brute_cover_cost(0) == 0.0


def test_sizes_and_costs_match_the_model():
    assert SA.SIZES == SO.SIZES and SA.COST == SO.COST


def test_cover_table_is_cost_optimal():
    tab = SA.cover_table(260).numpy()
    assert tab.shape == (261, 4) and tab.dtype == np.int32
    assert (tab[0] == 0).all()
    for r in range(1, 261):
        counts = tab[r]
        rows = sum(int(c) * s for c, s in zip(counts, SA.SIZES))
        cost = sum(int(c) * SA.COST[s] for c, s in zip(counts, SA.SIZES))
        assert rows >= r, r
        assert cost == pytest.approx(SO.brute_cover_cost(r), abs=1e-6), r
        # a cost-optimal cover pads less than its smallest block: every block
        # keeps a routed row
        smallest = min(s for c, s in zip(counts, SA.SIZES) if c)
        assert rows - r < smallest, r


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_layout_model_invariants(seed):
    rng = np.random.default_rng(seed)
    n_exp, T = 40, 3000
    p = rng.gamma(0.5, size=n_exp)
    ids = rng.choice(n_exp, size=T, p=p / p.sum()).astype(np.int64)
    ids[rng.choice(T, 50, replace=False)] = -1
    ids[rng.choice(T, 10, replace=False)] = n_exp + 3
    emap = np.arange(n_exp)
    emap[[3, 7]] = -1
    tab = SA.cover_table(T).numpy()
    out = SO.split_layout(ids.tolist(), n_exp, tab, emap)
    routed = [i for i, e in enumerate(ids) if 0 <= e < n_exp and emap[e] >= 0]
    seen = []
    for bs, (sorted_ids, eids) in out.items():
        assert len(sorted_ids) == bs * len(eids)
        for b, e in enumerate(eids):
            block = sorted_ids[b * bs:(b + 1) * bs]
            real = [i for i in block if i != T]
            assert real, "every block holds a routed row"
            assert all(emap[ids[i]] == e for i in real)
            # padding only at the end of a block
            assert block[:len(real)] == real
        seen += [i for i in sorted_ids if i != T]
    assert sorted(seen) == routed
    # within an expert, rows run in flat order from the largest list down
    for e in range(n_exp):
        rows = []
        for bs in SA.SIZES:
            sorted_ids, eids = out[bs]
            for b, owner in enumerate(eids):
                if owner == e:
                    rows += [i for i in sorted_ids[b * bs:(b + 1) * bs] if i != T]
        assert rows == sorted(rows)
