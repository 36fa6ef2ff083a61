"""CPU restatement of the split-cover MoE alignment (the reference's layout
contract: vllm_sm80/kernels/marlin_moe/split_align.py:1-31 and 173-188, and
the pure-Python model and brute-force cover of
tests/kernels/test_ampere_pp_marlin_prefill.py:55-82).

TEST INFRASTRUCTURE ONLY.  Only tests/ may import this module, as the
checker; the product path (vllm-cmp170hx_amd/) never does.

Pinned by: the cover cost of every r against exhaustive enumeration
(brute_cover_cost, which tries every multiset of 64/48/32-row blocks and
fills the rest with 16s), and the layout model against its invariants (every
routed row exactly once, in stable flat order within its expert; only an
expert's last block padded; every block holds a routed row) in
tests/test_oracle_split_align.py.
"""

from __future__ import annotations

SIZES = (64, 48, 32, 16)
COST = {64: 33.3, 48: 26.4, 32: 20.3, 16: 14.1}


def brute_cover_cost(r: int, sizes=SIZES, cost=COST) -> float:
    """Cheapest total cost of blocks covering r rows, by enumeration."""
    if r <= 0:
        return 0.0
    big = sizes[:-1]
    small = sizes[-1]
    best = None

    def rec(i, rest, acc):
        nonlocal best
        if i == len(big):
            n = max(0, -(-rest // small))
            c = acc + n * cost[small]
            if best is None or c < best - 1e-9:
                best = c
            return
        s = big[i]
        for n in range(0, max(rest, 0) // s + 2):
            rec(i + 1, rest - n * s, acc + n * cost[s])

    rec(0, r, 0.0)
    return best


def split_layout(ids, n_exp: int, table, expert_map=None):
    """{bs: (sorted ids, expert ids)} for flattened ids: expert e's routed
    rows (ascending flat index) fill table[r_e][k] blocks of size SIZES[k],
    largest first; the padding (sentinel len(ids)) ends the expert's last
    block.  Experts follow one another in every list."""
    T = len(ids)
    rows = [[] for _ in range(n_exp)]
    for i, e in enumerate(ids):
        e = int(e)
        if not (0 <= e < n_exp):
            continue
        if expert_map is not None:
            e = int(expert_map[e])
            if not (0 <= e < n_exp):
                continue
        rows[e].append(i)
    out = {bs: ([], []) for bs in SIZES}
    for e in range(n_exp):
        counts = table[len(rows[e])]
        pos = 0
        for k, bs in enumerate(SIZES):
            cnt = int(counts[k]) * bs
            if cnt == 0:
                continue
            got = rows[e][pos:pos + cnt]
            pos += cnt
            out[bs][0].extend(got + [T] * (cnt - len(got)))
            out[bs][1].extend([e] * (cnt // bs))
    return out
