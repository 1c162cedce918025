"""Pins the integer planner oracle: the reference's golden vectors plus
brute-force counting on small random inputs (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import plan as P

pytestmark = pytest.mark.cpu


@pytest.mark.parametrize(
    "groups,expected",
    [
        # tests/test_capacity_dropping.py L:42-80
        ([2, 0, 2, 1, 0, 2], [0, 0, 1, 0, 1, 2]),
        ([5, 5, 5, 5], [0, 1, 2, 3]),
        ([0, 1, 2, 3], [0, 0, 0, 0]),
        ([7], [0]),
        ([3, 1, 3, 1, 3, 0], [0, 0, 1, 1, 2, 0]),
        ([], []),
    ],
)
def test_cumcount_golden(groups, expected):
    assert P.cumcount(np.array(groups, dtype=np.int64)).tolist() == expected


def _brute_cumcount(g):
    return [sum(1 for j in range(i) if g[j] == g[i]) for i in range(len(g))]


@pytest.mark.parametrize("seed", range(5))
def test_cumcount_brute_force(seed):
    rng = np.random.default_rng(seed)
    g = rng.integers(0, 1 + seed * 3, size=200)
    assert P.cumcount(g).tolist() == _brute_cumcount(g.tolist())


def test_drop_mask_golden():
    # tests/test_capacity_dropping.py L:116-152
    assert P.drop_mask(np.array([[0], [0], [0], [1], [1]]), 2).tolist() == [[False], [False], [True], [False], [False]]
    assert not P.drop_mask(np.array([[0], [1], [0], [1]]), 100).any()
    assert P.drop_mask(np.array([[0], [1], [0], [1]]), 0).all()
    assert P.drop_mask(np.array([[0, 1], [0, 1]]), 1).tolist() == [[False, False], [True, True]]
    assert not P.drop_mask(np.array([[0]]), 1).any()


@pytest.mark.parametrize("seed", range(4))
def test_drop_mask_brute_force(seed):
    rng = np.random.default_rng(100 + seed)
    N, K, E = 120, 3, 5
    idx = rng.integers(0, E, size=(N, K))
    cap = int(rng.integers(0, 40))
    want = np.array([[c >= cap for c in _brute_cumcount(idx[:, k].tolist())] for k in range(K)]).T
    assert (P.drop_mask(idx, cap) == want).all()


@pytest.mark.parametrize("N,K,E", [(10, 2, 4), (7, 3, 4), (3, 2, 8), (16, 1, 5)])
def test_plan_reference_brute_force(N, K, E):
    rng = np.random.default_rng(N * 100 + K * 10 + E)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(N)])
    pl = P.plan_reference(idx, E)
    # stable sort on column 0, built by insertion
    order = sorted(range(N), key=lambda t: (idx[t, 0], t))
    assert pl["sort_order"].tolist() == order
    R = N * K
    chunk = max(1, R // E)
    for r in range(R):
        t = order[r // K]
        assert pl["row_slot"][r] == t * K + r % K
        assert pl["slot_row"][t * K + r % K] == r
    rex = P.row_expert(pl["offsets"], R)
    for r in range(R):
        e = r // chunk
        assert rex[r] == (e if e < E else -1)


@pytest.mark.parametrize("seed", range(3))
def test_plan_routed_brute_force(seed):
    rng = np.random.default_rng(7 + seed)
    N, K, E = 30, 3, 6
    idx = np.stack([rng.permutation(E)[:K] for _ in range(N)])
    drop = P.drop_mask(idx, 5)
    pl = P.plan_routed(idx, E, drop)
    rows = []
    for e in range(E):
        for s in range(N * K):
            if idx.reshape(-1)[s] == e and not drop.reshape(-1)[s]:
                rows.append(s)
        assert pl["offsets"][e + 1] == len(rows)
    assert pl["row_slot"].tolist() == rows
    for s in range(N * K):
        if drop.reshape(-1)[s]:
            assert pl["slot_row"][s] == -1
        else:
            assert rows[pl["slot_row"][s]] == s
