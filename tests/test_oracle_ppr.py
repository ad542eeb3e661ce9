"""Pins the APPNP personalised-PageRank oracle on the CPU."""
import numpy as np
import pytest
import torch

from oracle import ppr as OP


def _sym(ei):
    return np.concatenate([ei, ei[::-1]], axis=1)


def test_hand_derived_path_graph():
    # path 0 - 1 - 2, seed 0, alpha 0.85, K = 2
    ei = _sym(np.array([[0, 1], [1, 2]]))
    rowptr, col, inv, n = OP.transition_csr(ei)
    one = OP.appnp_row(rowptr, col, inv, 0, 0.85, 2, 1)
    assert [c for c, _ in one] == [0, 1]
    assert np.isclose(one[0][1], 0.85) and np.isclose(one[1][1], 0.15)
    two = OP.appnp_row(rowptr, col, inv, 0, 0.85, 2, 2)
    # node 1: 0.15 * (0.85 * 1) = 0.1275; node 0: 0.15 * (0.15 * 0.5) + 0.85 = 0.86125;
    # node 2: 0.15 * (0.15 * 0.5) = 0.01125 ranks third and is truncated by K = 2
    assert [c for c, _ in two] == [0, 1]
    assert np.isclose(two[0][1], 0.86125) and np.isclose(two[1][1], 0.1275)


@pytest.mark.parametrize("seed,K", [(0, 3), (1, 5), (2, 8)])
def test_matches_dense_fp64_recursion(seed, K):
    rng = np.random.default_rng(seed)
    n = 60
    ei = rng.integers(0, n, (2, 240))
    ei = np.concatenate([ei, [[5, 5, 7], [6, 6, 7]]], axis=1)  # duplicates, a self loop
    seeds = np.arange(0, n, 3)
    idx, val = OP.personal_pagerank_appnp(ei, 0.85, topk=K, num_iterations=6, num_nodes=n)
    S = OP.appnp_dense_fp64(ei, n, 0.85, K, 6, seeds)
    for r, s in enumerate(seeds):
        got = {int(c): float(v) for c, v in zip(idx[1][idx[0] == s], val[idx[0] == s])}
        want = {int(c): S[r, c] for c in np.flatnonzero(S[r])}
        kth = sorted(want.values(), reverse=True)[min(K, len(want)) - 1]
        for c in set(got) | set(want):
            if c in got and c in want:
                assert abs(got[c] - want[c]) <= 1e-5 * max(abs(want[c]), 1e-3), (s, c)
            else:  # only a near-tie at the truncation boundary may differ
                v = got.get(c, want.get(c))
                assert abs(v - kth) <= 1e-5, (s, c, v, kth)


def test_rank_matches_torch_topk_without_ties():
    rng = np.random.default_rng(4)
    vals = rng.permutation(200).astype(np.float32) / 3.0
    ids = rng.permutation(1000)[:200]
    got = OP.rank(list(zip(ids.tolist(), vals.tolist())), 7)
    tv, ti = torch.topk(torch.from_numpy(vals), 7, largest=True, sorted=True)
    assert [c for c, _ in got] == ids[ti.numpy()].tolist()
    assert [v for _, v in got] == tv.tolist()


def test_isolated_seed_keeps_its_teleport_mass():
    ei = _sym(np.array([[1], [2]]))
    idx, val = OP.personal_pagerank_appnp(ei, 0.85, topk=3, num_iterations=4, num_nodes=4)
    # node 0 and node 3 have no edges: their row is the teleport term alone
    for s in (0, 3):
        assert idx[1][idx[0] == s].tolist() == [s]
        assert val[idx[0] == s].tolist() == [np.float32(0.85)]
