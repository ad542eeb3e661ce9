"""Pins the window-refinement oracle (node_out / node_in) on the CPU."""
import numpy as np
import torch

from oracle import refine as OR


def test_node_out_hand_derived():
    # scores 0.9 tie at positions 1 and 3 (lower position first), keep int(5*0.6) = 3
    nodes = np.array([10, 11, 12, 13, 14])
    edges = np.array([[0, 1, 2, 3, 4, 1], [1, 3, 0, 4, 3, 0]])
    kept, kept_edges, expired = OR.node_out_window(nodes, edges, [0.5, 0.9, 0.1, 0.9, 0.3], 0.4)
    assert kept.tolist() == [10, 11, 13] and expired.tolist() == [12, 14]
    assert kept_edges.tolist() == [[0, 1, 1], [1, 2, 0]]
    # at least one node stays
    kept, _, expired = OR.node_out_window(np.array([3]), np.zeros((2, 0), np.int64), [1.0], 0.9)
    assert kept.tolist() == [3] and expired.size == 0


def test_node_out_ranking_matches_torch_argsort_without_ties():
    rng = np.random.default_rng(0)
    scores = rng.permutation(1000).astype(np.float32) / 7.0  # distinct
    nodes = np.arange(1000) * 3
    kept, _, expired = OR.node_out_window(nodes, np.zeros((2, 0), np.int64), scores, 0.3)
    order = torch.argsort(torch.from_numpy(scores), descending=True).numpy()
    assert kept.tolist() == sorted(nodes[order[:700]].tolist())
    assert expired.tolist() == sorted(nodes[order[700:]].tolist())


def test_node_in_hand_derived():
    nodes = np.array([0, 1, 2])
    buffer = np.array([5, 7, 5, 9, 1])
    ppr = np.array([[0, 1, 2, 3, 1], [5, 7, 5, 9, 9]])
    val = np.array([0.1, 0.25, 0.2, 0.9, 0.05], np.float32)
    edges = np.array([[0, 5, 7, 2, 9], [5, 0, 2, 7, 1]])
    new, new_edges, rest = OR.node_in_window(nodes, buffer, ppr, val, 2, edges, 10)
    # candidates outside the window: 5 (0.1 + 0.2), 7 (0.25), 9 (0.05; 3 -> 9 starts outside)
    assert new.tolist() == [0, 1, 2, 5, 7]
    assert rest.tolist() == [1, 5, 9]
    # global edges with both ends in {0,1,2,5,7}: (0,5) (5,0) (7,2) (2,7) -> positions
    assert new_edges.tolist() == [[0, 3, 4, 2], [3, 0, 2, 4]]
    assert OR.node_in_window(nodes, np.array([1, 2]), ppr, val, 2, edges, 10) is None


def test_node_in_scores_are_the_reference_index_add():
    """fp32 candidate scores: np.add.at in edge order == torch CPU index_add_."""
    rng = np.random.default_rng(3)
    idx = rng.integers(0, 50, 5000)
    vals = (rng.random(5000) * 1e-2).astype(np.float32)
    a = np.zeros(50, np.float32)
    np.add.at(a, idx, vals)
    b = torch.zeros(50).index_add_(0, torch.from_numpy(idx), torch.from_numpy(vals))
    np.testing.assert_array_equal(a, b.numpy())


def test_refiner_loop_semantics():
    ei = np.array([[0, 1, 1, 2, 3, 4, 5, 6], [1, 0, 2, 1, 4, 3, 6, 5]])
    ppr = np.array([[0, 3, 3, 5], [2, 2, 6, 2]])
    val = np.array([0.5, 0.2, 0.3, 0.1], np.float32)
    parts = [np.array([0, 1, 2]), np.array([3, 4, 5, 6])]
    subs = [OR.subgraph_coo(p, ei, 7) for p in parts]
    r = OR.Refiner(parts, subs, ei, 7, ppr, val)
    r.node_out([np.array([0.3, 0.2, 0.1], np.float32), np.array([0.4, 0.3, 0.2, 0.1], np.float32)],
               remove_ratio=0.5)
    assert [p.tolist() for p in r.partitions] == [[0], [3, 4]]
    assert sorted(r.buffer.tolist()) == [1, 2, 5, 6] and r.expired_num == {0: 2, 1: 2}
    r.node_in()
    # window 0 takes its two best-scored buffered nodes: 2 (0.5 from node 0), then 1 (1, 5
    # and 6 tie at 0; the lowest id wins)
    assert r.partitions[0].tolist() == [0, 1, 2]
    assert r.expired_num[0] == 0
    # window 1: candidates 5, 6 (scores 0 / 0.3 from node 3) -> both
    assert r.partitions[1].tolist() == [3, 4, 5, 6] and r.buffer.size == 0
    # a second node_in returns at window 0 (nothing to recover) and leaves window 1 alone
    r.expired_num[1] = 3
    r.node_in()
    assert r.expired_num == {0: 0, 1: 3}
