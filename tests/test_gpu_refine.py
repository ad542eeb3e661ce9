"""Window refinement on the GPU (node_out / node_in) against the oracle, bit
for bit: windows, their edge lists, the expired-node buffer and counts."""
import numpy as np
import pytest
import torch

from oracle import graph as OG
from oracle import refine as OR

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _t(a, dtype=torch.int64):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def _setup(seed, n=600, n_win=4, win=120, E=6000, P=8000):
    rng = np.random.default_rng(seed)
    ei = rng.integers(0, n, (2, E))
    ppr = rng.integers(0, n, (2, P))
    # PPR values with repeats so that candidate scores tie now and then
    val = (rng.integers(1, 20, P) / 1000.0).astype(np.float32)
    perm = rng.permutation(n)
    parts = [np.sort(perm[i * win:(i + 1) * win]) for i in range(n_win)]
    subs = [OG.subgraph_coo(p, ei, n) for p in parts]
    return rng, ei, ppr, val, parts, subs


@pytest.mark.parametrize("seed,ratio", [(0, 0.3), (1, 0.1), (2, 0.5)])
def test_refinement_round_matches_oracle(seed, ratio):
    from neutrongt_amd.refine import WindowRefiner

    rng, ei, ppr, val, parts, subs = _setup(seed)
    # node scores with ties (rounded)
    scores = [np.round(rng.random(p.size), 2).astype(np.float32) for p in parts]
    ref = OR.Refiner(parts, subs, ei, 600, ppr, val)
    gpu = WindowRefiner([_t(p) for p in parts], [_t(s) for s in subs], _t(ei), 600, _t(ppr),
                        _t(val, torch.float32))
    for rnd in range(2):
        ref.node_out(scores, remove_ratio=ratio)
        gpu.node_out([_t(s, torch.float32) for s in scores], remove_ratio=ratio)
        ref.node_in()
        gpu.node_in()
        for i in range(len(parts)):
            np.testing.assert_array_equal(gpu.partitioned_results[i].cpu().numpy(),
                                          ref.partitions[i])
            np.testing.assert_array_equal(
                gpu.sub_edge_index_for_partition_results[i].cpu().numpy(), ref.sub_edges[i])
        np.testing.assert_array_equal(np.sort(gpu.global_expired_node_buffer.cpu().numpy()),
                                      np.sort(ref.buffer))
        assert gpu.partition_expired_node_num == ref.expired_num
        scores = [np.round(rng.random(p.size), 2).astype(np.float32) for p in ref.partitions]


def test_node_in_scores_equal_sequential_fp32_sums():
    from neutrongt_amd.refine import _segment_sum

    rng = np.random.default_rng(4)
    lens = rng.integers(0, 300, 200)
    lens[5] = 20000  # a long segment
    vals = (rng.random(int(lens.sum())) * 1e-3).astype(np.float32)
    seg = np.concatenate([[0], np.cumsum(lens)])
    got = _segment_sum(_t(vals, torch.float32), _t(seg)).cpu().numpy()
    want = np.zeros(lens.size, np.float32)
    np.add.at(want, np.repeat(np.arange(lens.size), lens), vals)
    np.testing.assert_array_equal(got, want)


def test_node_out_rejects_mismatched_scores():
    from neutrongt_amd.refine import node_out_window

    with pytest.raises(ValueError):
        node_out_window(_t(np.arange(5)), _t(np.zeros((2, 0), np.int64)),
                        torch.ones(4, device=DEV), 0.3)


def test_node_in_rejects_out_of_range_ids():
    from neutrongt_amd.refine import node_in_window

    nodes, buf = _t(np.array([0, 1])), _t(np.array([2, 3]))
    ppr = _t(np.array([[0, 1], [2, 9]]))
    with pytest.raises(IndexError):
        node_in_window(nodes, buf, ppr, torch.ones(2, device=DEV), 1, _t(np.zeros((2, 0))), 5)
