"""Induced window subgraphs on the GPU (ngt_subgraph_coo / ngt_subgraph_csr)
against the oracle restatements, bit for bit."""
import numpy as np
import pytest
import torch

from oracle import graph as OG

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _csr_of(ei, n):
    order = np.argsort(ei[0], kind="stable")
    rowptr = np.zeros(n + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(ei[0], minlength=n))
    return rowptr, ei[1][order]


def _gpu(*arrays):
    return [torch.from_numpy(np.ascontiguousarray(a, dtype=np.int64)).to(DEV) for a in arrays]


def _graph(n, E, seed, hub=0):
    rng = np.random.default_rng(seed)
    ei = rng.integers(0, n, (2, E))
    if hub:  # one hub row and one hub column, plus duplicated edges
        ei = np.concatenate([ei, np.stack([np.zeros(hub, np.int64), rng.integers(0, n, hub)]),
                             np.stack([rng.integers(0, n, hub), np.full(hub, 1)]), ei[:, :50]],
                            axis=1)
    return ei


@pytest.mark.parametrize("n,E,n_set,seed,hub", [(500, 5000, 120, 0, 0), (300, 20000, 200, 1, 5000),
                                                (64, 300, 64, 2, 0), (1000, 9000, 7, 3, 0)])
def test_subgraph_coo_bit_exact(n, E, n_set, seed, hub):
    from neutrongt_amd.window import subgraph

    ei = _graph(n, E, seed, hub)
    subset = np.random.default_rng(seed + 100).permutation(n)[:n_set]
    if hub:
        subset = np.concatenate([[0, 1], subset[~np.isin(subset, [0, 1])]])
    want = OG.subgraph_coo(subset, ei, n)
    s_d, ei_d = _gpu(subset, ei)
    got = subgraph(s_d, ei_d, n)
    assert got.dtype == torch.int64 and got.shape == want.shape
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("n,E,n_set,seed,hub", [(500, 5000, 120, 0, 0), (300, 20000, 200, 1, 5000),
                                                (64, 300, 64, 2, 0), (1000, 9000, 7, 3, 0)])
def test_subgraph_from_csr_bit_exact(n, E, n_set, seed, hub):
    from neutrongt_amd.window import subgraph_from_csr

    ei = _graph(n, E, seed, hub)
    rowptr, col = _csr_of(ei, n)
    node_set = np.random.default_rng(seed + 200).permutation(n)[:n_set]
    if hub:
        node_set = np.concatenate([[0, 1], node_set[~np.isin(node_set, [0, 1])]])
    want = OG.subgraph_from_csr(node_set, rowptr, col)
    got = subgraph_from_csr(*_gpu(node_set, rowptr, col))
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_subgraph_empty_and_disjoint_cases():
    from neutrongt_amd.window import subgraph, subgraph_from_csr

    ei = np.array([[0, 1, 2], [1, 2, 0]])
    rowptr, col = _csr_of(ei, 5)
    for subset in (np.zeros(0, np.int64), np.array([3, 4])):
        assert subgraph(*_gpu(subset, ei), 5).shape == (2, 0)
        assert subgraph_from_csr(*_gpu(subset, rowptr, col)).shape == (2, 0)
    no_edges = np.zeros((2, 0), np.int64)
    assert subgraph(*_gpu(np.array([1, 0]), no_edges), 5).shape == (2, 0)


def test_subgraph_rejects_bad_input():
    from neutrongt_amd.window import subgraph, subgraph_from_csr

    ei = np.array([[0, 1, 2], [1, 2, 0]])
    rowptr, col = _csr_of(ei, 3)
    with pytest.raises(IndexError, match="duplicate"):
        subgraph(*_gpu(np.array([0, 1, 0]), ei), 3)
    with pytest.raises(IndexError, match="out of range"):
        subgraph(*_gpu(np.array([0, 7]), ei), 3)
    with pytest.raises(IndexError, match="endpoint"):
        subgraph(*_gpu(np.array([0, 1]), np.array([[0, 5], [1, 0]])), 3)
    with pytest.raises(IndexError, match="duplicate"):
        subgraph_from_csr(*_gpu(np.array([2, 2]), rowptr, col))
    bad_rowptr = np.array([0, 1, 9, 3])  # row 1 runs past col
    with pytest.raises(IndexError, match="CSR row"):
        subgraph_from_csr(*_gpu(np.array([1, 0]), bad_rowptr, col))
    with pytest.raises(IndexError, match="CSR row"):  # row 1 ends before it starts
        subgraph_from_csr(*_gpu(np.array([1, 0]), np.array([0, 2, 1, 3]), col))


def test_subgraphs_from_csr_in_flight_match_one_at_a_time():
    """Several windows' CSR-walk subgraphs with 1, 2 or 4 in flight (a stream
    each): the oracle's edges for every window, an empty window among them; a
    repeated node in a later window still raises."""
    from neutrongt_amd.window import subgraphs_from_csr

    n = 800
    ei = _graph(n, 12000, 7, hub=2000)
    rowptr, col = _csr_of(ei, n)
    rng = np.random.default_rng(77)
    sets = [rng.permutation(n)[:k] for k in (150, 0, 400, 37, 800, 260)]
    want = [OG.subgraph_from_csr(s, rowptr, col) for s in sets]
    rp_d, col_d = _gpu(rowptr, col)
    sets_d = _gpu(*sets)
    for streams in (1, 2, 4):
        for got, w in zip(subgraphs_from_csr(sets_d, rp_d, col_d, streams=streams), want):
            np.testing.assert_array_equal(got.cpu().numpy(), w)
    with pytest.raises(IndexError, match="duplicate"):
        subgraphs_from_csr(sets_d[:3] + _gpu(np.array([5, 9, 5])), rp_d, col_d, streams=2)


def test_subgraph_full_size_window():
    """A 32,768-node window of a 2,000,000-node, 24M-edge graph (both forms)."""
    from neutrongt_amd.window import subgraph, subgraph_from_csr

    n, E = 2_000_000, 24_000_000
    rng = np.random.default_rng(7)
    ei = rng.integers(0, n, (2, E))
    window = rng.choice(n, 32768, replace=False)
    # densify the window so it has a realistic number of internal edges
    inner = rng.integers(0, window.size, (2, 1_500_000))
    ei = np.concatenate([ei, window[inner]], axis=1)
    got = subgraph(*_gpu(window, ei), n).cpu().numpy()
    np.testing.assert_array_equal(got, OG.subgraph_coo(window, ei, n))
    rowptr, col = _csr_of(ei, n)
    got = subgraph_from_csr(*_gpu(window, rowptr, col)).cpu().numpy()
    # vectorised statement of the CSR form: edges grouped by set position in set
    # order, CSR order inside a row
    pos = np.full(n, -1, np.int64)
    pos[window] = np.arange(window.size)
    deg = rowptr[window + 1] - rowptr[window]
    row_of = np.repeat(np.arange(window.size), deg)
    starts = np.repeat(rowptr[window] - np.concatenate([[0], np.cumsum(deg)[:-1]]), deg)
    nb = col[np.arange(deg.sum()) + starts]
    keep = pos[nb] >= 0
    np.testing.assert_array_equal(got, np.stack([row_of[keep], pos[nb[keep]]]))
