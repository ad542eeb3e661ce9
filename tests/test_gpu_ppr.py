"""APPNP personalised PageRank on the GPU (ngt_ppr_count / ngt_ppr_step)
against the oracle, bit for bit (same fp32 operations in the same order)."""
import numpy as np
import pytest
import torch

from oracle import ppr as OP

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _graph(n, E, seed, hub=False):
    rng = np.random.default_rng(seed)
    ei = rng.integers(0, n - 3, (2, E))  # the last 3 nodes stay isolated
    if hub:
        ei = np.concatenate([ei, np.stack([np.zeros(3000, np.int64), rng.integers(0, n - 3, 3000)])],
                            axis=1)
    ei = np.concatenate([ei, ei[::-1], ei[:, :40]], axis=1)  # symmetric, with duplicates
    return ei


@pytest.mark.parametrize("n,E,K,batch,iters,seed,hub", [
    (200, 800, 5, 8, 10, 0, False),     # the shipped setting: topk 5, 10 iterations
    (300, 1500, 1, 64, 4, 1, False),
    (400, 1200, 16, 1000, 6, 2, True),  # hub rows with thousands of products
    (150, 300, 64, 7, 3, 3, False),
])
def test_appnp_bit_exact(n, E, K, batch, iters, seed, hub):
    from neutrongt_amd.ppr import personal_pagerank_appnp

    ei = _graph(n, E, seed, hub)
    want_i, want_v = OP.personal_pagerank_appnp(ei, 0.85, topk=K, num_iterations=iters,
                                                num_nodes=n, iter_topk=K)
    got_i, got_v = personal_pagerank_appnp(torch.from_numpy(ei), 0.85, topk=K,
                                           num_iterations=iters, batch_size=batch, device=DEV,
                                           num_nodes=n, iter_topk=K)
    np.testing.assert_array_equal(got_i.cpu().numpy(), want_i)
    np.testing.assert_array_equal(got_v.cpu().numpy(), want_v)


def test_appnp_csr_input_source_range_and_final_topk():
    from neutrongt_amd.ppr import personal_pagerank_appnp

    n = 250
    ei = _graph(n, 1000, 5)
    rowptr, col, _, _ = OP.transition_csr(ei, n)
    want_i, want_v = OP.personal_pagerank_appnp(ei, 0.5, topk=3, num_iterations=5, num_nodes=n,
                                                iter_topk=6, source_start=40, source_end=170)
    got_i, got_v = personal_pagerank_appnp(
        None, 0.5, topk=3, num_iterations=5, batch_size=50, device=DEV,
        csr_data={"rowptr": torch.from_numpy(rowptr), "col": torch.from_numpy(col)},
        iter_topk=6, source_start=40, source_end=170)
    np.testing.assert_array_equal(got_i.cpu().numpy(), want_i)
    np.testing.assert_array_equal(got_v.cpu().numpy(), want_v)


def test_appnp_rejects_unbounded_state_and_bad_ids():
    from neutrongt_amd.ppr import personal_pagerank_appnp

    ei = torch.tensor([[0, 1], [1, 0]])
    with pytest.raises(NotImplementedError):
        personal_pagerank_appnp(ei, 0.85, topk=5, device=DEV, iter_topk=0)
    bad = {"rowptr": torch.tensor([0, 1, 2]), "col": torch.tensor([1, 7])}
    with pytest.raises(IndexError):
        personal_pagerank_appnp(None, 0.85, topk=2, device=DEV, csr_data=bad, iter_topk=2)


def test_appnp_row_chunks_match_one_pass():
    """A step split into row chunks (product budget far below the batch's)
    gives the same rows as the oracle."""
    from neutrongt_amd import ppr as PPR

    n = 300
    ei = _graph(n, 1500, 7, hub=True)
    rowptr, col, inv, _ = OP.transition_csr(ei, n)
    seeds = torch.arange(0, 120, device=DEV)
    cols, vals, cnt = PPR.appnp_batch(torch.from_numpy(rowptr).to(DEV),
                                      torch.from_numpy(col).to(DEV),
                                      torch.from_numpy(inv).to(DEV), n, seeds, 0.85, 5, 4,
                                      max_products=700)
    cols, vals, cnt = cols.cpu().numpy(), vals.cpu().numpy(), cnt.cpu().numpy()
    for r in range(120):
        want = OP.appnp_row(rowptr, col, inv, r, 0.85, 5, 4)
        assert cnt[r] == len(want)
        assert cols[r, :cnt[r]].tolist() == [c for c, _ in want]
        np.testing.assert_array_equal(vals[r, :cnt[r]], np.array([v for _, v in want], np.float32))
