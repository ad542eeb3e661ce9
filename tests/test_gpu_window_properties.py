"""Property tests of the window preparation on the GPU (hypothesis,
derandomized): random power-law global graphs of varying size and density
with duplicate edges and (optionally) many tied PPR values; the METIS
weights built from them; a random partition; the related-node expansion, the induced subgraph in global edge
order and the CSR-walk subgraph in set order -- each bit for bit against the
oracle."""
import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from neutrongt_amd import synthetic as S
from neutrongt_amd import window as W
from oracle import graph as OG

pytestmark = pytest.mark.gpu


def _d(a, dtype=torch.int64):
    return torch.as_tensor(np.ascontiguousarray(a), dtype=dtype).cuda()


@settings(max_examples=40, deadline=None, database=None, derandomize=True,
          suppress_health_check=[HealthCheck.too_slow])
@given(n=st.integers(1, 3000), mean_degree=st.floats(0.0, 30.0, allow_nan=False),
       gamma=st.floats(2.0, 3.0, allow_nan=False), seed=st.integers(0, 2**31 - 1),
       part_frac=st.floats(0.0, 1.0, allow_nan=False), pct=st.integers(0, 100),
       ties=st.booleans(), dup_frac=st.sampled_from([0.0, 0.1]))
def test_window_preparation_matches_the_oracle(n, mean_degree, gamma, seed, part_frac, pct, ties,
                                               dup_frac):
    rng = np.random.default_rng(seed)
    u, v = S.chung_lu_edges(n, mean_degree, gamma, seed)
    ei = np.stack([np.concatenate([u, v]), np.concatenate([v, u])])
    n_dup = int(dup_frac * ei.shape[1])
    if n_dup:
        ei = np.concatenate([ei, ei[:, rng.integers(0, ei.shape[1], n_dup)]], axis=1)
    ei = ei[:, rng.permutation(ei.shape[1])].astype(np.int64)
    E = ei.shape[1]
    val = (rng.integers(1, 5, E) / 1000 if ties else rng.random(E) / 100).astype(np.float32)
    xadj, adjncy, ew = OG.adj_weights(ei, val)
    # the METIS weights themselves (keys summed in entry order, truncated)
    gx, ga, gw = W.adj_weights(_d(ei), _d(val, torch.float32))
    for g, w in ((gx, xadj), (ga, adjncy), (gw, ew)):
        np.testing.assert_array_equal(g.cpu().numpy(), w)
    n_nodes = int(xadj.shape[0]) - 1
    part = rng.permutation(n_nodes)[: int(part_frac * n_nodes)].astype(np.int64)
    print(f"case window n={n} E={E} nodes={n_nodes} part={part.shape[0]} pct={pct} ties={ties} "
          f"mean_deg={mean_degree:.2f} gamma={gamma:.2f} seed={seed}", flush=True)
    # related-node expansion (sorted union of the partition and its top pct % external neighbours)
    want, _ = OG.merge_related_nodes(xadj, adjncy, ew, part, pct)
    got = W.merge_related_nodes(_d(xadj, torch.int32), _d(adjncy, torch.int32),
                                _d(ew, torch.int32), _d(part), pct)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    # the window's induced subgraph: global edge order, and CSR order over the set in a
    # random order (the set order is the relabelling)
    win = want
    want_coo = OG.subgraph_coo(win, ei, n_nodes)
    got_coo = W.subgraph(_d(win), _d(ei), n_nodes)
    np.testing.assert_array_equal(got_coo.cpu().numpy(), want_coo)
    node_set = win[rng.permutation(win.shape[0])]
    rowptr, col = xadj.astype(np.int64), adjncy.astype(np.int64)
    want_csr = OG.subgraph_from_csr(node_set, rowptr, col)
    got_csr = W.subgraph_from_csr(_d(node_set), _d(rowptr), _d(col))
    np.testing.assert_array_equal(got_csr.cpu().numpy(), want_csr)
