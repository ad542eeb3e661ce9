"""Pins the integer window-preparation oracle (no GPU) and checks the torch
host logic of neutrongt_amd.window against it."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import graph as OG
from tests._util import random_coo

GOLDEN = Path(__file__).parent / "golden"


# ------------------------------------------------------------------ CSR
def _brute_csr(src, dst, n_q):
    rows = [[] for _ in range(n_q)]
    for e, (s, d) in enumerate(zip(src.tolist(), dst.tolist())):
        rows[d].append((s, e))
    col, perm, rowptr = [], [], [0]
    for r in rows:
        for s, e in sorted(r):
            col.append(s)
            perm.append(e)
        rowptr.append(len(col))
    return np.array(rowptr), np.array(col), np.array(perm)


@pytest.mark.parametrize("n_q,n_k,E,seed", [(30, 30, 200, 0), (25, 60, 300, 1), (5, 5, 0, 2),
                                             (1, 1, 7, 3)])
def test_csr_matches_bruteforce(n_q, n_k, E, seed):
    ei = random_coo(n_q, n_k, E, seed=seed) if E else np.zeros((2, 0), np.int64)
    c = OG.csr_from_coo(ei[0], ei[1], n_q, n_k)
    rp, col, perm = _brute_csr(ei[0], ei[1], n_q)
    np.testing.assert_array_equal(c["rowptr"], rp)
    np.testing.assert_array_equal(c["col"], col)
    np.testing.assert_array_equal(c["perm"], perm)
    trp, tcol, tperm = _brute_csr(ei[1], ei[0], n_k)
    np.testing.assert_array_equal(c["t_rowptr"], trp)
    np.testing.assert_array_equal(c["t_col"], tcol)
    np.testing.assert_array_equal(c["t_perm"], tperm)
    # q2t maps each query-major edge to the same edge id in key-major order
    if E:
        np.testing.assert_array_equal(c["t_perm"][c["q2t"]], c["perm"])


def test_csr_matches_torch_sparse_on_duplicate_free_input():
    """Convention of NeutronGT/utils/trans2csr.py:23-35 (sparse_coo -> csr)."""
    rng = np.random.default_rng(5)
    n = 40
    key = np.unique(rng.integers(0, n * n, 300))
    dst, src = key // n, key % n
    perm = rng.permutation(key.shape[0])
    src, dst = src[perm], dst[perm]
    c = OG.csr_from_coo(src, dst, n, n)
    t = torch.sparse_coo_tensor(torch.from_numpy(np.stack([dst, src])), torch.ones(len(src)),
                                (n, n)).coalesce().to_sparse_csr()
    np.testing.assert_array_equal(c["rowptr"], t.crow_indices().numpy())
    np.testing.assert_array_equal(c["col"], t.col_indices().numpy())


def test_work_items_cover_each_row_once():
    ei = random_coo(50, 50, 900, seed=3)
    ei = np.concatenate([ei, np.stack([np.arange(300) % 50, np.zeros(300, np.int64)])], axis=1)
    c = OG.csr_from_coo(ei[0], ei[1], 50, 50)
    items, splits, packed = OG.work_items(c["rowptr"], chunk=16, small=4)
    cover = np.zeros(ei.shape[1], np.int64)
    for r, b, e, p in items.tolist():
        assert c["rowptr"][r] <= b <= e <= c["rowptr"][r + 1] and e - b <= 16
        cover[b:e] += 1
    deg = np.diff(c["rowptr"])
    for r in packed.tolist():
        assert deg[r] <= 4
        cover[c["rowptr"][r]:c["rowptr"][r + 1]] += 1
    assert (cover == 1).all()
    assert len({r for r, *_ in items.tolist()} | set(packed.tolist())) == 50
    n_split = sum(int(n) for _, _, n, _ in splits.tolist())
    assert (items[:n_split, 3] == np.arange(n_split)).all() and (items[n_split:, 3] == -1).all()
    # longest first among the single-item rows and the packed rows
    single = deg[items[n_split:, 0]]
    assert (np.diff(single) <= 0).all() and (np.diff(deg[packed]) <= 0).all()


# ------------------------------------------------------- related nodes
def test_merge_related_nodes_hand_derived():
    """Partition [2, 0, 1] of an 8-node weighted graph.  External neighbours in
    first-seen order: 6 (w 2), 7 (1), 3 (5), 4 (2+3=5), 5 (2).  Stable ranking by
    weight: 3, 4, 6, 5, 7 -- 6 precedes 5 (tie, seen first)."""
    z = np.load(GOLDEN / "related_small.npz")
    expect = {0: [0, 1, 2], 25: [0, 1, 2, 3], 50: [0, 1, 2, 3, 4], 60: [0, 1, 2, 3, 4, 6],
              100: [0, 1, 2, 3, 4, 5, 6, 7]}
    for pct, want in expect.items():
        out, n_ext = OG.merge_related_nodes(z["xadj"], z["adjncy"], z["eweights"], z["partition"],
                                            pct)
        assert out.tolist() == want and n_ext == 5
        assert z[f"out_{pct}"].tolist() == want


def _related_alt(xadj, adjncy, ew, part, pct):
    """Independent formulation: per external node, weight sum and first
    traversal index; rank by (-weight, first index)."""
    inpart = np.zeros(len(xadj) - 1, bool)
    inpart[part] = True
    w, first = {}, {}
    t = 0
    for u in part:
        for a in range(xadj[u], xadj[u + 1]):
            nb = adjncy[a]
            if not inpart[nb]:
                w[nb] = w.get(nb, 0) + ew[a]
                first.setdefault(nb, t)
            t += 1
    order = sorted(w, key=lambda x: (-w[x], first[x]))
    n_sel = len(order) * pct // 100 if pct > 0 else 0
    return np.array(sorted(set(part.tolist()) | set(order[:n_sel])), np.int64)


@pytest.mark.parametrize("seed", range(4))
def test_merge_related_nodes_matches_alternative(seed):
    rng = np.random.default_rng(seed)
    n = 200
    ei = rng.integers(0, n, (2, 1500))
    val = rng.integers(1, 4, 1500).astype(np.float32) / 1000  # many weight ties
    xadj, adjncy, ew = OG.adj_weights(ei, val)
    part = rng.permutation(n)[:40]
    for pct in (0, 7, 33, 50, 100):
        out, _ = OG.merge_related_nodes(xadj, adjncy, ew, part, pct)
        np.testing.assert_array_equal(out, _related_alt(xadj, adjncy, ew, part, pct))


# ------------------------------------------------------------- dup / cache
def test_duplicate_rerange_and_cache_hand_derived():
    parts = [np.array([5, 1, 9, 3]), np.array([3, 7, 5]), np.array([8, 2])]
    rer, dups = OG.duplicate_rerange(parts)
    assert [r.tolist() for r in rer] == [[5, 3, 1, 9], [3, 5, 7], [8, 2]]
    assert [d.tolist() for d in dups] == [[5, 3], [3, 5], []]
    cache_ids, idx = OG.dup_cache_metadata(dups)
    assert cache_ids.tolist() == [3, 5]
    assert [i.tolist() for i in idx] == [[1, 0], [0, 1], []]
    feat = np.arange(20, dtype=np.float32).reshape(10, 2)
    for r, i in zip(rer, idx):
        np.testing.assert_array_equal(OG.assemble_window_features(feat, cache_ids, i, r), feat[r])


def _dup_alt(parts):
    """Duplicate layout by counting with a dict and list scans (no unique,
    isin or searchsorted): the independent form the oracle is checked against."""
    count = {}
    for p in parts:
        for x in p.tolist():
            count[x] = count.get(x, 0) + 1
    rer, dups = [], []
    for p in parts:
        xs = p.tolist()
        d = [x for x in xs if count[x] >= 2]
        rer.append(d + [x for x in xs if count[x] < 2])
        dups.append(d)
    cache = sorted({x for x, c in count.items() if c >= 2})
    idx = [[cache.index(x) for x in d] for d in dups]
    return rer, dups, cache, idx


def dup_cases():
    """Hand-made windows: none duplicated, all duplicated, a node in 3+
    windows, an empty window, a node twice in one window, negative and large
    ids; plus random sets."""
    cases = [
        [np.array([4, 2, 9]), np.array([1, 7]), np.array([3])],
        [np.array([5, 6]), np.array([6, 5]), np.array([5, 6])],
        [np.array([0, 11, 3]), np.array([11, 4]), np.array([8, 11, 0]), np.array([11])],
        [np.array([], dtype=np.int64), np.array([2, 3]), np.array([3, 9])],
        [np.array([7, 7, 1]), np.array([2])],
        [np.array([-3, 2**40, 5]), np.array([5, -3]), np.array([2**40 + 1])],
        [np.array([], dtype=np.int64), np.array([], dtype=np.int64)],
        [np.array([12])],
    ]
    rng = np.random.default_rng(11)
    for t in range(6):
        W = int(rng.integers(2, 9))
        n = int(rng.integers(20, 4000))
        cases.append([rng.choice(n, int(rng.integers(0, min(n, 600))), replace=False)
                      for _ in range(W)])
    return cases


def test_dup_oracle_matches_counting_form():
    for parts in dup_cases():
        rer, dups = OG.duplicate_rerange(parts)
        cache, idx = OG.dup_cache_metadata(dups)
        rer_a, dups_a, cache_a, idx_a = _dup_alt(parts)
        assert [r.tolist() for r in rer] == rer_a
        assert [d.tolist() for d in dups] == dups_a
        assert cache.tolist() == cache_a
        assert [i.tolist() for i in idx] == idx_a


# -------------------------------------------------------------- adj weights
def test_adj_weights_hand_derived():
    # PPR pairs: (0,1) 0.0026 + (1,0) 0.0010 -> 0.0036*1000 = 3.6 -> 3; (2,0) 0.0004 -> 1 (clamp)
    ei = np.array([[0, 1, 2], [1, 0, 0]])
    val = np.array([0.0026, 0.0010, 0.0004], np.float32)
    xadj, adjncy, ew = OG.adj_weights(ei, val)
    assert xadj.tolist() == [0, 2, 3, 4]
    assert adjncy.tolist() == [1, 2, 0, 0]
    assert ew.tolist() == [3, 1, 3, 1]


def test_adj_weights_sums_each_key_in_entry_order():
    """Three PPR entries of one undirected key whose fp32 sum truncates to 2 in
    entry order ((0 + a) + b) + c and to 3 in the reverse order: the oracle
    follows the reference's sequential scatter_add_ (entry order)."""
    a, b, c = np.float32(0.0005994238), np.float32(0.0004226872), np.float32(0.0019778889)
    f = np.float32
    assert int(f(f(f(f(0) + a) + b) + c) * f(1000)) == 2
    assert int(f(f(f(f(0) + c) + b) + a) * f(1000)) == 3
    ei = np.array([[4, 1, 4], [1, 4, 1]])
    xadj, adjncy, ew = OG.adj_weights(ei, np.array([a, b, c], np.float32))
    assert ew.tolist() == [2, 2] and adjncy.tolist() == [4, 1]
    xadj, adjncy, ew = OG.adj_weights(ei[:, ::-1], np.array([c, b, a], np.float32))
    assert ew.tolist() == [3, 3]


def test_host_adj_weights_has_no_cpu_path():
    from neutrongt_amd import window as W

    ei = torch.tensor([[0, 1], [1, 0]])
    with pytest.raises(ValueError):
        W.adj_weights(ei, torch.tensor([0.1, 0.2]))


def test_subgraph_relabel_by_position():
    ei = np.array([[0, 3, 4, 3, 9], [3, 0, 3, 9, 4]])
    sub = OG.subgraph_coo(np.array([4, 3, 0]), ei, 10)
    # kept edges in global order: (0,3), (3,0), (4,3) -> positions (2,1), (1,2), (0,1)
    assert sub.tolist() == [[2, 1, 0], [1, 2, 1]]


def _csr_of(ei, n):
    """Row-major CSR of a COO (rows = edge_index[0]), neighbours in edge order,
    and the COO listed in that CSR order (graph_data.py:28-35 convention)."""
    order = np.argsort(ei[0], kind="stable")
    rowptr = np.zeros(n + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(ei[0], minlength=n))
    return rowptr, ei[1][order], ei[:, order]


def test_subgraph_from_csr_hand_derived():
    # CSR of 6 nodes; set [4, 1, 3]: row 4 -> (1, 3), row 1 -> (4, 2, 4), row 3 -> (5)
    rowptr = np.array([0, 1, 4, 5, 6, 8, 8])
    col = np.array([1, 4, 2, 4, 0, 5, 1, 3])
    out = OG.subgraph_from_csr(np.array([4, 1, 3]), rowptr, col)
    assert out.tolist() == [[0, 0, 1, 1], [1, 2, 0, 0]]


@pytest.mark.parametrize("seed", range(3))
def test_subgraph_from_csr_matches_brute_force_and_coo_form(seed):
    rng = np.random.default_rng(seed)
    n = 300
    ei = rng.integers(0, n, (2, 3000))
    rowptr, col, ei_csr = _csr_of(ei, n)
    node_set = rng.permutation(n)[:90]
    got = OG.subgraph_from_csr(node_set, rowptr, col)
    where = {int(g): i for i, g in enumerate(node_set)}
    want = [(i, where[int(c)]) for i, g in enumerate(node_set)
            for c in col[rowptr[g]:rowptr[g + 1]] if int(c) in where]
    assert got.T.tolist() == [list(t) for t in want]
    # sorted set: the CSR form lists edges in the same order as the COO form
    # over the CSR-ordered edge list
    s = np.sort(node_set)
    np.testing.assert_array_equal(OG.subgraph_from_csr(s, rowptr, col),
                                  OG.subgraph_coo(s, ei_csr, n))


@pytest.mark.parametrize("seed", range(3))
def test_subgraph_coo_matches_brute_force(seed):
    rng = np.random.default_rng(seed + 10)
    n = 200
    ei = rng.integers(0, n, (2, 2500))
    subset = rng.permutation(n)[:70]
    where = {int(g): i for i, g in enumerate(subset)}
    want = [(where[int(a)], where[int(b)]) for a, b in ei.T if int(a) in where and int(b) in where]
    assert OG.subgraph_coo(subset, ei, n).T.tolist() == [list(t) for t in want]


def test_chung_lu_degree_cap():
    """The generator's degree cap flattens only the heaviest weights: without
    it the draw is unchanged (the benchmark windows depend on that), with it
    the largest degree drops to about the cap while the mean degree holds."""
    from neutrongt_amd import synthetic as S
    n, mean = 20000, 14.0
    u0, v0 = S.chung_lu_edges(n, mean, 2.1, S.SEED)
    u1, v1 = S.chung_lu_edges(n, mean, 2.1, S.SEED, degree_cap=None)
    assert np.array_equal(u0, u1) and np.array_equal(v0, v1)
    d0 = np.bincount(np.concatenate([u0, v0]), minlength=n)
    u2, v2 = S.chung_lu_edges(n, mean, 2.1, S.SEED, degree_cap=200)
    d2 = np.bincount(np.concatenate([u2, v2]), minlength=n)
    assert d0.max() > 1000 and d2.max() < 1.3 * 200
    assert abs(d2.mean() - mean) < 0.05 * mean
    assert np.all(u2 < v2)
    # a cap above the heaviest expected degree changes nothing
    u3, v3 = S.chung_lu_edges(n, mean, 2.1, S.SEED, degree_cap=1e9)
    assert np.array_equal(u0, u3) and np.array_equal(v0, v3)
