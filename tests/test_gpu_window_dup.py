"""GPU duplicate-node layout (ngt_window_dup_layout) against the oracle's
restatement of _compute_local_duplicate_nodes and build_dup_cache_metadata
(NeutronGT/core/node_level_pipeline/window_state.py:52-73, :181-205),
bit-exact: reranged windows, per-window duplicate lists, the sorted cache ids
and the per-window cache indices; then the window features assembled from the
cache equal feature[window] bit for bit."""
import numpy as np
import pytest
import torch

from neutrongt_amd import window as W
from oracle import graph as OG
from tests.test_oracle_graph import dup_cases

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _oracle(parts):
    rer, dups = OG.duplicate_rerange(parts)
    cache, idx = OG.dup_cache_metadata(dups)
    return rer, dups, cache, idx


def _same(got, want, what):
    assert got.dtype == torch.int64, (what, got.dtype)
    assert got.is_cuda, what
    np.testing.assert_array_equal(got.cpu().numpy(), np.asarray(want, np.int64), err_msg=what)


@pytest.mark.parametrize("case", range(len(dup_cases())))
def test_dup_layout_matches_oracle(case):
    parts = dup_cases()[case]
    _say(f"case dup layout {case}: {len(parts)} windows, {sum(len(p) for p in parts)} nodes")
    rer_o, dups_o, cache_o, idx_o = _oracle(parts)
    # CPU windows in (as the reference holds them), and GPU windows in
    for src in ([torch.from_numpy(np.asarray(p, np.int64)) for p in parts],
                [torch.from_numpy(np.asarray(p, np.int64)).cuda() for p in parts]):
        rer, dups, cache, idx = W.window_dup_layout(src)
        assert len(rer) == len(dups) == len(idx) == len(parts)
        for w in range(len(parts)):
            _same(rer[w], rer_o[w], f"reranged[{w}]")
            _same(dups[w], dups_o[w], f"dups[{w}]")
            _same(idx[w], idx_o[w], f"dup_index[{w}]")
        _same(cache, cache_o, "cache_ids")
    # the two reference functions one by one
    rer2, dups2 = W.duplicate_rerange([torch.from_numpy(np.asarray(p, np.int64)) for p in parts])
    for w in range(len(parts)):
        _same(rer2[w], rer_o[w], f"duplicate_rerange[{w}]")
    cache2, idx2 = W.dup_cache_metadata(dups2)
    _same(cache2, cache_o, "dup_cache_metadata cache")
    assert len(idx2) == len(parts)
    for w in range(len(parts)):
        _same(idx2[w], idx_o[w], f"dup_cache_metadata idx[{w}]")


def test_dup_layout_empty_rank():
    _say("case dup layout no windows")
    rer, dups, cache, idx = W.window_dup_layout([])
    assert rer == [] and dups == [] and idx == [] and cache.numel() == 0
    cache, idx = W.dup_cache_metadata([])
    assert cache.numel() == 0 and idx == []


def test_dup_cache_metadata_of_lists_with_single_ids():
    # build_dup_cache_metadata takes any lists: an id listed once is cached too
    _say("case dup cache metadata, ids listed once")
    lists = [np.array([9, 4]), np.array([], dtype=np.int64), np.array([4, 1, 30])]
    cache_o, idx_o = OG.dup_cache_metadata(lists)
    cache, idx = W.dup_cache_metadata([torch.from_numpy(x) for x in lists])
    _same(cache, cache_o, "cache")
    for w in range(len(lists)):
        _same(idx[w], idx_o[w], f"idx[{w}]")


def test_dup_layout_rank_scale_and_feature_assembly():
    # 16 windows of 32,768 nodes over a 600,000-node graph (a GPH_Large rank's
    # share of windows with related-node overlap), then x_i from the cache
    _say("case dup layout 16 x 32768 windows")
    rng = np.random.default_rng(5)
    n = 600_000
    parts = [rng.choice(n, 32_768, replace=False) for _ in range(16)]
    rer_o, dups_o, cache_o, idx_o = _oracle(parts)
    rer, dups, cache, idx = W.window_dup_layout([torch.from_numpy(p) for p in parts])
    _same(cache, cache_o, "cache_ids")
    for w in range(len(parts)):
        _same(rer[w], rer_o[w], f"reranged[{w}]")
        _same(idx[w], idx_o[w], f"dup_index[{w}]")
    feat = torch.randn(n, 100, generator=torch.Generator().manual_seed(1))
    fd = feat.cuda()
    fcache = W.dup_feature_cache(fd, cache)
    assert torch.equal(fcache.cpu(), feat[torch.from_numpy(cache_o)])
    for w in (0, 7, 15):
        x = W.assemble_window_features(fd, fcache, idx[w], rer[w])
        assert torch.equal(x.cpu(), feat[torch.from_numpy(rer_o[w])])


@pytest.mark.parametrize("use_cache,route", [(True, "coo"), (True, "csr"), (False, "coo")])
def test_rebuild_local_windows_matches_oracle(use_cache, route):
    """A rank's windows rebuilt as _rebuild_local_window_structures does
    (window_state.py:223-260): duplicate layout and feature cache, then each
    window's induced subgraph over its (reranged) partition, from the global
    COO or CSR; x_i from the cache equals feature[partition]."""
    _say(f"case rebuild local windows cache={use_cache} route={route}")
    rng = np.random.default_rng(17)
    n, E = 3000, 40000
    src = rng.integers(0, n, E)
    dst = rng.integers(0, n, E)
    order = np.lexsort((dst, src))  # CSR order for the csr route
    ei = np.stack([src[order], dst[order]]).astype(np.int64)
    rowptr = np.searchsorted(ei[0], np.arange(n + 1)).astype(np.int64)
    parts = [np.sort(rng.choice(n, 700, replace=False)) for _ in range(5)]  # overlapping windows
    feat = torch.randn(n, 24, generator=torch.Generator().manual_seed(3))
    fd = feat.cuda()
    kw = (dict(edge_index=torch.from_numpy(ei).cuda(), num_nodes=n) if route == "coo" else
          dict(rowptr=torch.from_numpy(rowptr).cuda(), col=torch.from_numpy(ei[1]).cuda()))
    lw = W.rebuild_local_windows([torch.from_numpy(p) for p in parts], fd, use_cache=use_cache, **kw)
    if use_cache:
        rer_o, dups_o, cache_o, idx_o = _oracle(parts)
    else:
        rer_o, dups_o = parts, [np.zeros(0, np.int64)] * len(parts)
        cache_o, idx_o = np.zeros(0, np.int64), []
    assert len(lw.partitions) == len(parts) and len(lw.sub_edge_index) == len(parts)
    assert lw.feature_cache.shape == (len(cache_o), 24)
    assert torch.equal(lw.feature_cache.cpu(), feat[torch.from_numpy(np.asarray(cache_o, np.int64))])
    for w in range(len(parts)):
        _same(lw.partitions[w], rer_o[w], f"partition[{w}]")
        _same(lw.dup_nodes[w], dups_o[w], f"dups[{w}]")
        if use_cache:
            _same(lw.dup_indices[w], idx_o[w], f"dup_index[{w}]")
        want = (OG.subgraph_coo(rer_o[w], ei, n) if route == "coo"
                else OG.subgraph_from_csr(rer_o[w], rowptr, ei[1]))
        _same(lw.sub_edge_index[w], want, f"sub_edge_index[{w}]")
        x = lw.features(w, fd)
        assert torch.equal(x.cpu(), feat[torch.from_numpy(np.asarray(rer_o[w], np.int64))])
    assert set(lw.timings) == {"local_dup_cache_rebuild_time", "local_subgraph_rebuild_time",
                               "local_spatial_rebuild_time"}
