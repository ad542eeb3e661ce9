"""APPNP personalised PageRank on the GPU (ngt_ppr_count with
ngt_ppr_step_direct or ngt_ppr_step) against the oracle, bit for bit (same
fp32 operations in the same order), and the two step forms against each
other on graphs too large for the oracle."""
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


METHODS = ("direct", "sort")


@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("n,E,K,batch,iters,seed,hub", [
    (200, 800, 5, 8, 10, 0, False),     # the shipped setting: topk 5, 10 iterations
    (300, 1500, 1, 64, 4, 1, False),
    (400, 1200, 16, 1000, 6, 2, True),  # hub rows with thousands of products
    (150, 300, 64, 7, 3, 3, False),
    (600, 2400, 5, 600, 10, 4, True),   # hub rows over many 512-position chunks
])
def test_appnp_bit_exact(n, E, K, batch, iters, seed, hub, method):
    from neutrongt_amd.ppr import personal_pagerank_appnp

    ei = _graph(n, E, seed, hub)
    want_i, want_v = OP.personal_pagerank_appnp(ei, 0.85, topk=K, num_iterations=iters,
                                                num_nodes=n, iter_topk=K)
    got_i, got_v = personal_pagerank_appnp(torch.from_numpy(ei), 0.85, topk=K,
                                           num_iterations=iters, batch_size=batch, device=DEV,
                                           num_nodes=n, iter_topk=K, method=method)
    np.testing.assert_array_equal(got_i.cpu().numpy(), want_i)
    np.testing.assert_array_equal(got_v.cpu().numpy(), want_v)


@pytest.mark.parametrize("method", METHODS)
def test_appnp_csr_input_source_range_and_final_topk(method):
    from neutrongt_amd.ppr import personal_pagerank_appnp

    n = 250
    ei = _graph(n, 1000, 5)
    rowptr, col, _, _ = OP.transition_csr(ei, n)
    want_i, want_v = OP.personal_pagerank_appnp(ei, 0.5, topk=3, num_iterations=5, num_nodes=n,
                                                iter_topk=6, source_start=40, source_end=170)
    got_i, got_v = personal_pagerank_appnp(
        None, 0.5, topk=3, num_iterations=5, batch_size=50, device=DEV,
        csr_data={"rowptr": torch.from_numpy(rowptr), "col": torch.from_numpy(col)},
        iter_topk=6, source_start=40, source_end=170, method=method)
    np.testing.assert_array_equal(got_i.cpu().numpy(), want_i)
    np.testing.assert_array_equal(got_v.cpu().numpy(), want_v)


@pytest.mark.parametrize("method", METHODS)
def test_appnp_csr_rows_in_any_order(method):
    """A CSR whose rows list their columns in shuffled order gives the
    oracle's result: transition_csr sorts the rows for the direct step, and a
    row's order never changes a sum (repeats carry one product)."""
    from neutrongt_amd.ppr import personal_pagerank_appnp

    n = 220
    ei = _graph(n, 900, 6, hub=True)
    rowptr, col, _, _ = OP.transition_csr(ei, n)
    rng = np.random.default_rng(6)
    shuffled = col.copy()
    for r in range(n):
        rng.shuffle(shuffled[rowptr[r]:rowptr[r + 1]])
    assert not np.array_equal(shuffled, col)
    want_i, want_v = OP.personal_pagerank_appnp(ei, 0.85, topk=5, num_iterations=6, num_nodes=n,
                                                iter_topk=5)
    got_i, got_v = personal_pagerank_appnp(
        None, 0.85, topk=5, num_iterations=6, batch_size=64, device=DEV,
        csr_data={"rowptr": torch.from_numpy(rowptr), "col": torch.from_numpy(shuffled)},
        iter_topk=5, method=method)
    np.testing.assert_array_equal(got_i.cpu().numpy(), want_i)
    np.testing.assert_array_equal(got_v.cpu().numpy(), want_v)


def test_direct_step_flags_rows_out_of_order():
    """Handed an unsorted CSR directly, the direct step reports it (status[1])
    and appnp_batch raises."""
    from neutrongt_amd import ppr as PPR

    rowptr = torch.tensor([0, 3, 5, 6, 8], device=DEV)
    col = torch.tensor([2, 1, 3, 0, 2, 3, 1, 0], device=DEV)
    inv = 1.0 / (rowptr[1:] - rowptr[:-1]).clamp_min(1).float()
    seeds = torch.arange(4, device=DEV)
    with pytest.raises(ValueError, match="ascending"):
        PPR.appnp_batch(rowptr, col, inv, 4, seeds, 0.85, 3, 2, method="direct")
    PPR.appnp_batch(rowptr, col, inv, 4, seeds, 0.85, 3, 2, method="sort")


def test_direct_step_flags_a_total_below_the_counts():
    """A product total too small for the state's lists (its chunks would not
    fit the workspace sized from it) is flagged in status[1] and nothing is
    written past the workspace."""
    import ctypes as C

    from neutrongt_amd import _lib

    lib = _lib.load()
    # a star: node 0 adjacent to nodes 1..2000, each adjacent to node 0
    n = 2001
    rowptr = torch.cat([torch.tensor([0]), torch.arange(2000, 4001)]).to(DEV)
    col = torch.cat([torch.arange(1, 2001), torch.zeros(2000, dtype=torch.long)]).to(DEV)
    inv = 1.0 / (rowptr[1:] - rowptr[:-1]).float()
    K, B = 1, 1
    st_col = torch.zeros(B, K, dtype=torch.int32, device=DEV)  # state: node 0, 2,000 entries
    st_val = torch.ones(B, K, device=DEV)
    st_cnt = torch.ones(B, dtype=torch.int32, device=DEV)
    seeds = torch.zeros(B, dtype=torch.long, device=DEV)
    total = 1  # room for 1 * (K + 1) + 1 = 3 chunks; node 0's list needs 4
    sb = C.c_size_t()
    _lib.check(lib.ngt_ppr_step_direct_workspace_bytes(total, B, K, C.byref(sb)))
    ws = torch.empty(sb.value, dtype=torch.uint8, device=DEV)
    out_col = torch.empty_like(st_col)
    out_val = torch.empty_like(st_val)
    out_cnt = torch.empty_like(st_cnt)
    status = torch.zeros(2, dtype=torch.int32, device=DEV)
    _lib.check(lib.ngt_ppr_step_direct(rowptr.data_ptr(), col.data_ptr(), inv.data_ptr(), n,
                                       st_col.data_ptr(), st_val.data_ptr(), st_cnt.data_ptr(),
                                       seeds.data_ptr(), B, K, 0.85, 0.15, 1, total,
                                       out_col.data_ptr(), out_val.data_ptr(),
                                       out_cnt.data_ptr(), status.data_ptr(), ws.data_ptr(),
                                       sb.value, _lib.stream_ptr(DEV)))
    assert status.tolist() == [0, 1]


def _simple_graph(n, E, hubs, hub_deg, seed):
    """Random edges plus hub nodes adjacent to hub_deg distinct others,
    symmetric, without self loops or duplicate edges (max_repeats = 1)."""
    rng = np.random.default_rng(seed)
    ei = rng.integers(0, n, (2, E))
    h = np.stack([np.repeat(np.arange(hubs), hub_deg),
                  np.concatenate([rng.choice(n, hub_deg, replace=False) for _ in range(hubs)])])
    ei = np.concatenate([ei, h], axis=1)
    ei = np.concatenate([ei, ei[::-1]], axis=1)
    return np.unique(ei[:, ei[0] != ei[1]], axis=1)


@pytest.mark.parametrize("K", [5, 2])
def test_direct_step_prunes_without_changing_a_bit(K):
    """A graph without duplicate edges and with hub rows, where the direct
    step's bound drops most hub columns before their exact evaluation (a CPU
    emulation of the kernel counted 22,648 of 38,272 columns dropped at K = 5):
    the rows equal the oracle's bit for bit."""
    from neutrongt_amd import ppr as PPR

    n = 1500
    ei = _simple_graph(n, 6000, 3, 700, 9)
    rowptr, col, inv, _ = OP.transition_csr(ei, n)
    assert PPR.max_repeats(torch.from_numpy(rowptr), torch.from_numpy(col)) == 1
    seeds = torch.tensor([0, 1, 2, 5, 50, 700, 1499, 3, 4, 60, 900], device=DEV)
    cols, vals, cnt = PPR.appnp_batch(torch.from_numpy(rowptr).to(DEV),
                                      torch.from_numpy(col).to(DEV),
                                      torch.from_numpy(inv).to(DEV), n, seeds, 0.85, K, 5)
    cols, vals, cnt = cols.cpu().numpy(), vals.cpu().numpy(), cnt.cpu().numpy()
    for i, sd in enumerate(seeds.tolist()):
        want = OP.appnp_row(rowptr, col, inv, sd, 0.85, K, 5)
        assert cnt[i] == len(want)
        assert cols[i, :cnt[i]].tolist() == [c for c, _ in want]
        np.testing.assert_array_equal(vals[i, :cnt[i]], np.array([v for _, v in want], np.float32))


@pytest.mark.parametrize("K,hub_deg", [(5, 20000), (32, 3000)])
def test_direct_and_sorted_steps_agree_on_a_large_graph(K, hub_deg):
    """Past the oracle's reach: a 30,000-node random graph with hub rows (one
    node adjacent to hub_deg others), all seeds, 10 iterations; the direct
    step (with and without its pruning) and the sorted product list give the
    same bits."""
    from neutrongt_amd import ppr as PPR

    n = 30000
    rng = np.random.default_rng(11)
    ei = rng.integers(0, n, (2, 12 * n))
    hubs = np.stack([np.repeat(np.arange(4), hub_deg), rng.integers(0, n, 4 * hub_deg)])
    ei = np.concatenate([ei, hubs], axis=1)
    ei = torch.from_numpy(np.concatenate([ei, ei[::-1]], axis=1))
    rowptr, col, inv, _ = PPR.transition_csr(ei, num_nodes=n, device=DEV)
    mult = PPR.max_repeats(rowptr, col)
    seeds = torch.arange(n, device=DEV)
    got = [PPR.appnp_batch(rowptr, col, inv, n, seeds, 0.85, K, 10, method=m, max_mult=mm)
           for m, mm in (("direct", mult), ("direct", 0), ("sort", None))]
    live = torch.arange(K, device=DEV)[None, :] < got[0][2][:, None]  # slots past cnt: unset
    for c, v, k in got[1:]:
        assert torch.equal(k, got[0][2]) and torch.equal(c[live], got[0][0][live])
        assert torch.equal(v[live].view(torch.int32), got[0][1][live].view(torch.int32))
    full = _simple_graph(n, 12 * n, 4, hub_deg, 12)
    got = [PPR.personal_pagerank_appnp(torch.from_numpy(full), 0.85, topk=K, num_iterations=10,
                                       batch_size=8192, device=DEV, num_nodes=n, iter_topk=K,
                                       method=m) for m in METHODS]
    assert got[0][0].shape[1] == n * K
    assert torch.equal(got[0][0], got[1][0])
    assert torch.equal(got[0][1].view(torch.int32), got[1][1].view(torch.int32))


def test_appnp_rejects_unbounded_state_and_bad_ids():
    from neutrongt_amd.ppr import personal_pagerank_appnp

    ei = torch.tensor([[0, 1], [1, 0]])
    with pytest.raises(NotImplementedError):
        personal_pagerank_appnp(ei, 0.85, topk=5, device=DEV, iter_topk=0)
    bad = {"rowptr": torch.tensor([0, 1, 2]), "col": torch.tensor([1, 7])}
    for method in METHODS:
        with pytest.raises(IndexError):
            personal_pagerank_appnp(None, 0.85, topk=2, device=DEV, csr_data=bad, iter_topk=2,
                                    method=method)


def test_appnp_batches_in_flight_give_the_same_bits():
    """Batches run with 1, 2, 3 or 8 in flight (a stream each) give the same
    bits as the oracle, with more batches than streams and a short last
    batch; an id out of range in a later batch still raises."""
    from neutrongt_amd.ppr import personal_pagerank_appnp

    n = 700
    ei = _graph(n, 3000, 13, hub=True)
    want_i, want_v = OP.personal_pagerank_appnp(ei, 0.85, topk=5, num_iterations=6, num_nodes=n,
                                                iter_topk=5)
    for streams in (1, 2, 3, 8):
        got_i, got_v = personal_pagerank_appnp(torch.from_numpy(ei), 0.85, topk=5,
                                               num_iterations=6, batch_size=45, device=DEV,
                                               num_nodes=n, iter_topk=5, streams=streams)
        np.testing.assert_array_equal(got_i.cpu().numpy(), want_i)
        np.testing.assert_array_equal(got_v.cpu().numpy(), want_v)
    # called on a stream of the caller's: the graph is made on it, and the
    # result is read there without a device-wide sync
    user = torch.cuda.Stream(DEV)
    with torch.cuda.stream(user):
        ei_dev = torch.from_numpy(ei).to(DEV, non_blocking=False)
        got_i, got_v = personal_pagerank_appnp(ei_dev, 0.85, topk=5, num_iterations=6,
                                               batch_size=45, device=DEV, num_nodes=n,
                                               iter_topk=5, streams=4)
        host_i, host_v = got_i.cpu(), got_v.cpu()
    np.testing.assert_array_equal(host_i.numpy(), want_i)
    np.testing.assert_array_equal(host_v.numpy(), want_v)
    rowptr = torch.arange(0, 41, device=DEV)
    col = (torch.arange(40, device=DEV) + 1) % 40
    col[37] = 99  # only the last batch's seeds reach it
    for streams in (1, 3):
        with pytest.raises(IndexError):
            personal_pagerank_appnp(None, 0.85, topk=2, batch_size=8, device=DEV,
                                    csr_data={"rowptr": rowptr, "col": col}, iter_topk=2,
                                    num_iterations=2, streams=streams)


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
                                      max_products=700, method="sort")
    cols, vals, cnt = cols.cpu().numpy(), vals.cpu().numpy(), cnt.cpu().numpy()
    for r in range(120):
        want = OP.appnp_row(rowptr, col, inv, r, 0.85, 5, 4)
        assert cnt[r] == len(want)
        assert cols[r, :cnt[r]].tolist() == [c for c, _ in want]
        np.testing.assert_array_equal(vals[r, :cnt[r]], np.array([v for _, v in want], np.float32))


def _random_case(seed):
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(20, 3000))
    E = int(rng.integers(n, 12 * n))
    ei = rng.integers(0, n, (2, E))
    if rng.random() < 0.5:  # hubs
        h = int(rng.integers(1, 4))
        deg = int(rng.integers(n // 4, n))
        ei = np.concatenate([ei, np.stack([rng.integers(0, n, h * deg) % h,
                                           rng.integers(0, n, h * deg)])], axis=1)
    if rng.random() < 0.7:
        ei = np.concatenate([ei, ei[::-1]], axis=1)
    if rng.random() < 0.5:  # simple graph: max_repeats 1
        ei = np.unique(ei[:, ei[0] != ei[1]], axis=1)
    K = int(rng.choice([1, 2, 5, 8, 33, 64]))
    alpha = float(rng.choice([0.0, 0.15, 0.5, 0.85, 1.0]))
    iters = int(rng.integers(2, 7))
    return n, torch.from_numpy(ei), K, alpha, iters


@pytest.mark.parametrize("seed", range(40))
def test_direct_and_sorted_steps_agree_on_random_graphs(seed):
    """Random graphs (duplicate edges or none, hubs, isolated nodes), K from 1
    to 64 (states past 32 lists take the direct step's per-lane slice
    search), alpha from 0 (keep 1) to 1 (keep 0: no pruning bound): the
    direct step with and without its bound and the sorted products give the
    same bits for every seed."""
    from neutrongt_amd import ppr as PPR

    n, ei, K, alpha, iters = _random_case(seed)
    print(f"case ppr random seed={seed} n={n} E={ei.shape[1]} K={K} alpha={alpha}", flush=True)
    rowptr, col, inv, _ = PPR.transition_csr(ei, num_nodes=n, device=DEV)
    mult = PPR.max_repeats(rowptr, col)
    seeds = torch.arange(n, device=DEV)
    got = [PPR.appnp_batch(rowptr, col, inv, n, seeds, alpha, min(K, n), iters, method=m,
                           max_mult=mm)
           for m, mm in (("direct", mult), ("direct", 0), ("sort", None))]
    live = torch.arange(min(K, n), device=DEV)[None, :] < got[0][2][:, None]  # slots past cnt: unset
    for c, v, k in got[1:]:
        assert torch.equal(k, got[0][2])
        assert torch.equal(c[live], got[0][0][live])
        assert torch.equal(v[live].view(torch.int32), got[0][1][live].view(torch.int32))
