"""Property tests of the oracle over random Chung-Lu windows of varying size
and density (hypothesis): the restatement of the reference's op sequence
against the float64 dense masked form, its autograd against the hand-derived
backward and exact identities of that backward, and the CSR / work-list
restatements against their defining invariants."""
import math

import numpy as np
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from neutrongt_amd import synthetic as S
from oracle import attention as OA
from oracle import graph as OG
from tests._strategies import windows
from tests._util import assert_close, relerr

PROPS = settings(max_examples=40, deadline=None, database=None, derandomize=True,
                 suppress_health_check=[HealthCheck.too_slow])


def _qkv(n_q, n_k, H, d, qscale, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n_q, H, d, generator=g) * qscale
    k = torch.randn(n_k, H, d, generator=g)
    v = torch.randn(n_k, H, d, generator=g)
    go = torch.randn(n_q, H, d, generator=g)
    return q, k, v, go


@PROPS
@given(win=windows(), H=st.sampled_from([1, 2, 4]), d=st.sampled_from([2, 4, 8]),
       qscale=st.sampled_from([0.3, 1.0, 4.0]))
def test_forward_matches_dense_fp64(win, H, d, qscale):
    q, k, v, go = _qkv(win.n_q, win.n_k, H, d, qscale, seed=len(win.desc))
    ei = torch.from_numpy(win.edge_index)
    got = OA.sparse_fwd_bwd(q, k, v, ei, go, H)
    x64, z64 = OA.sparse_bruteforce_fp64(q, k, v, ei)
    assert_close(got["x"], x64, torch.float32, f"x {win.desc}")
    # node score of row i: mean over heads of Z, rows up to max(dst)
    n_s = int(win.edge_index[1].max()) + 1 if win.edge_index.shape[1] else 0
    assert got["node_scores"].shape[0] == n_s
    assert_close(got["node_scores"], z64.mean(1)[:n_s], torch.float32, f"ns {win.desc}")


@PROPS
@given(win=windows(), H=st.sampled_from([1, 3]), d=st.sampled_from([4, 8]),
       qscale=st.sampled_from([0.5, 3.0]))
def test_backward_matches_closed_form_and_identities(win, H, d, qscale):
    q, k, v, go = _qkv(win.n_q, win.n_k, H, d, qscale, seed=7 + len(win.desc))
    ei = torch.from_numpy(win.edge_index)
    # float64 autograd of the restatement: the backward of a row with few
    # edges is ill-conditioned (dp = r (G.V - G.X) with X close to V), so fp32
    # would pin only its rounding; in float64 a wrong formula still shows
    got = OA.sparse_fwd_bwd(q, k, v, ei, go, H, dtype=torch.float64)
    dq, dk, dv = OA.sparse_backward_closed_form(q, k, v, ei, go)
    for name, ref in (("dq", dq), ("dk", dk), ("dv", dv)):
        e = relerr(got[name], ref)
        assert e <= 1e-9, f"{name} {win.desc}: relative error {e:.3e}"
    # identities of the closed form: <dQ,Q> = <dK,K> = sum_e da_e a_e, and
    # sum_j dV_j = sum_i Z_i / (Z_i + eps) G_i per head
    j, i = ei[0], ei[1]
    q64, k64, g64 = q.double(), k.double(), go.double()
    a = (k64[j] * q64[i]).sum(-1) / math.sqrt(d)
    _, z = OA.sparse_bruteforce_fp64(q, k, v, ei)
    lhs_q = (dq * q64).sum()
    lhs_k = (dk * k64).sum()
    x64, _ = OA.sparse_bruteforce_fp64(q, k, v, ei)
    r = 1.0 / (z + OA.EPS)
    dd = (g64 * x64).sum(-1)
    p = torch.exp(a.clamp(OA.CLAMP_LO, OA.CLAMP_HI))
    inside = ((a >= OA.CLAMP_LO) & (a <= OA.CLAMP_HI)).double()
    da = r[i] * ((g64[i] * v.double()[j]).sum(-1) - dd[i]) * p * inside
    rhs = (da * a).sum()
    scale = max(1.0, rhs.abs().item())
    assert abs(lhs_q.item() - rhs.item()) <= 1e-9 * scale
    assert abs(lhs_k.item() - rhs.item()) <= 1e-9 * scale
    sv = (z / (z + OA.EPS)).unsqueeze(-1) * g64
    assert relerr(dv.sum(0), sv.sum(0)) <= 1e-9 or sv.abs().max() == 0


@PROPS
@given(win=windows(max_n=60, max_related=30), chunk=st.sampled_from([1, 3, 8, 64, 256]),
       small=st.sampled_from([0, 1, 2, 8]))
def test_csr_and_work_lists_invariants(win, chunk, small):
    small = min(small, chunk - 1)  # the host keeps small < chunk (WindowAdjacency)
    src, dst = win.edge_index
    E = src.shape[0]
    c = OG.csr_from_coo(src, dst, win.n_q, win.n_k)
    perm, t_perm, q2t = (c[n].astype(np.int64) for n in ("perm", "t_perm", "q2t"))
    # both orders are permutations of the edge ids
    assert np.array_equal(np.sort(perm), np.arange(E))
    assert np.array_equal(np.sort(t_perm), np.arange(E))
    # query-major: sorted by (dst, src, edge id); key-major by (src, dst, edge id)
    kq = np.stack([dst[perm], src[perm], perm], 1)
    assert all(tuple(kq[t]) < tuple(kq[t + 1]) for t in range(E - 1))
    kk = np.stack([src[t_perm], dst[t_perm], t_perm], 1)
    assert all(tuple(kk[t]) < tuple(kk[t + 1]) for t in range(E - 1))
    assert np.array_equal(c["col"], src[perm]) and np.array_equal(c["t_col"], dst[t_perm])
    assert np.array_equal(np.diff(c["rowptr"]), np.bincount(dst, minlength=win.n_q))
    assert np.array_equal(np.diff(c["t_rowptr"]), np.bincount(src, minlength=win.n_k))
    # q2t: the key-major position of each query-major edge
    assert np.array_equal(t_perm[q2t], perm)
    # work lists: every edge of every row exactly once, chunks <= chunk edges
    for rp in (c["rowptr"], c["t_rowptr"]):
        items, splits, packed = OG.work_items(rp, chunk, small)
        deg = np.diff(rp.astype(np.int64))
        cover = np.zeros(E, np.int64)
        for r, b, e, part in items:
            assert 0 < e - b <= chunk and rp[r] <= b and e <= rp[r + 1]
            cover[b:e] += 1
        for r in packed:
            assert deg[r] <= small
            cover[rp[r]:rp[r + 1]] += 1
        assert np.all(cover == 1)
        assert np.all(deg[packed] <= small) and len(set(packed.tolist())) == packed.shape[0]
        assert int((deg > chunk).sum()) == splits.shape[0]


@PROPS
@given(n=st.integers(0, 300), mean_degree=st.floats(0.0, 400.0, allow_nan=False),
       gamma=st.floats(2.0, 3.0, allow_nan=False), seed=st.integers(0, 2**31 - 1))
def test_chung_lu_generator_stays_bounded(n, mean_degree, gamma, seed):
    """Any size and density, including targets a small graph cannot hold:
    distinct undirected pairs u < v inside [0, n), never more than exist."""
    u, v = S.chung_lu_edges(n, mean_degree, gamma, seed)
    assert u.shape == v.shape
    assert np.all(u < v) and np.all(u >= 0) and np.all(v < max(n, 1))
    assert np.unique(u * max(n, 1) + v).shape[0] == u.shape[0]
    assert u.shape[0] <= n * (n - 1) // 2
