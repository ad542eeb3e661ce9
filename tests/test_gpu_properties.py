"""Property tests on the GPU (hypothesis, derandomized: every run draws the
same cases): random Chung-Lu windows of varying size, density and power-law
exponent, with related key rows, duplicate edges and shuffled edge order,
across head counts, head dims, dtypes, chunk sizes and packing thresholds.
Each case checks the CSR, the transposed CSR and both work lists bit for bit
against the oracle, and forward + backward against the oracle at the path's
tolerance."""
import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from neutrongt_amd import SparseAttentionFunction, WindowAdjacency
from oracle import attention as OA
from oracle import graph as OG
from tests._strategies import windows
from tests._util import TOL, assert_close

pytestmark = pytest.mark.gpu

GPU_PROPS = settings(max_examples=80, deadline=None, database=None, derandomize=True,
                     suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])


@GPU_PROPS
@given(win=windows(max_n=300, max_degree=24.0, max_related=200),
       H=st.sampled_from([1, 2, 3, 8, 32]), d=st.sampled_from([8, 16, 24, 32, 64]),
       dtype=st.sampled_from([torch.float32, torch.bfloat16]),
       chunk=st.sampled_from([4, 16, 64, 256]), small=st.sampled_from([0, 2, 8, 31]),
       qscale=st.sampled_from([0.5, 2.0]))
def test_random_windows_match_the_oracle(win, H, d, dtype, chunk, small, qscale):
    if H * d > 512:
        H = max(1, 512 // d)
    print(f"case {win.desc} H={H} d={d} {dtype} chunk={chunk} small={small}", flush=True)
    ei = win.edge_index
    eid = torch.from_numpy(ei).cuda()
    adj = WindowAdjacency(eid, win.n_q, win.n_k, chunk, small)
    # CSR, transposed CSR and work lists: bit for bit
    ref = OG.csr_from_coo(ei[0], ei[1], win.n_q, win.n_k)
    for n in ref:
        got = getattr(adj, n).cpu().numpy()[: ref[n].shape[0]]
        np.testing.assert_array_equal(got, ref[n], err_msg=f"{n}: {win.desc}")
    for side, rp in (("q", ref["rowptr"]), ("k", ref["t_rowptr"])):
        items, splits, packed = OG.work_items(rp, chunk, min(small, chunk - 1))
        for n, r in (("items_", items), ("splits_", splits), ("packed_", packed)):
            got = getattr(adj, n + side).cpu().numpy()[: r.shape[0]]
            np.testing.assert_array_equal(got, r, err_msg=f"{n}{side}: {win.desc}")
    # forward + backward against the oracle
    g = torch.Generator().manual_seed(H * 1000 + d)
    q = (torch.randn(win.n_q, H, d, generator=g) * qscale).to(dtype)
    k = torch.randn(win.n_k, H, d, generator=g).to(dtype)
    v = torch.randn(win.n_k, H, d, generator=g).to(dtype)
    go = torch.randn(win.n_q, H, d, generator=g).to(dtype)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    x, ns = SparseAttentionFunction.apply(qd, kd, vd, adj, float(d) ** 0.5, -5.0, 5.0, 1e-6)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    eic = torch.from_numpy(ei)
    want = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), eic, go.float(), H)
    got = {"x": x.detach(), "node_scores": ns, "dq": qd.grad, "dk": kd.grad, "dv": vd.grad}
    for name in ("x", "node_scores"):  # convex combinations and positive sums
        assert got[name].shape == want[name].shape, (name, win.desc)
        assert_close(got[name].float().cpu(), want[name].float(), dtype, f"{name}: {win.desc}")
    ref = dict(zip(("dq", "dk", "dv"), OA.sparse_backward_closed_form(q.float(), k.float(),
                                                                         v.float(), eic,
                                                                         go.float())))
    scale = _grad_term_scales(q.float(), k.float(), v.float(), eic, go.float())
    for name in ("dq", "dk", "dv"):
        assert got[name].shape == ref[name].shape, (name, win.desc)
        _assert_grad_close(got[name].double().cpu(), ref[name], scale[name], dtype,
                           f"{name}: {win.desc}")


def _grad_term_scales(q, k, v, edge_index, go):
    """The size of the terms each gradient sums, in float64: with
    t_e = p_e r_i (|G_i.V_j| + |D_i|) [lo <= a_e <= hi] (a bound on |da_e|),
    dQ_i ~ sum t_e |K_j| / s, dK_j ~ sum t_e |Q_i| / s, dV_j ~ sum p_e r_i |G_i|.
    A row whose weight sits on one edge has X_i close to V_j and
    dp = r G.(V_j - X_i) nearly cancels: its true gradient is tiny and any
    finite-precision result is rounding noise of the size of these terms."""
    q, k, v, g = (t.double() for t in (q, k, v, go))
    n_q, n_k, d = q.shape[0], k.shape[0], q.shape[-1]
    s = d ** 0.5
    j, i = edge_index[0].long(), edge_index[1].long()
    a = (k[j] * q[i]).sum(-1) / s
    p = torch.exp(a.clamp(OA.CLAMP_LO, OA.CLAMP_HI))
    inside = ((a >= OA.CLAMP_LO) & (a <= OA.CLAMP_HI)).double()
    z = torch.zeros(n_q, q.shape[1], dtype=torch.float64).index_add_(0, i, p)
    r = 1.0 / (z + OA.EPS)
    x = torch.zeros_like(q).index_add_(0, i, p.unsqueeze(-1) * v[j]) * r.unsqueeze(-1)
    dd = (g * x).sum(-1)
    t = p * r[i] * ((g[i] * v[j]).sum(-1).abs() + dd[i].abs()) * inside
    return {
        "dq": torch.zeros_like(q).index_add_(0, i, t.unsqueeze(-1) * k[j].abs() / s),
        "dk": torch.zeros(n_k, *q.shape[1:], dtype=torch.float64).index_add_(
            0, j, t.unsqueeze(-1) * q[i].abs() / s),
        "dv": torch.zeros(n_k, *q.shape[1:], dtype=torch.float64).index_add_(
            0, j, (p * r[i]).unsqueeze(-1) * g[i].abs()),
    }


def _assert_grad_close(ours, ref64, term_scale, dtype, what):
    """Normwise error within the path's tolerance of max(|ref|, |terms|) (the
    two agree for rows without cancellation), plus an elementwise guard on the
    same scale."""
    tol = TOL[dtype]
    denom = max(ref64.norm().item(), term_scale.norm().item())
    err = (ours - ref64).norm().item()
    assert err <= tol * denom or denom == 0 and err == 0, (
        f"{what}: error {err:.3e} > {tol:.0e} x {denom:.3e}")
    if ref64.numel():
        atol = 10 * tol * max(ref64.abs().max().item(), term_scale.abs().max().item())
        worst = (ours - ref64).abs().max().item()
        assert worst <= atol, f"{what}: max abs diff {worst:.3e} > {atol:.3e}"


@settings(max_examples=40, deadline=None, database=None, derandomize=True,
          suppress_health_check=[HealthCheck.too_slow])
@given(n_q=st.integers(1, 400), n_k=st.integers(1, 400), H=st.sampled_from([1, 2, 5]),
       d=st.sampled_from([8, 16, 24, 32, 64]),
       dtype=st.sampled_from([torch.float32, torch.bfloat16]),
       p=st.sampled_from([0.0, 0.0, 0.3]), seed=st.integers(0, 2**40))
def test_dense_random_sizes_match_the_oracle(n_q, n_k, H, d, dtype, p, seed):
    """Dense all-pairs attention at random sizes (tails of the 32-row tiles
    and 128-row stages on both sides), with and without dropout."""
    from neutrongt_amd import DenseAttentionFunction
    from tests._util import assert_parity

    print(f"case dense n_q={n_q} n_k={n_k} H={H} d={d} {dtype} p={p} seed={seed}", flush=True)
    g = torch.Generator().manual_seed(seed % (2**31))
    q, k, v = (torch.randn(n, H, d, generator=g).to(dtype) for n in (n_q, n_k, n_k))
    go = torch.randn(n_q, H, d, generator=g).to(dtype)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    x, ns = DenseAttentionFunction.apply(qd, kd, vd, float(d) ** 0.5, True, p, seed)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, p) if p > 0 else None
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float(), dropout_mult=mult)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(),
                            dtype=torch.float64, dropout_mult=mult)
    got = {"x": x.detach(), "node_scores": ns, "dq": qd.grad, "dk": kd.grad, "dv": vd.grad}
    for name in ("x", "node_scores"):
        assert got[name].shape == ref[name].shape, name
        assert_parity(got[name].float().cpu(), ref[name], ref64[name], dtype, name)
    scale = _dense_term_scales(q.float(), k.float(), v.float(), go.float(), float(d) ** 0.5,
                               mult)
    for name in ("dq", "dk", "dv"):
        assert got[name].shape == ref[name].shape, name
        _assert_grad_close(got[name].double().cpu(), ref64[name].double(), scale[name], dtype,
                           f"dense {name}")


def _dense_term_scales(q, k, v, go, scale, mult):
    """The size of the terms each dense gradient sums (float64): with
    dP = (G V^T) o M, D_i = sum_j P_ij dP_ij and t = P o (|dP| + |D|),
    dQ ~ scale t |K|, dK ~ scale t^T |Q|, dV ~ (P o M)^T |G|.  One key (or one
    dominant key) makes dS = P (dP - D) cancel to about zero: the kernels
    recompute P from the saved log-sum-exp and leave rounding noise of the
    terms' size there, where the restatement's exact P = 1 may cancel exactly."""
    q, k, v, g = (t.double() for t in (q, k, v, go))
    m = torch.ones(q.shape[1], q.shape[0], k.shape[0], dtype=torch.float64) if mult is None \
        else torch.as_tensor(mult, dtype=torch.float64)
    s = torch.einsum("ihc,jhc->hij", q * scale, k)
    p = torch.softmax(s, dim=-1)
    dp = torch.einsum("ihc,jhc->hij", g, v) * m
    dd = (p * dp).sum(-1, keepdim=True)
    t = p * (dp.abs() + dd.abs())
    return {
        "dq": scale * torch.einsum("hij,jhc->ihc", t, k.abs()),
        "dk": scale * torch.einsum("hij,ihc->jhc", t, q.abs()),
        "dv": torch.einsum("hij,ihc->jhc", p * m, g.abs()),
    }
