"""Pins the CPU oracle of the attention core (no GPU).

The restatement in oracle/attention.py is checked against forms that do not
share its op sequence: a float64 dense masked-matrix formula, hand-derived
gradients, torch.autograd.gradcheck, closed-form special cases and the
committed golden fixtures.
"""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as OA
from tests._util import random_coo, relerr

GOLDEN = Path(__file__).parent / "golden"


def _inputs(n_q, n_k, H, d, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n_q, H, d, generator=g, dtype=dtype)
    k = torch.randn(n_k, H, d, generator=g, dtype=dtype)
    v = torch.randn(n_k, H, d, generator=g, dtype=dtype)
    go = torch.randn(n_q, H, d, generator=g, dtype=dtype)
    return q, k, v, go


@pytest.mark.parametrize("n_q,n_k,H,d,E", [(40, 40, 4, 8, 300), (30, 55, 2, 16, 200),
                                           (64, 64, 8, 8, 1500)])
def test_sparse_forward_matches_bruteforce_fp64(n_q, n_k, H, d, E):
    ei = torch.from_numpy(random_coo(n_q, n_k, E, seed=n_q + E))
    q, k, v, _ = _inputs(n_q, n_k, H, d, seed=1)
    qf = torch.zeros(n_k, H, d, dtype=torch.float64)
    qf[:n_q] = q
    x, ns = OA.sparse_attention_bias(qf[None], k[None], v[None], ei, H)
    xb, zb = OA.sparse_bruteforce_fp64(q, k, v, ei)
    assert relerr(x[:n_q], xb) < 1e-12
    # node_scores = mean over heads of Z, length max(dst) + 1
    dst_end = int(ei[1].max()) + 1
    assert ns.shape == (dst_end,)
    assert relerr(ns, zb.mean(1)[:dst_end]) < 1e-12


def test_sparse_backward_autograd_matches_closed_form():
    n_q, n_k, H, d = 35, 50, 4, 8
    ei = torch.from_numpy(random_coo(n_q, n_k, 260, seed=7))
    q, k, v, go = _inputs(n_q, n_k, H, d, seed=3)
    # push some scores past the clamp so the mask matters
    q = q * 3.0
    res = OA.sparse_fwd_bwd(q, k, v, ei, go, H, dtype=torch.float64)
    dq, dk, dv = OA.sparse_backward_closed_form(q, k, v, ei, go)
    assert relerr(res["dq"], dq) < 1e-12
    assert relerr(res["dk"], dk) < 1e-12
    assert relerr(res["dv"], dv) < 1e-12


def test_sparse_gradcheck_fp64():
    n, H, d = 9, 2, 4
    ei = torch.from_numpy(random_coo(n, n, 30, seed=11))
    q, k, v, _ = _inputs(n, n, H, d, seed=5)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    f = lambda a, b, c: OA.sparse_attention_bias(a[None], b[None], c[None], ei, H)[0]
    assert torch.autograd.gradcheck(f, (q, k, v), eps=1e-6, atol=1e-7)


def test_sparse_special_cases():
    H, d = 2, 4
    n = 5
    q, k, v, _ = _inputs(n, n, H, d, seed=9)
    # row 0: single edge 3->0; row 1: empty; row 2: two edges with q = 0 (p = 1 each)
    ei = torch.tensor([[3, 1, 4], [0, 2, 2]])
    q2 = q.clone()
    q2[2] = 0
    x, ns = OA.sparse_attention_bias(q2[None], k[None], v[None], ei, H)
    a = (k[3] * q2[0]).sum(-1) / math.sqrt(d)
    p = torch.exp(a.clamp(-5, 5))
    torch.testing.assert_close(x[0], v[3] * (p / (p + 1e-6)).unsqueeze(-1), rtol=1e-12, atol=0)
    assert torch.all(x[1] == 0)
    torch.testing.assert_close(x[2], (v[1] + v[4]) / (2 + 1e-6), rtol=1e-12, atol=0)
    assert ns.shape == (3,) and ns[1] == 0 and abs(ns[2].item() - 2.0) < 1e-12
    # duplicate edges count twice
    ei_dup = torch.tensor([[3, 3], [0, 0]])
    xd, nsd = OA.sparse_attention_bias(q[None], k[None], v[None], ei_dup, H)
    torch.testing.assert_close(nsd[0], 2 * p.mean(), rtol=1e-12, atol=0)
    torch.testing.assert_close(xd[0], v[3] * (2 * p / (2 * p + 1e-6)).unsqueeze(-1), rtol=1e-12,
                               atol=0)


def test_clamp_boundary_gradient_is_inclusive():
    """a = +-5 exactly: torch.clamp's backward passes the gradient (mask is
    lo <= a <= hi); a planted exclusive mask must differ."""
    H, d = 1, 16  # scale = 4, exact in binary
    q = torch.zeros(3, H, d, dtype=torch.float64)
    k = torch.zeros(3, H, d, dtype=torch.float64)
    v = torch.randn(3, H, d, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    q[0, 0, 0] = 4.0
    k[1, 0, 0] = 5.0  # a = 20/4 = +5
    k[2, 0, 0] = -5.0  # a = -5
    ei = torch.tensor([[1, 2], [0, 0]])
    go = torch.randn(3, H, d, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    res = OA.sparse_fwd_bwd(q, k, v, ei, go, H, dtype=torch.float64)
    dq, dk, dv = OA.sparse_backward_closed_form(q, k, v, ei, go)
    assert relerr(res["dq"], dq) < 1e-10 and relerr(res["dk"], dk) < 1e-10
    assert res["dq"].abs().sum() > 0  # gradient flows at the boundary
    dq_excl, _, _ = OA.sparse_backward_closed_form(q, k, v, ei, go, lo=-5 + 1e-9, hi=5 - 1e-9)
    assert relerr(dq_excl, res["dq"]) > 1e-3


def test_max_subtraction_would_break_parity():
    """The reference has no max subtraction: eps sits outside a sum that is not
    rescaled, so a max-subtracted softmax changes low-degree rows."""
    H, d = 1, 4
    q = torch.full((1, H, d), -3.0, dtype=torch.float64)
    k = torch.full((2, H, d), 2.0, dtype=torch.float64)
    v = torch.randn(2, H, d, dtype=torch.float64)
    ei = torch.tensor([[0], [0]])
    qf = torch.zeros(2, H, d, dtype=torch.float64)
    qf[:1] = q
    x, _ = OA.sparse_attention_bias(qf[None], k[None], v[None], ei, H)
    p = math.exp(-5.0)  # clamped
    assert abs(x[0, 0, 0].item() - v[0, 0, 0].item() * p / (p + 1e-6)) < 1e-12
    # max-subtracted form gives p' = 1 -> v / (1 + 1e-6): relative change ~1.5e-4
    alt = v[0, 0, 0].item() / (1 + 1e-6)
    assert abs(alt - x[0, 0, 0].item()) / abs(x[0, 0, 0].item()) > 1e-4


@pytest.mark.parametrize("n_q,n_k,H,d", [(20, 20, 2, 8), (17, 33, 3, 4)])
def test_full_attention_matches_fp64(n_q, n_k, H, d):
    q, k, v, go = _inputs(n_q, n_k, H, d, seed=4)
    x, ns = OA.full_attention(q[None], k[None], v[None])
    xb, nsb = OA.full_attention_fp64(q, k, v)
    assert relerr(x[0], xb) < 1e-12 and relerr(ns, nsb) < 1e-12
    # x = softmax(sqrt(d) q k^T) v: check one row by hand
    for h in range(H):
        srow = (q[0, h] * math.sqrt(d)) @ k[:, h].T
        w = torch.softmax(srow, 0)
        torch.testing.assert_close(x[0, 0, h], w @ v[:, h], rtol=1e-12, atol=1e-14)


def test_full_attention_gradcheck_fp64():
    q, k, v, _ = _inputs(6, 7, 2, 4, seed=8)
    for t in (q, k, v):
        t.requires_grad_(True)
    f = lambda a, b, c: OA.full_attention(a[None], b[None], c[None])[0]
    assert torch.autograd.gradcheck(f, (q, k, v), eps=1e-6, atol=1e-7)


def test_naive_attention_hand_row():
    """The flash branch (graphormer_dist_node_level.py:100-105): softmax of
    q k^T / sqrt(d), the dropout multiplier applied to the probabilities with
    no renormalisation, then v.  One query row worked by hand: d = 4, so
    1/sqrt(d) = 1/2, and keys whose scores are 0, 1, 2, 3; key 1 dropped at
    p = 0.5 (kept keys scaled by 2)."""
    H, d = 1, 4
    q = torch.zeros(1, 1, H, d, dtype=torch.float64)
    q[0, 0, 0, 0] = 2.0
    k = torch.zeros(1, 4, H, d, dtype=torch.float64)
    v = torch.zeros(1, 4, H, d, dtype=torch.float64)
    for j in range(4):
        k[0, j, 0, 0] = float(j)       # s_j = 2 * j / 2 = j
        v[0, j, 0, :] = torch.tensor([1.0, float(j), float(j * j), -1.0])
    mult = np.array([[[2.0, 0.0, 2.0, 2.0]]])  # [H, n_q, n_k]
    x = OA.naive_attention(q, k, v, dropout_mult=mult)[0, 0, 0]
    z = sum(math.exp(j) for j in range(4))
    w = [math.exp(j) / z * m for j, m in zip(range(4), (2.0, 0.0, 2.0, 2.0))]
    want = [sum(w), sum(wj * j for j, wj in enumerate(w)), sum(wj * j * j for j, wj in enumerate(w)),
            -sum(w)]
    torch.testing.assert_close(x, torch.tensor(want, dtype=torch.float64), rtol=1e-13, atol=0)
    # a x sqrt(d) scale (full_attention's) gives scores 0, 4, 8, 12: far from the row above
    xs, _ = OA.full_attention(q, k, v, dropout_mult=mult)
    assert relerr(xs[0, 0, 0], torch.tensor(want)) > 0.1
    # without dropout the weights sum to one: x[0] == 1, x[3] == -1
    x0 = OA.naive_attention(q, k, v)[0, 0, 0]
    assert abs(x0[0].item() - 1.0) < 1e-15 and abs(x0[3].item() + 1.0) < 1e-15


@pytest.mark.parametrize("n_q,n_k,H,d,p", [(9, 13, 2, 8, 0.0), (12, 7, 3, 16, 0.5)])
def test_naive_attention_matches_fp64_form_and_gradcheck(n_q, n_k, H, d, p):
    """naive_attention equals the einsum form softmax((q / sqrt(d)) k^T) v with
    the same multiplier; its autograd backward passes gradcheck."""
    q, k, v, _ = _inputs(n_q, n_k, H, d, seed=n_q + d)
    mult = OA.dropout_multiplier(123, H, n_q, n_k, p) if p else None
    x = OA.naive_attention(q[None], k[None], v[None], dropout_mult=mult)[0]
    xb, _ = OA.full_attention_fp64(q, k, v, scale=1.0 / math.sqrt(d), dropout_mult=mult)
    assert relerr(x, xb) < 1e-12
    qs, ks, vs = (t[:5, :, :4].clone().requires_grad_(True) for t in (q, k, v))
    m = OA.dropout_multiplier(5, H, 5, 5, p) if p else None
    f = lambda a, b, c: OA.naive_attention(a[None], b[None], c[None], dropout_mult=m)
    assert torch.autograd.gradcheck(f, (qs, ks, vs), eps=1e-6, atol=1e-7)


def test_golden_fixtures_reproduce():
    files = sorted(GOLDEN.glob("attn_*.npz"))
    assert files, "golden fixtures missing (tests/golden/make_golden.py)"
    for f in files:
        z = np.load(f)
        kind = str(z["kind"])
        q, k, v, go = (torch.from_numpy(z[n]) for n in ("q", "k", "v", "go"))
        if kind == "sparse":
            ei = torch.from_numpy(z["edge_index"])
            res = OA.sparse_fwd_bwd(q, k, v, ei, go, q.shape[1], dtype=torch.float32)
        else:
            res = OA.full_fwd_bwd(q, k, v, go, dtype=torch.float32)
        for name in ("x", "node_scores", "dq", "dk", "dv"):
            assert relerr(res[name], torch.from_numpy(z[name])) < 1e-6, (f.name, name)
        # and against float64 forms that share none of the op sequence
        if kind == "sparse":
            xb, _ = OA.sparse_bruteforce_fp64(q, k, v, ei)
            dq, dk, dv = OA.sparse_backward_closed_form(q, k, v, ei, go)
            assert relerr(torch.from_numpy(z["dq"]), dq) < 1e-5
            assert relerr(torch.from_numpy(z["dk"]), dk) < 1e-5
            assert relerr(torch.from_numpy(z["dv"]), dv) < 1e-5
        else:
            xb, _ = OA.full_attention_fp64(q, k, v)
        assert relerr(torch.from_numpy(z["x"]), xb) < 1e-5


# ------------------------------------------------------- dense dropout masks
def test_mix32_is_a_bijection_on_a_block():
    """Odd multipliers and xor-shifts make lowbias32 invertible: 2^20
    consecutive inputs give 2^20 distinct words (a wrong shift or an even
    constant collides)."""
    x = np.arange(1 << 20, dtype=np.uint32) * np.uint32(2654435761)
    with np.errstate(over="ignore"):
        w = OA._mix32(x)
    assert np.unique(w).size == x.size
    assert OA._mix32(np.zeros(1, np.uint32))[0] == 0


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_dropout_mask_keep_rate_and_values(p):
    H, n_q, n_k = 3, 257, 300
    m = OA.dropout_multiplier(42, H, n_q, n_k, p)
    thr, scale = OA.dropout_params(p)
    assert set(np.unique(m).tolist()) <= {0.0, float(scale)}
    assert abs(float(scale) - 1.0 / (1.0 - p)) < 1e-6 / (1.0 - p)
    keep = (m > 0).mean()
    n = m.size
    sigma = math.sqrt(p * (1 - p) / n)
    assert abs(keep - (1 - thr / 65536.0)) < 5 * sigma
    assert abs(thr / 65536.0 - p) <= 1.0 / 65536


def test_dropout_mask_limits():
    assert np.all(OA.dropout_multiplier(7, 2, 20, 21, 0.0) == 1.0)
    assert np.all(OA.dropout_multiplier(7, 2, 20, 21, 1.0) == 0.0)


def test_dropout_mask_independence():
    """Neighbouring keys (the two halves of one word), neighbouring queries,
    heads and seeds are uncorrelated (|r| < 0.01 on 2^18 pairs, sigma ~ 0.002)."""
    m = (OA.dropout_multiplier(99, 2, 512, 512, 0.5) > 0).astype(np.float64)
    m2 = (OA.dropout_multiplier(100, 2, 512, 512, 0.5) > 0).astype(np.float64)

    def corr(a, b):
        return float(np.corrcoef(a.ravel(), b.ravel())[0, 1])

    assert abs(corr(m[0, :, 0::2], m[0, :, 1::2])) < 0.01   # same word
    assert abs(corr(m[0, :-1, :], m[0, 1:, :])) < 0.01      # next query
    assert abs(corr(m[0, :, :-2], m[0, :, 2:])) < 0.01      # next word
    assert abs(corr(m[0], m[1])) < 0.01                     # next head
    assert abs(corr(m, m2)) < 0.01                          # next seed


def test_dropout_is_unbiased_and_matches_fp64():
    """Averaged over seeds, dropout(P) v tends to P v (the 1/(1-p) scale
    matches the keep rate); one masked forward agrees with the float64 form."""
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, n, 2, 8, generator=g) for n in (6, 9, 9))
    base, _ = OA.full_attention(q, k, v)
    acc = torch.zeros_like(base)
    n_seeds = 400
    for s in range(n_seeds):
        mult = OA.dropout_multiplier(1000 + s, 2, 6, 9, 0.5)
        x, _ = OA.full_attention(q, k, v, dropout_mult=mult)
        acc += x
        if s == 0:
            x64, _ = OA.full_attention_fp64(q, k, v, dropout_mult=mult)
            assert torch.allclose(x[0], x64.float(), rtol=1e-5, atol=1e-6)
    mean = acc / n_seeds
    # measured: max 0.15, mean 0.028 at the right scale; a scale 10 % off
    # gives mean 0.095, so the bounds separate the two
    assert (mean - base).abs().max().item() < 0.3
    assert (mean - base).abs().mean().item() < 0.06


def test_sparse_bias_added_after_clamp_and_its_gradient():
    """The optional per-pair bias (graphormer_dist_node_level.py:81-84): a
    dense [1, H, N, N] tensor indexed [0, h, src, dst] and added to each
    edge's score after the clamp.  Worked with explicit float64 loops on a
    3-node window with a duplicate edge and a clamped edge: the output, the
    bias's gradient (the score gradient of every edge, not masked by the
    clamp, summed over the duplicate pair) and dQ (masked by the clamp).
    bias[0, 1, 0] != bias[0, 0, 1], so a transposed index fails."""
    H, d, n = 1, 2, 3
    src = np.array([0, 1, 1, 2, 0])
    dst = np.array([0, 0, 0, 0, 1])
    q = np.array([[[1.0, 0.5]], [[0.25, -1.0]], [[0.0, 0.0]]])           # [n, H, d]
    k = np.array([[[0.5, 1.0]], [[8.0, 6.0]], [[-1.0, 0.5]]])            # key 1: a > 5 at query 0
    v = np.array([[[1.0, 2.0]], [[-1.0, 0.5]], [[0.25, -2.0]]])
    g = np.array([[[0.5, -1.0]], [[2.0, 1.0]], [[0.0, 0.0]]])
    bias = np.zeros((H, n, n))
    bias[0, 1, 0], bias[0, 0, 1], bias[0, 0, 0], bias[0, 2, 0] = 0.3, -0.7, 0.1, -0.2
    sq = math.sqrt(d)
    a = np.array([k[j, 0] @ q[i, 0] / sq for j, i in zip(src, dst)])
    assert a[1] > 5 and a[2] > 5
    s = np.clip(a, -5.0, 5.0) + np.array([bias[0, j, i] for j, i in zip(src, dst)])
    p = np.exp(s)
    Z = np.zeros(n)
    x = np.zeros((n, d))
    for e, (j, i) in enumerate(zip(src, dst)):
        Z[i] += p[e]
        x[i] += p[e] * v[j, 0]
    x = x / (Z + 1e-6)[:, None]
    r = 1.0 / (Z + 1e-6)
    D = np.array([g[i, 0] @ x[i] for i in range(n)])
    dscore = np.array([p[e] * r[i] * (g[i, 0] @ v[j, 0] - D[i]) for e, (j, i) in enumerate(zip(src, dst))])
    dbias = np.zeros((H, n, n))
    for e, (j, i) in enumerate(zip(src, dst)):
        dbias[0, j, i] += dscore[e]
    da = np.where((a >= -5) & (a <= 5), dscore, 0.0)
    dq = np.zeros((n, d))
    for e, (j, i) in enumerate(zip(src, dst)):
        dq[i] += da[e] * k[j, 0] / sq
    ei = torch.from_numpy(np.stack([src, dst]))
    T = lambda t: torch.from_numpy(t)
    ref = OA.sparse_fwd_bwd(T(q), T(k), T(v), ei, T(g), H, dtype=torch.float64, attn_bias=T(bias))
    np.testing.assert_allclose(ref["x"][:, 0].numpy(), x, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ref["dbias"].numpy(), dbias, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ref["dq"][:, 0].numpy(), dq, rtol=1e-12, atol=1e-14)
    assert dbias[0, 1, 0] != 0.0  # the clamped duplicate pair still passes gradient to its bias
    # the same with the bias transposed differs
    bad = OA.sparse_fwd_bwd(T(q), T(k), T(v), ei, T(g), H, dtype=torch.float64,
                            attn_bias=T(bias.transpose(0, 2, 1).copy()))
    assert np.abs(bad["x"][:, 0].numpy() - x).max() > 1e-3


def test_full_attention_bias_pruning_mask_by_hand():
    """full_attention's optional terms (graphormer_dist_node_level.py:51-58):
    z = (q sqrt(d)) k^T + attn_bias + pruning_mask, then masked_fill(mask,
    -1e9), softmax over keys.  One head, 2 queries, 3 keys worked in float64:
    query 0 has key 2 masked; query 1 has every key masked (the reference then
    weighs all keys equally).  The biases' gradient is dS, zero where masked;
    the node scores ignore both terms."""
    H, d = 1, 2
    q = torch.tensor([[[0.5, -1.0]], [[1.0, 0.25]]], dtype=torch.float64)      # [2, H, d]
    k = torch.tensor([[[1.0, 0.5]], [[-0.5, 1.0]], [[2.0, 0.0]]], dtype=torch.float64)
    v = torch.tensor([[[1.0, 0.0]], [[0.0, 2.0]], [[-1.0, 1.0]]], dtype=torch.float64)
    g = torch.tensor([[[1.0, -0.5]], [[0.5, 2.0]]], dtype=torch.float64)
    ab = torch.tensor([[[[0.1, -0.2, 0.3], [0.0, 0.4, -0.1]]]], dtype=torch.float64)
    pm = torch.tensor([[[[-1.0, 0.0, 0.5], [0.2, 0.0, 0.0]]]], dtype=torch.float64)
    mask = torch.tensor([[False, False, True], [True, True, True]])
    sq = math.sqrt(d)
    Q, K, V, G = q[:, 0].numpy(), k[:, 0].numpy(), v[:, 0].numpy(), g[:, 0].numpy()
    S = (Q * sq) @ K.T
    Z = S + ab[0, 0].numpy() + pm[0, 0].numpy()
    Z = np.where(mask.numpy(), -1e9, Z)
    P = np.exp(Z - Z.max(1, keepdims=True))
    P /= P.sum(1, keepdims=True)
    X = P @ V
    dP = G @ V.T
    dS = P * (dP - (P * dP).sum(1, keepdims=True))
    dZ = np.where(mask.numpy(), 0.0, dS)
    ref = OA.full_fwd_bwd(q, k, v, g, dtype=torch.float64, attn_bias=ab, pruning_mask=pm,
                          mask=mask)
    np.testing.assert_allclose(ref["x"][:, 0].numpy(), X, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(X[1], V.mean(0), rtol=1e-12)  # all keys masked: equal weights
    np.testing.assert_allclose(ref["dbias"][0, 0].numpy(), dZ, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ref["dpruning"][0, 0].numpy(), dZ, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ref["node_scores"].numpy(), np.abs(S).sum(0), rtol=1e-12)
    np.testing.assert_allclose(ref["dq"][:, 0].numpy(), sq * (dZ @ K), rtol=1e-12, atol=1e-14)
