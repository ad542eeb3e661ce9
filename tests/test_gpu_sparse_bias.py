"""GPU parity of the sparse path with the reference's optional per-pair bias
(attn_bias, graphormer_dist_node_level.py:81-84) against the oracle, through
the C ABI: output, node scores, dQ/dK/dV and the bias's own gradient."""
import numpy as np
import pytest
import torch

from neutrongt_amd import CoreAttention, SparseAttentionBiasFunction, WindowAdjacency, sparse_attention
from oracle import attention as OA
from tests._util import TOL, assert_close, hub_coo, random_coo

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _inputs(n_q, n_k, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q, go = (torch.randn(n_q, H, d, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(n_k, H, d, generator=g).to(dtype) for _ in range(2))
    bias = torch.randn(H, n_k, n_q, generator=g) * 0.5
    return q, k, v, go, bias


def _check(res, ref, dtype, what):
    for name in ("x", "node_scores", "dq", "dk", "dv", "dbias"):
        assert res[name].shape == ref[name].shape, (what, name, res[name].shape, ref[name].shape)
        assert_close(res[name].float(), ref[name].float(), dtype, f"{what}:{name}")


def _run(q, k, v, go, bias, ei, chunk, small, n_main=None):
    n_q, n_k = q.shape[0], k.shape[0]
    n_main = n_k if n_main is None else n_main
    qd = q.cuda().requires_grad_(True)
    kd = k[:n_main].cuda().requires_grad_(True)
    vd = v[:n_main].cuda().requires_grad_(True)
    kx = k[n_main:].cuda() if n_main < n_k else None
    vx = v[n_main:].cuda() if n_main < n_k else None
    bd = bias.cuda().requires_grad_(True)
    adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n_q, n_k, chunk, small)
    x, ns = SparseAttentionBiasFunction.apply(qd, kd, vd, bd, adj, float(q.shape[-1]) ** 0.5, -5.0,
                                              5.0, 1e-6, kx, vx)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    return {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
            "dk": kd.grad.cpu(), "dv": vd.grad.cpu(), "dbias": bd.grad.cpu()}


@pytest.mark.parametrize("n_q,n_k,H,d,dtype,chunk,small,hub", [
    (200, 200, 8, 8, torch.float32, 256, 4, False),
    (150, 230, 4, 16, torch.float32, 32, 0, True),
    (180, 180, 32, 24, torch.bfloat16, 64, 8, True),
    (120, 160, 8, 64, torch.bfloat16, 256, 2, False),
])
def test_sparse_bias_matches_oracle(n_q, n_k, H, d, dtype, chunk, small, hub):
    _say(f"case bias n_q={n_q} n_k={n_k} H={H} d={d} {dtype} chunk={chunk} hub={hub}")
    ei = hub_coo(n_q, n_k, 700, seed=8) if hub else random_coo(n_q, n_k, 10 * n_q, seed=9)
    q, k, v, go, bias = _inputs(n_q, n_k, H, d, dtype, seed=n_q + d)
    ref = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), torch.from_numpy(ei), go.float(), H,
                            attn_bias=bias)
    res = _run(q, k, v, go, bias, ei, chunk, small)
    _check(res, ref, dtype, "bias")


def test_sparse_bias_duplicate_edges_sum_in_order():
    """Every edge repeated 3 times: the bias of each pair gets the sum of its
    three score gradients, and two runs give identical bits (fixed order)."""
    _say("case bias duplicates")
    n, H, d = 100, 4, 8
    base = random_coo(n, n, 600, seed=12)
    ei = np.concatenate([base, base, base], axis=1)
    q, k, v, go, bias = _inputs(n, n, H, d, torch.float32, seed=13)
    ref = OA.sparse_fwd_bwd(q, k, v, torch.from_numpy(ei), go, H, attn_bias=bias)
    a = _run(q, k, v, go, bias, ei, 16, 2)
    b = _run(q, k, v, go, bias, ei, 16, 2)
    _check(a, ref, torch.float32, "bias dup")
    for name in a:
        assert torch.equal(a[name], b[name]), name


def test_sparse_bias_with_extra_key_rows():
    """Key rows from a second buffer (related keys): the bias covers all
    N_k = N_main + R keys; the extra rows get no K/V gradient."""
    _say("case bias ext")
    n_q, n_main, R, H, d = 160, 160, 70, 8, 16
    n_k = n_main + R
    rng = np.random.default_rng(14)
    ei = np.stack([rng.integers(0, n_k, 1800), rng.integers(0, n_q, 1800)]).astype(np.int64)
    q, k, v, go, bias = _inputs(n_q, n_k, H, d, torch.float32, seed=15)
    ref = OA.sparse_fwd_bwd(q, k, v, torch.from_numpy(ei), go, H, attn_bias=bias)
    res = _run(q, k, v, go, bias, ei, 64, 4, n_main=n_main)
    ref["dk"], ref["dv"] = ref["dk"][:n_main], ref["dv"][:n_main]
    _check(res, ref, torch.float32, "bias ext")


def test_sparse_bias_without_gradient_and_zero_bias():
    """A bias that needs no gradient takes the same path; an all-zero bias
    reproduces the bias-free outputs bit for bit (the add is exact)."""
    _say("case bias zero")
    n, H, d = 180, 8, 8
    ei = torch.from_numpy(random_coo(n, n, 1500, seed=16)).cuda()
    g = torch.Generator().manual_seed(17)
    q, k, v, go = (torch.randn(n, H, d, generator=g).cuda() for _ in range(4))
    x0, ns0 = sparse_attention(q, k, v, ei)
    zero = torch.zeros(1, H, n, n, device="cuda")
    x1, ns1 = sparse_attention(q, k, v, ei, attn_bias=zero)
    assert torch.equal(x0, x1) and torch.equal(ns0, ns1)


def test_core_attention_sparse_with_attn_bias():
    """CoreAttention.forward(attn_type='sparse', attn_bias=[1, H, N, N]) as
    the reference's struct_enc path calls it, against the oracle."""
    _say("case bias module")
    n, H, d = 150, 4, 16
    ei = random_coo(n, n, 1200, seed=18)
    q, k, v, go, bias = _inputs(n, n, H, d, torch.float32, seed=19)
    m = CoreAttention(H * d, 0.0, H).cuda()
    qd, kd, vd = (t.cuda().unsqueeze(0).requires_grad_(True) for t in (q, k, v))
    ab = bias.unsqueeze(0).cuda().requires_grad_(True)
    x, score = m(qd, kd, vd, attn_bias=ab, edge_index=torch.from_numpy(ei).cuda(),
                 attn_type="sparse")
    x.backward(go.reshape(1, n, H * d).cuda())
    ref = OA.sparse_fwd_bwd(q, k, v, torch.from_numpy(ei), go, H, attn_bias=bias)
    assert_close(x.detach().cpu().view(n, H, d), ref["x"], torch.float32, "module x")
    assert_close(score.cpu(), ref["node_scores"], torch.float32, "module score")
    assert_close(ab.grad.cpu()[0], ref["dbias"], torch.float32, "module dbias")
    assert_close(qd.grad.cpu()[0], ref["dq"], torch.float32, "module dq")


def test_sparse_bias_shape_is_checked():
    n, H, d = 40, 2, 8
    ei = torch.from_numpy(random_coo(n, n, 200, seed=20)).cuda()
    q = torch.randn(n, H, d, device="cuda")
    with pytest.raises(ValueError):
        sparse_attention(q, q, q, ei, attn_bias=torch.zeros(1, H, n - 1, n, device="cuda"))
    with pytest.raises(ValueError):
        sparse_attention(q, q, q, ei, attn_bias=torch.zeros(1, H + 1, n, n, device="cuda"))
