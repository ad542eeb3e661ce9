"""GPU parity of the dense full-window attention (forward + backward)."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from neutrongt_amd import CoreAttention, dense_attention
from neutrongt_amd import synthetic as S
from oracle import attention as OA
from tests._util import TOL, assert_close, assert_parity, relerr

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _run(q, k, v, go):
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    x, ns = dense_attention(qd, kd, vd)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    return {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
            "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}


def _qkv(n_q, n_k, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(n, H, d, generator=g).to(dtype) for n in (n_q, n_k, n_k, n_q))


@pytest.mark.parametrize("n_q,n_k,H,d,dtype", [
    (70, 70, 2, 8, torch.float32), (130, 90, 3, 16, torch.float32), (64, 200, 2, 24, torch.float32),
    (50, 77, 1, 32, torch.float32), (40, 40, 2, 64, torch.float32),
    (100, 100, 8, 8, torch.bfloat16), (96, 150, 4, 16, torch.bfloat16),
    (60, 61, 2, 24, torch.bfloat16), (70, 45, 3, 32, torch.bfloat16),
    (33, 47, 2, 64, torch.bfloat16), (1, 1, 1, 8, torch.bfloat16), (130, 33, 2, 8, torch.bfloat16)])
def test_dense_parity(n_q, n_k, H, d, dtype):
    _say(f"case dense n_q={n_q} n_k={n_k} H={H} d={d} {dtype}")
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=n_q + d)
    res = _run(q, k, v, go)
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float())
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64)
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert res[name].shape == ref[name].shape
        assert_parity(res[name].float(), ref[name], ref64[name], dtype, name)


def test_dense_golden():
    for f in sorted((Path(__file__).parent / "golden").glob("attn_dense_*.npz")):
        _say(f"case golden {f.name}")
        z = np.load(f)
        q, k, v, go = (torch.from_numpy(z[n]) for n in ("q", "k", "v", "go"))
        res = _run(q, k, v, go)
        for name in ("x", "node_scores", "dq", "dk", "dv"):
            assert_close(res[name], torch.from_numpy(z[name]), torch.float32, f"{f.name}:{name}")


def test_dense_module_drop_in():
    _say("case dense module")
    H, d, n = 2, 8, 50
    mod = CoreAttention(H * d, 0.0, H).cuda()
    q, k, v, go = _qkv(n, n, H, d, torch.float32, seed=5)
    x, score = mod(q[None].cuda(), k[None].cuda(), v[None].cuda(), None, None, "full")
    assert x.shape == (1, n, H * d)
    ref = OA.full_fwd_bwd(q, k, v, go)
    assert_close(x[0].view(n, H, d).cpu(), ref["x"], torch.float32, "x")
    assert_close(score.cpu(), ref["node_scores"], torch.float32, "score")
    mod.att_dropout.p = 0.5
    with pytest.raises(NotImplementedError):
        mod(q[None].cuda(), k[None].cuda(), v[None].cuda(), None, None, "full")


def test_dense_full_size_sampled_rows_and_invariants():
    """16,000-node all-pairs window (H=8, d=8, bf16): sampled query rows against
    the float64 row formula, column scores against a chunked CPU sum, and the
    size-independent identities <dQ,Q> = <dK,K>, sum_j dV_j = sum_i G_i."""
    cfg = S.CONFIGS["dense_slim"]
    _say(f"case dense full-size n={cfg.n_q}")
    q, k, v, go = S.make_qkv(cfg, cfg.n_q)
    res = _run(q, k, v, go)
    n, H, d = cfg.n_q, cfg.n_heads, cfg.head_dim
    sc = math.sqrt(d)
    qd, kd, vd, gd = (t.double() for t in (q, k, v, go))
    rows = np.random.default_rng(1).choice(n, 48, replace=False)
    for h in range(H):
        s = (qd[rows, h] * sc) @ kd[:, h].T  # [48, n]
        p = torch.softmax(s, -1)
        x = p @ vd[:, h]
        dp = gd[rows, h] @ vd[:, h].T
        dd = (gd[rows, h] * x).sum(-1, keepdim=True)
        dq = sc * (p * (dp - dd)) @ kd[:, h]
        assert relerr(res["x"][rows, h], x) < TOL[cfg.dtype]
        assert relerr(res["dq"][rows, h], dq) < TOL[cfg.dtype]
    ns = torch.zeros(n, dtype=torch.float64)
    for h in range(H):
        for c in range(0, n, 2000):
            ns += ((qd[c:c + 2000, h] * sc) @ kd[:, h].T).abs().sum(0)
    ns /= H
    assert relerr(res["node_scores"], ns) < TOL[cfg.dtype]
    lhs = (res["dq"].double() * qd).sum().item()
    rhs = (res["dk"].double() * kd).sum().item()
    assert abs(lhs - rhs) / max(abs(lhs), abs(rhs)) < 10 * TOL[cfg.dtype]
    assert relerr(res["dv"].double().sum(0), gd.sum(0)) < 10 * TOL[cfg.dtype]
