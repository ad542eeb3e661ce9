"""The sparse backward's two ways of handing each edge's score gradient to the
query-major pass: read from the workspace (written by the key-major pass), or
recomputed from the edge's K and V rows, chosen for windows with at least 32
edges per key row.  Both must give the oracle's result, and the same bits."""
import numpy as np
import pytest
import torch

from neutrongt_amd import SparseAttentionFunction, WindowAdjacency
from oracle import attention as OA
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _qkv(n_q, n_k, H, d, dtype, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(n_q, H, d, generator=g) * scale).to(dtype)
    k = torch.randn(n_k, H, d, generator=g).to(dtype)
    v = torch.randn(n_k, H, d, generator=g).to(dtype)
    go = torch.randn(n_q, H, d, generator=g).to(dtype)
    return q, k, v, go


def _dense_reuse_coo(n_q, n_k, per_key, seed, hub=0):
    """About per_key edges per key row (duplicates allowed), every query with
    at least one edge, plus an optional query hub of degree `hub`."""
    rng = np.random.default_rng(seed)
    E = per_key * n_k
    src = np.concatenate([rng.integers(0, n_k, E), np.arange(n_q) % n_k,
                          rng.integers(0, n_k, hub)])
    dst = np.concatenate([rng.integers(0, n_q, E), np.arange(n_q), np.zeros(hub, np.int64)])
    return np.stack([src, dst]).astype(np.int64)


def _run(q, k, v, ei, go, chunk, small, n_main=None):
    n_q, n_k = q.shape[0], k.shape[0]
    n_main = n_k if n_main is None else n_main
    qd = q.cuda().requires_grad_(True)
    kd = k[:n_main].cuda().requires_grad_(True)
    vd = v[:n_main].cuda().requires_grad_(True)
    kx = k[n_main:].cuda() if n_main < n_k else None
    vx = v[n_main:].cuda() if n_main < n_k else None
    adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n_q, n_k, chunk, small, tiled=False)
    x, ns = SparseAttentionFunction.apply(qd, kd, vd, adj, float(q.shape[-1]) ** 0.5, -5.0, 5.0,
                                          1e-6, kx, vx)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    return {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
            "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}


CASES = [
    # n_q, n_k, n_main, H, d, dtype, per_key, hub, chunk, small
    (400, 96, 96, 8, 16, torch.bfloat16, 40, 0, 128, 16),
    (300, 64, 64, 8, 8, torch.float32, 48, 900, 64, 16),
    (256, 80, 80, 32, 24, torch.bfloat16, 36, 700, 128, 32),
    (200, 72, 60, 4, 32, torch.float32, 40, 500, 32, 8),  # keys in two buffers
    (160, 40, 40, 2, 64, torch.bfloat16, 64, 300, 64, 4),
]


@pytest.mark.parametrize("n_q,n_k,n_main,H,d,dtype,per_key,hub,chunk,small", CASES)
def test_recompute_matches_oracle_and_the_workspace_path(monkeypatch, n_q, n_k, n_main, H, d,
                                                         dtype, per_key, hub, chunk, small):
    _say(f"case recompute n_q={n_q} n_k={n_k} n_main={n_main} H={H} d={d} {dtype} "
         f"per_key={per_key} hub={hub} chunk={chunk} small={small}")
    ei = _dense_reuse_coo(n_q, n_k, per_key, seed=n_q + H, hub=hub)
    assert ei.shape[1] >= 32 * n_k  # the default picks the recomputation here
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=H * 7 + d)
    monkeypatch.delenv("NGT_DQ_RECOMPUTE", raising=False)
    default = _run(q, k, v, ei, go, chunk, small, n_main)
    monkeypatch.setenv("NGT_DQ_RECOMPUTE", "1")
    recomputed = _run(q, k, v, ei, go, chunk, small, n_main)
    monkeypatch.setenv("NGT_DQ_RECOMPUTE", "0")
    stored = _run(q, k, v, ei, go, chunk, small, n_main)
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert torch.equal(recomputed[name], stored[name]), name
        assert torch.equal(default[name], recomputed[name]), name
    ref = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), torch.from_numpy(ei), go.float(), H,
                            dtype=torch.float32)
    ref["dk"], ref["dv"] = ref["dk"][:n_main], ref["dv"][:n_main]
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert_close(default[name].float(), ref[name].float(), dtype, f"recompute:{name}")


def test_recompute_forced_on_a_low_reuse_window_gives_the_same_bits(monkeypatch):
    """Few edges per key row (the default reads the workspace): forcing the
    recomputation changes no bit of dQ (dK/dV and the forward are untouched)."""
    n_q = n_k = 500
    rng = np.random.default_rng(3)
    ei = np.stack([rng.integers(0, n_k, 4000), rng.integers(0, n_q, 4000)]).astype(np.int64)
    q, k, v, go = _qkv(n_q, n_k, 8, 16, torch.bfloat16, seed=9)
    monkeypatch.setenv("NGT_DQ_RECOMPUTE", "0")
    a = _run(q, k, v, ei, go, 64, 8)
    monkeypatch.setenv("NGT_DQ_RECOMPUTE", "1")
    b = _run(q, k, v, ei, go, 64, 8)
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert torch.equal(a[name], b[name]), name


def test_nontemporal_score_gradient_stores_give_the_same_bits(monkeypatch):
    """The key-major pass writes the score gradients with non-temporal stores
    when they are too large to stay cached (GPH_Large); forcing either store
    kind on a small window changes no bit, and both match the oracle."""
    n_q, n_k, H, d = 400, 450, 8, 16
    rng = np.random.default_rng(11)
    src = np.concatenate([rng.integers(0, n_k, 5000), np.full(700, 3)])
    dst = np.concatenate([rng.integers(0, n_q, 5000), rng.integers(0, n_q, 700)])
    ei = np.stack([src, dst]).astype(np.int64)
    q, k, v, go = _qkv(n_q, n_k, H, d, torch.bfloat16, seed=12)
    monkeypatch.setenv("NGT_DQ_RECOMPUTE", "0")
    monkeypatch.setenv("NGT_DS_NT", "0")
    a = _run(q, k, v, ei, go, 64, 16)
    monkeypatch.setenv("NGT_DS_NT", "1")
    b = _run(q, k, v, ei, go, 64, 16)
    ref = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), torch.from_numpy(ei), go.float(), H,
                            dtype=torch.float32)
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert torch.equal(a[name], b[name]), name
        assert_close(b[name].float(), ref[name].float(), torch.bfloat16, f"nt:{name}")


@pytest.mark.parametrize("H,d,dtype,n_main", [(8, 8, torch.float32, None),
                                              (8, 16, torch.bfloat16, 380),
                                              (32, 24, torch.bfloat16, None),
                                              (2, 64, torch.float32, None)])
def test_rowstat_folded_into_the_key_major_pass_gives_the_same_bits(monkeypatch, H, d, dtype,
                                                                    n_main):
    """On small windows the key-major pass forms each query's {r, r D} from
    its out row and rinv itself (no k_rowstat launch), with k_rowstat's
    arithmetic: forcing the fold on and off changes no bit; split, medium and
    packed key rows; keys in one or two buffers."""
    _say(f"case rowstat fold H={H} d={d} {dtype} n_main={n_main}")
    n_q, n_k = 420, 450
    rng = np.random.default_rng(H + d)
    src = np.concatenate([rng.integers(0, n_k, 5000), np.full(700, 3), np.full(300, n_k - 2)])
    dst = np.concatenate([rng.integers(0, n_q, 5000), rng.integers(0, n_q, 700),
                          rng.integers(0, n_q, 300)])
    ei = np.stack([src, dst]).astype(np.int64)
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=13)
    monkeypatch.setenv("NGT_DQ_RECOMPUTE", "0")
    monkeypatch.setenv("NGT_FOLD_ROWSTAT", "0")
    a = _run(q, k, v, ei, go, 64, 8, n_main=n_main)
    monkeypatch.setenv("NGT_FOLD_ROWSTAT", "1")
    b = _run(q, k, v, ei, go, 64, 8, n_main=n_main)
    ref = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), torch.from_numpy(ei), go.float(), H,
                            dtype=torch.float32)
    if n_main is not None:
        ref["dk"], ref["dv"] = ref["dk"][:n_main], ref["dv"][:n_main]
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert torch.equal(a[name], b[name]), name
        assert_close(b[name].float(), ref[name].float(), dtype, f"fold:{name}")
