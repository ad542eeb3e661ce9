"""The tiled sparse kernels (dense windows: a block of rows sweeps column
blocks staged in LDS) against the oracle, through the C ABI, with the tiled
path forced on (NGT_TILED=1) and off (=0) on the same windows: output, node
scores, dQ, dK and dV within the path's tolerance either way; the tiled path
bitwise reproducible; related keys served from a second buffer; the rows'
degree orders bit-exact (checked with the CSR in test_gpu_sparse.py)."""
import numpy as np
import pytest
import torch

from neutrongt_amd import AdjacencyCache, SparseAttentionFunction, WindowAdjacency, sparse_attention
from oracle import attention as OA
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _dense_window(n_q, n_k, density, seed, hub=True, related=0):
    """Uniform edges over the window's own n_q x n_q pairs at `density`, a
    query hub row and a key hub (most of the window), empty last rows, and
    `related` extra keys per query among the columns n_q .. n_k-1."""
    rng = np.random.default_rng(seed)
    n_sw = min(n_q, n_k)
    E = int(density * n_q * n_sw)
    src = [rng.integers(0, n_sw, E)]
    dst = [rng.integers(0, max(1, n_q - n_q // 8), E)]  # the last rows stay empty
    if hub:
        src += [rng.integers(0, n_sw, 3 * n_sw // 4), np.full(n_q // 2, 1)]
        dst += [np.zeros(3 * n_sw // 4, np.int64), rng.integers(0, n_q, n_q // 2)]
    if related and n_k > n_q:
        src.append(rng.integers(n_q, n_k, related * n_q))
        dst.append(np.repeat(np.arange(n_q), related))
    return np.stack([np.concatenate(src), np.concatenate(dst)]).astype(np.int64)


def _qkv(n_q, n_k, H, d, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(n_q, H, d, generator=g) * scale).to(dtype)
    k = torch.randn(n_k, H, d, generator=g).to(dtype)
    v = torch.randn(n_k, H, d, generator=g).to(dtype)
    go = torch.randn(n_q, H, d, generator=g).to(dtype)
    return q, k, v, go


def _run(q, k, v, ei, go, n_main=None):
    """fwd + bwd with a fresh adjacency; key rows >= n_main from a second buffer."""
    n_main = k.shape[0] if n_main is None else n_main
    qd = q.cuda().requires_grad_(True)
    kd = k[:n_main].cuda().requires_grad_(True)
    vd = v[:n_main].cuda().requires_grad_(True)
    kv_ext = (k[n_main:].cuda(), v[n_main:].cuda()) if n_main < k.shape[0] else None
    x, ns = sparse_attention(qd, kd, vd, torch.from_numpy(ei).cuda(), cache=AdjacencyCache(),
                             kv_ext=kv_ext)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    return {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
            "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}


def _check(res, q, k, v, ei, go, H, dtype, what, n_main=None):
    ref = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), torch.from_numpy(ei), go.float(), H,
                            dtype=torch.float32)
    if n_main is not None:
        ref["dk"], ref["dv"] = ref["dk"][:n_main], ref["dv"][:n_main]
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert res[name].shape == ref[name].shape, (what, name, res[name].shape, ref[name].shape)
        assert_close(res[name].float(), ref[name].float(), dtype, f"{what}:{name}")


CASES = [
    # n_q, n_k, H, d, density, dtype
    (300, 300, 8, 16, 0.10, torch.bfloat16),
    (260, 260, 8, 8, 0.08, torch.float32),
    (200, 200, 4, 32, 0.10, torch.float32),
    (150, 150, 2, 64, 0.12, torch.float32),
    (170, 170, 3, 8, 0.10, torch.float32),   # 3 heads: one group of 3
    (220, 220, 12, 24, 0.06, torch.bfloat16),  # 3 groups of 4
    (180, 180, 32, 24, 0.05, torch.bfloat16),  # 8 groups of 4
    (1200, 1200, 8, 16, 0.04, torch.bfloat16),  # several column blocks and parts
    (40, 40, 8, 16, 0.5, torch.float32),
]


@pytest.mark.parametrize("tiled", ["1", "0"])
@pytest.mark.parametrize("n_q,n_k,H,d,density,dtype", CASES)
def test_tiled_and_work_list_match_oracle(monkeypatch, tiled, n_q, n_k, H, d, density, dtype):
    _say(f"case tiled={tiled} n_q={n_q} n_k={n_k} H={H} d={d} dens={density} {dtype}")
    monkeypatch.setenv("NGT_TILED", tiled)
    ei = _dense_window(n_q, n_k, density, seed=n_q + H)
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=H * 10 + d, scale=2.0)
    _check(_run(q, k, v, ei, go), q, k, v, ei, go, H, dtype, f"tiled={tiled}")


@pytest.mark.parametrize("n_q,n_k,related,H,d,dtype", [
    (400, 1400, 6, 8, 16, torch.bfloat16), (300, 700, 3, 4, 8, torch.float32),
    (500, 2600, 10, 8, 16, torch.float32)])
def test_tiled_with_related_keys_from_a_second_buffer(monkeypatch, n_q, n_k, related, H, d,
                                                      dtype):
    """The high-degree GT layout: window keys in k/v, related keys (sparse
    columns past the window) from the cache buffer: the last part gathers
    them, and only the window's keys get dK/dV."""
    _say(f"case tiled related n_q={n_q} n_k={n_k} related={related} H={H} d={d} {dtype}")
    monkeypatch.setenv("NGT_TILED", "1")
    ei = _dense_window(n_q, n_k, 0.08, seed=related, related=related)
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=related + 3)
    res = _run(q, k, v, ei, go, n_main=n_q)
    _check(res, q, k, v, ei, go, H, dtype, "tiled related", n_main=n_q)


def test_tiled_forward_with_keys_needing_gradients_past_the_window(monkeypatch):
    """N_q < N_k with every key row in one buffer (all get dK/dV): the forward
    runs tiled, the backward falls back to the work-list kernels (the tiled
    key-major pass covers the window's own keys only)."""
    _say("case tiled fwd, work-list bwd")
    monkeypatch.setenv("NGT_TILED", "1")
    n_q, n_k, H, d = 300, 600, 8, 16
    ei = _dense_window(n_q, n_k, 0.1, seed=9, related=4)
    q, k, v, go = _qkv(n_q, n_k, H, d, torch.float32, seed=9)
    _check(_run(q, k, v, ei, go), q, k, v, ei, go, H, torch.float32, "tiled fwd")


@pytest.mark.parametrize("heads", ["8", "2", "1"])
def test_tiled_head_group_widths(monkeypatch, heads):
    _say(f"case tiled heads per group {heads}")
    monkeypatch.setenv("NGT_TILED", "1")
    monkeypatch.setenv("NGT_TILE_HEADS", heads)
    n, H, d = 350, 8, 16
    ei = _dense_window(n, n, 0.07, seed=4)
    q, k, v, go = _qkv(n, n, H, d, torch.bfloat16, seed=4, scale=2.0)
    _check(_run(q, k, v, ei, go), q, k, v, ei, go, H, torch.bfloat16, f"heads {heads}")


def test_tiled_clamp_boundary_and_empty_rows(monkeypatch):
    """Scores exactly at +5 and -5 (q = 4 e_0 at d = 16, so a = k_0 exactly,
    with k_0 = +-5 on two thirds of the keys and the keys' other components
    random, so that no two keys are parallel) and rows without edges."""
    _say("case tiled clamp boundary")
    monkeypatch.setenv("NGT_TILED", "1")
    n, H, d = 120, 2, 16
    ei = _dense_window(n, n, 0.2, seed=2)
    q, k, v, go = _qkv(n, n, H, d, torch.float32, seed=2)
    q[:, :, :] = 0.0
    q[:, :, 0] = 4.0
    k[::3, :, 0] = 5.0
    k[1::3, :, 0] = -5.0
    _check(_run(q, k, v, ei, go), q, k, v, ei, go, H, torch.float32, "tiled clamp")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tiled_bitwise_reproducible(monkeypatch, dtype):
    _say(f"case tiled reproducible {dtype}")
    monkeypatch.setenv("NGT_TILED", "1")
    n, H, d = 900, 8, 16
    ei = _dense_window(n, n, 0.05, seed=6)
    q, k, v, go = _qkv(n, n, H, d, dtype, seed=6)
    a = _run(q, k, v, ei, go)
    b = _run(q, k, v, ei, go)
    for name in a:
        assert torch.equal(a[name], b[name]), name


def test_no_row_orders_means_work_lists(monkeypatch):
    """An adjacency built without the row orders never runs tiled, even when
    asked to: same results as the work-list kernels bit for bit."""
    _say("case tiled off without orders")
    n, H, d = 300, 8, 16
    ei = _dense_window(n, n, 0.1, seed=8)
    q, k, v, go = _qkv(n, n, H, d, torch.bfloat16, seed=8)
    outs = []
    for tiled_env in ("1", "0"):
        monkeypatch.setenv("NGT_TILED", tiled_env)
        adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n, n, 128, 16, tiled=False)
        qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
        x, ns = SparseAttentionFunction.apply(qd, kd, vd, adj, float(d) ** 0.5, -5.0, 5.0, 1e-6)
        x.backward(go.cuda())
        torch.cuda.synchronize()
        outs.append([x.detach().cpu(), ns.cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
