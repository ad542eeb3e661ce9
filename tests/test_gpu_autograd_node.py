"""The C++ autograd node (ngt_autograd.so) against SparseAttentionFunction.

Both drive the same library entry points, so every output and gradient must
agree bit for bit (the path has no atomics); the oracle parity of those
entry points is covered by test_gpu_sparse.py."""
import gc

import numpy as np
import pytest
import torch

from neutrongt_amd import SparseAttentionFunction, WindowAdjacency, _lib, window_attention
from tests._util import hub_coo, random_coo

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _inputs(n_q, n_k, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, H, d, generator=g).to(dtype).cuda() for n in (n_q, n_k, n_k, n_q)]


def _fwd_bwd(fn, q, k, v, go, adj, ext=None):
    qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
    kx, vx = ext if ext is not None else (None, None)
    x, ns = fn(qd, kd, vd, adj, float(q.shape[-1]) ** 0.5, -5.0, 5.0, 1e-6, kx, vx)
    x.backward(go)
    torch.cuda.synchronize()
    return [x.detach(), ns, qd.grad, kd.grad, vd.grad]


def test_node_is_built_and_bound():
    ext = _lib.autograd_ext()
    assert ext is not None, "ngt_autograd.so is not built (neutrongt_amd.build.build_autograd_ext)"
    assert ext.csr_struct_bytes() == _lib.C.sizeof(_lib.WindowCSR)


@pytest.mark.parametrize("n_q,n_k,H,d,dtype,chunk,small,hub", [
    (300, 300, 8, 8, torch.float32, 256, 4, False),
    (200, 350, 32, 24, torch.bfloat16, 64, 2, True),
    (128, 128, 4, 16, torch.bfloat16, 32, 0, True),
])
def test_node_matches_function_bitwise(n_q, n_k, H, d, dtype, chunk, small, hub):
    _say(f"case node n_q={n_q} n_k={n_k} H={H} d={d} {dtype} chunk={chunk} hub={hub}")
    ei = hub_coo(n_q, n_k, 900, seed=3) if hub else random_coo(n_q, n_k, 8 * n_q, seed=4)
    adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n_q, n_k, chunk, small)
    q, k, v, go = _inputs(n_q, n_k, H, d, dtype, seed=n_q)
    a = _fwd_bwd(window_attention, q, k, v, go, adj)
    b = _fwd_bwd(SparseAttentionFunction.apply, q, k, v, go, adj)
    for name, x, y in zip(("x", "node_scores", "dq", "dk", "dv"), a, b):
        assert torch.equal(x, y), name


def test_node_external_keys_get_no_gradient():
    n_q, n_main, n_ext, H, d = 150, 150, 60, 8, 8
    rng = np.random.default_rng(7)
    ei = np.stack([rng.integers(0, n_main + n_ext, 1500), rng.integers(0, n_q, 1500)])
    adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n_q, n_main + n_ext, 64, 2)
    q, k, v, go = _inputs(n_q, n_main, H, d, torch.float32, seed=9)
    kx, vx = (t.cuda() for t in _inputs(n_ext, n_ext, H, d, torch.float32, seed=10)[:2])
    a = _fwd_bwd(window_attention, q, k, v, go, adj, (kx, vx))
    b = _fwd_bwd(SparseAttentionFunction.apply, q, k, v, go, adj, (kx, vx))
    for name, x, y in zip(("x", "node_scores", "dq", "dk", "dv"), a, b):
        assert torch.equal(x, y), name
    assert kx.grad is None and vx.grad is None


def test_node_keeps_the_window_until_backward():
    """The node holds the window's device memory and struct bytes: dropping
    every Python reference to the adjacency between forward and backward frees
    none of its arena, and the backward then matches the function's."""
    n, H, d = 400, 8, 8
    ei = torch.from_numpy(random_coo(n, n, 4000, seed=11)).cuda()
    q, k, v, go = _inputs(n, n, H, d, torch.float32, seed=12)
    adj = WindowAdjacency(ei, n, n, 128, 4)
    want = _fwd_bwd(SparseAttentionFunction.apply, q, k, v, go, adj)
    qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
    x, _ = window_attention(qd, kd, vd, adj, d ** 0.5)
    torch.cuda.synchronize()
    arena = adj.mem.numel() * adj.mem.element_size()
    before = torch.cuda.memory_allocated()
    del adj
    gc.collect()
    assert before - torch.cuda.memory_allocated() < arena, "the window's arena was freed"
    x.backward(go)
    torch.cuda.synchronize()
    for name, got, ref in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), want[2:]):
        assert torch.equal(got, ref), name


def test_node_forward_without_grad():
    n, H, d = 200, 4, 8
    ei = torch.from_numpy(random_coo(n, n, 1600, seed=13)).cuda()
    adj = WindowAdjacency(ei, n, n, 64, 2)
    q, k, v, go = _inputs(n, n, H, d, torch.float32, seed=14)
    with torch.no_grad():
        x0, ns0 = window_attention(q, k, v, adj, d ** 0.5)
    x1, ns1 = SparseAttentionFunction.apply(q, k, v, adj, d ** 0.5, -5.0, 5.0, 1e-6)
    assert torch.equal(x0, x1) and torch.equal(ns0, ns1)
    # node scores carry no gradient; a loss that zeroes the output still runs the backward
    qd = q.clone().requires_grad_(True)
    x, ns = window_attention(qd, k, v, adj, d ** 0.5)
    assert not ns.requires_grad
    (x.sum() * 0).backward()
    assert qd.grad is not None
