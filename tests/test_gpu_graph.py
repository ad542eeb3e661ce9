"""The sparse and dense paths under HIP graph capture: every replay must equal
the eager result bit for bit (the kernels use no atomics and no memsets), with
the program's own eager work and synchronisations between replays."""
import numpy as np
import pytest
import torch

from neutrongt_amd import SparseAttentionFunction, WindowAdjacency, dense_attention
from neutrongt_amd import chunk_for_heads, small_for_heads
from neutrongt_amd.attention import draw_seed
from neutrongt_amd.layernorm import _AddLayerNormFn
from tests._util import random_coo

pytestmark = pytest.mark.gpu


def _capture_and_check(make_step, tensors):
    """make_step() runs fwd+bwd and returns the list of output tensors."""
    eager = [t.clone() for t in make_step()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        make_step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = make_step()
    for rep in range(3):
        # unrelated eager work that reuses the allocator and the stream
        junk = torch.randn(4096, 64, device="cuda") @ torch.randn(64, 64, device="cuda")
        for t in tensors:
            t.grad = None if rep == 0 else t.grad
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b), f"replay {rep} differs from eager"
        del junk


@pytest.mark.parametrize("H,d,dtype", [(8, 8, torch.float32), (32, 24, torch.bfloat16)])
def test_sparse_graph_replay_matches_eager(H, d, dtype):
    print(f"case graph sparse H={H} d={d} {dtype}", flush=True)
    n = 300
    ei = torch.from_numpy(random_coo(n, n, 3000, seed=5)).cuda()
    adj = WindowAdjacency(ei, n, n, chunk_for_heads(H), small_for_heads(H))
    g = torch.Generator().manual_seed(1)
    q, k, v, go = (torch.randn(n, H, d, generator=g).to(dtype).cuda() for _ in range(4))
    for t in (q, k, v):
        t.requires_grad_(True)

    def step():
        for t in (q, k, v):
            t.grad = None
        x, ns = SparseAttentionFunction.apply(q, k, v, adj, d ** 0.5, -5.0, 5.0, 1e-6)
        x.backward(go)
        return [x.detach(), ns, q.grad, k.grad, v.grad]

    _capture_and_check(step, (q, k, v))


@pytest.mark.parametrize("n_q,n_k,H,d,dtype", [
    (500, 500, 4, 8, torch.bfloat16),   # matrix-core kernels
    (300, 2100, 2, 8, torch.float32),   # vector-ALU kernels, keys split over 4 blocks + combine
])
def test_dense_graph_replay_matches_eager(n_q, n_k, H, d, dtype):
    print(f"case graph dense n_q={n_q} n_k={n_k} H={H} d={d} {dtype}", flush=True)
    g = torch.Generator().manual_seed(2)
    q, k, v, go = (torch.randn(n, H, d, generator=g).to(dtype).cuda()
                   for n in (n_q, n_k, n_k, n_q))
    for t in (q, k, v):
        t.requires_grad_(True)

    def step():
        for t in (q, k, v):
            t.grad = None
        x, ns = dense_attention(q, k, v)
        x.backward(go)
        return [x.detach(), ns, q.grad, k.grad, v.grad]

    _capture_and_check(step, (q, k, v))


def _capture(make_step):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        make_step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = make_step()
    return g, outs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dense_dropout_graph_replays_draw_new_masks(dtype):
    """Dropout inside a captured graph: the seed is drawn on the device (torch's
    graph-safe generator) and read by the kernels when they run, so each
    replay draws a new mask; each replay equals the eager call with the seed
    that replay drew, forward and backward."""
    print(f"case graph dense dropout {dtype}", flush=True)
    n, H, d = 200, 2, 16
    gen = torch.Generator().manual_seed(3)
    q, k, v, go = (torch.randn(n, H, d, generator=gen).to(dtype).cuda() for _ in range(4))
    for t in (q, k, v):
        t.requires_grad_(True)

    def step():
        for t in (q, k, v):
            t.grad = None
        seed = draw_seed(q.device)
        x, _ = dense_attention(q, k, v, dropout_p=0.5, seed=seed)
        x.backward(go)
        return [seed, x.detach(), q.grad, k.grad, v.grad]

    g, outs = _capture(step)
    seen = []
    for rep in range(3):
        junk = torch.randn(2048, 64, device="cuda") @ torch.randn(64, 64, device="cuda")
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        seed = int(got[0].item())
        seen.append(seed)
        for t in (q, k, v):
            t.grad = None
        x, _ = dense_attention(q, k, v, dropout_p=0.5, seed=seed)
        x.backward(go)
        torch.cuda.synchronize()
        for a, b in zip(got[1:], [x.detach(), q.grad, k.grad, v.grad]):
            assert torch.equal(a, b), f"replay {rep} differs from the eager call with its seed"
        del junk
    assert len(set(seen)) == 3, seen


def test_add_layernorm_dropout_graph_replays_draw_new_masks():
    """The fused residual add + dropout + LayerNorm under graph capture: new
    mask per replay, each equal to the eager pass with that replay's seed."""
    print("case graph add-layernorm dropout", flush=True)
    n, c, p = 300, 96, 0.3
    gen = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(n, c, generator=gen, device="cuda").to(torch.bfloat16).requires_grad_(True)
    y = torch.randn(n, c, generator=gen, device="cuda").to(torch.bfloat16).requires_grad_(True)
    w = torch.randn(c, generator=gen, device="cuda").requires_grad_(True)
    b = torch.randn(c, generator=gen, device="cuda").requires_grad_(True)
    gy = torch.randn(n, c, generator=gen, device="cuda").to(torch.bfloat16)

    def step(seed=None):
        for t in (x, y, w, b):
            t.grad = None
        st = draw_seed(x.device) if seed is None else seed
        _, out = _AddLayerNormFn.apply(x, y, w, b, 1e-5, p, 0, True, st)
        out.backward(gy)
        return [st, out.detach(), x.grad, y.grad, w.grad, b.grad]

    g, outs = _capture(step)
    seen = []
    for rep in range(3):
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        seen.append(int(got[0].item()))
        ref = step(seed=got[0].clone())
        torch.cuda.synchronize()
        for a, r in zip(got[1:], ref[1:]):
            assert torch.equal(a, r), f"replay {rep} differs from the eager pass with its seed"
    assert len(set(seen)) == 3, seen
