"""Gradients of the sparse path written with a row stride
(ngt_sparse_bwd_strided): dQ, dK and dV as column blocks of one
[N, 3 * H * d] matrix, for a caller that projects q, k and v from one input.
They must equal the contiguous gradients bit for bit on every backward
variant (split hub rows and their finalize passes, packed rows, recomputed
dQ, folded row statistics, related keys from a second buffer), through the
C ABI, the Python function and the C++ autograd node."""
import ctypes as C

import numpy as np
import pytest
import torch

from neutrongt_amd import AdjacencyCache, SparseAttentionFunction, WindowAdjacency, _lib
from neutrongt_amd import sparse_attention
from tests._util import hub_coo

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _inputs(n, n_ext, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v, go = (torch.randn(n + (n_ext if i in (1, 2) else 0), H, d, generator=g).to(dtype)
                   for i in range(4))
    return q, k, v, go


def _grads(q, k, v, go, adj, n_main, interleave, fn):
    qd = q.cuda().requires_grad_(True)
    kd = k[:n_main].cuda().requires_grad_(True)
    vd = v[:n_main].cuda().requires_grad_(True)
    ext = (k[n_main:].cuda(), v[n_main:].cuda()) if n_main < k.shape[0] else (None, None)
    d = q.shape[-1]
    seen = []  # the gradients as the core hands them over (a leaf's .grad is a dense copy)
    for t in (qd, kd, vd):
        t.register_hook(lambda g: seen.append(g))
    if fn == "function":
        x, _ = SparseAttentionFunction.apply(qd, kd, vd, adj, float(d) ** 0.5, -5.0, 5.0, 1e-6,
                                             ext[0], ext[1], interleave)
    else:
        from neutrongt_amd.attention import window_attention
        x, _ = window_attention(qd, kd, vd, adj, float(d) ** 0.5, k_ext=ext[0], v_ext=ext[1],
                                interleave_grads=interleave)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    return (qd.grad, kd.grad, vd.grad), sorted(seen, key=lambda g: g.data_ptr())


@pytest.mark.parametrize("fn", ["function", "node"])
@pytest.mark.parametrize("H,d,dtype,chunk,small,n_ext,env", [
    (32, 24, torch.bfloat16, 32, 2, 0, {}),
    (32, 24, torch.bfloat16, 32, 2, 150, {}),  # related keys from a second buffer
    (8, 8, torch.float32, 16, 3, 0, {}),
    (8, 16, torch.float32, 16, 3, 0, {"NGT_DQ_RECOMPUTE": "1"}),
    (8, 8, torch.bfloat16, 64, 8, 0, {"NGT_FOLD_ROWSTAT": "1"}),
    (4, 32, torch.bfloat16, 48, 4, 60, {"NGT_DQ_RECOMPUTE": "1"}),
])
def test_interleaved_gradients_equal_contiguous_ones(monkeypatch, fn, H, d, dtype, chunk, small,
                                                     n_ext, env):
    _say(f"case interleaved {fn} H={H} d={d} {dtype} chunk={chunk} ext={n_ext} {env}")
    if fn == "node" and _lib.autograd_ext() is None:
        pytest.skip("the C++ autograd node is not built")
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    n = 700
    ei = hub_coo(n, n + n_ext, 6000, seed=H + d)
    q, k, v, go = _inputs(n, n_ext, H, d, dtype, seed=H * d)
    adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n, n + n_ext, chunk, small, tiled=False)
    ref, _ = _grads(q, k, v, go, adj, n, False, fn)
    got, handed = _grads(q, k, v, go, adj, n, True, fn)
    # handed over as views of one [n, 3, H, d] buffer: dQ, dK, dV of a row side by side
    w = 3 * H * d
    es = handed[0].element_size()
    assert len(handed) == 3
    for i, gr in enumerate(handed):
        assert gr.shape == (n, H, d) and gr.stride() == (w, d, 1), (i, gr.stride())
        assert gr.data_ptr() == handed[0].data_ptr() + i * H * d * es
    for name, a, b in zip(("dq", "dk", "dv"), ref, got):
        assert torch.equal(a, b), name


def test_strided_gradient_rows_through_the_c_abi():
    """A wider row stride than 3 H d (gaps between rows): the gaps keep their
    contents, the rows equal the contiguous gradients."""
    _say("case strided C ABI")
    lib = _lib.load()
    n, H, d = 500, 8, 16
    ei = hub_coo(n, n, 4000, seed=7)
    q, k, v, go = _inputs(n, 0, H, d, torch.bfloat16, seed=7)
    q, k, v, go = (t.cuda() for t in (q, k, v, go))
    adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n, n, 32, 2, tiled=False)
    fb, bb = adj.workspace_bytes(H, d)
    out = torch.empty_like(q)
    rinv = torch.empty(n, H, dtype=torch.float32, device="cuda")
    ns = torch.empty(adj.dst_end, dtype=torch.float32, device="cuda")
    ws = torch.empty(max(fb, bb, 1), dtype=torch.uint8, device="cuda")
    st = _lib.stream_ptr(q.device)
    _lib.check(lib.ngt_sparse_fwd(1, q.data_ptr(), k.data_ptr(), v.data_ptr(), adj.ptr(), H, d,
                                  4.0, -5.0, 5.0, 1e-6, out.data_ptr(), rinv.data_ptr(),
                                  ns.data_ptr(), int(ns.numel()), ws.data_ptr(), fb, st))
    sep = [torch.empty_like(q) for _ in range(3)]
    _lib.check(lib.ngt_sparse_bwd(1, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                  go.data_ptr(), rinv.data_ptr(), adj.ptr(), H, d, 4.0, -5.0, 5.0,
                                  *(t.data_ptr() for t in sep), ws.data_ptr(), bb, st))
    ld = 4 * H * d + 8  # a multiple of 16 bytes in bf16
    buf = torch.full((n, ld), 7.0, dtype=torch.bfloat16, device="cuda")
    views = [buf[:, i * H * d:(i + 1) * H * d] for i in range(3)]
    _lib.check(lib.ngt_sparse_bwd_strided(
        1, q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, n, out.data_ptr(), go.data_ptr(),
        rinv.data_ptr(), adj.ptr(), H, d, 4.0, -5.0, 5.0, *(t.data_ptr() for t in views), ld,
        ws.data_ptr(), bb, st))
    torch.cuda.synchronize()
    for a, b in zip(sep, views):
        assert torch.equal(a.reshape(n, -1), b)
    assert (buf[:, 3 * H * d:] == 7.0).all()
