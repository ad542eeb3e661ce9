"""ngt_sparse_fwd_noalloc (scratch in a static device array, nothing
allocated) against ngt_sparse_fwd with a caller workspace, through the C ABI:
bit-identical outputs on two calls in a row, the second on a smaller window,
and both within the path's tolerance of the oracle."""
import ctypes as C

import numpy as np
import pytest
import torch

from neutrongt_amd import _lib
from neutrongt_amd.csr import WindowAdjacency
from oracle import attention as OA
from tests._util import assert_close, hub_coo

pytestmark = pytest.mark.gpu


def _window(n, hub, H, d, dtype, seed):
    ei = hub_coo(n, n, hub, seed=seed)
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(n, H, d, generator=g).to(dtype) for _ in range(3))
    return ei, q, k, v


def _fwd(lib, adj, q, k, v, noalloc):
    n_q, H, d = q.shape
    dev = q.device
    out = torch.empty_like(q)
    rinv = torch.empty(n_q, H, dtype=torch.float32, device=dev)
    ns = torch.empty(adj.dst_end, dtype=torch.float32, device=dev)
    dt = _lib.NGT_F32 if q.dtype == torch.float32 else _lib.NGT_BF16
    st = _lib.stream_ptr(dev)
    scale = float(d) ** 0.5
    if noalloc:
        _lib.check(lib.ngt_sparse_fwd_noalloc(dt, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                              adj.ptr(), H, d, scale, -5.0, 5.0, 1e-6,
                                              out.data_ptr(), rinv.data_ptr(), ns.data_ptr(),
                                              int(ns.numel()), st))
    else:
        fb, bb = C.c_size_t(), C.c_size_t()
        _lib.check(lib.ngt_sparse_workspace_bytes(adj.ptr(), H, d, C.byref(fb), C.byref(bb)))
        ws = torch.empty(max(fb.value, 1), dtype=torch.uint8, device=dev)
        _lib.check(lib.ngt_sparse_fwd(dt, q.data_ptr(), k.data_ptr(), v.data_ptr(), adj.ptr(),
                                      H, d, scale, -5.0, 5.0, 1e-6, out.data_ptr(),
                                      rinv.data_ptr(), ns.data_ptr(), int(ns.numel()),
                                      ws.data_ptr(), fb.value, st))
    torch.cuda.synchronize()
    return out.cpu(), rinv.cpu(), ns.cpu()


@pytest.mark.parametrize("H,d,dtype", [(8, 16, torch.bfloat16), (4, 8, torch.float32)])
def test_noalloc_forward_matches_workspace_forward(H, d, dtype):
    lib = _lib.load()
    # the larger window first, then a smaller one: the second call reuses the
    # static scratch that the first left filled
    for n, hub, chunk, seed in ((900, 2500, 64, 1), (300, 700, 32, 2)):
        print(f"case noalloc n={n} hub={hub} H={H} d={d} {dtype}", flush=True)
        ei, q, k, v = _window(n, hub, H, d, dtype, seed)
        adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n, n, chunk, 2, tiled=False)
        assert adj.struct.n_splits_q > 0  # split rows: the partials live in the scratch
        qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
        ref = _fwd(lib, adj, qd, kd, vd, noalloc=False)
        got = _fwd(lib, adj, qd, kd, vd, noalloc=True)
        for a, b, name in zip(got, ref, ("out", "rinv", "node_score")):
            assert torch.equal(a, b), f"{name} differs from ngt_sparse_fwd (n={n})"
        orc = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), torch.from_numpy(ei),
                                torch.zeros(n, H, d), H)
        assert_close(got[0].float(), orc["x"], dtype, "noalloc x vs oracle")
        assert_close(got[2], orc["node_scores"], dtype, "noalloc node scores vs oracle")
