"""The window adjacency cache across the reference loop's per-step device
copies (NeutronGT/core/node_level_pipeline/train_eval.py:244 makes a fresh
.to(device) copy of the window's edge_index every step): equal contents reuse
the cached CSR with one build, results unchanged; an in-place change or other
contents build again; the cache stays within its byte bound."""
import numpy as np
import pytest
import torch

from neutrongt_amd import sparse_attention
from neutrongt_amd.csr import AdjacencyCache
from tests._util import hub_coo

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _qkv(n, H, d, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, H, d, generator=g).cuda() for _ in range(3)]


def test_fresh_device_copies_of_one_window_build_once():
    _say("case csr cache: per-step device copies")
    n, H, d = 700, 8, 16
    ei_host = torch.from_numpy(hub_coo(n, n, 3000, seed=3))
    q, k, v = _qkv(n, H, d, 1)
    cache = AdjacencyCache()
    outs = []
    for step in range(3):
        ei = ei_host.to("cuda")  # a new device tensor each step, as the reference loop makes
        for _layer in range(2):  # the layers of a step share the step's tensor
            x, ns = sparse_attention(q, k, v, ei, cache=cache)
        outs.append((x.cpu(), ns.cpu()))
    assert cache.builds == 1, cache.builds
    assert cache.content_hits == 2, cache.content_hits  # one compare per later step
    for x, ns in outs[1:]:
        assert torch.equal(x, outs[0][0]) and torch.equal(ns, outs[0][1])
    # other contents of the same shape: a build of their own
    ei2 = ei_host.clone()
    ei2[0, :5] = torch.arange(5)
    x2, _ = sparse_attention(q, k, v, ei2.cuda(), cache=cache)
    assert cache.builds == 2
    ref2, _ = sparse_attention(q, k, v, ei2.cuda(), cache=AdjacencyCache())
    assert torch.equal(x2.cpu(), ref2.cpu())


def test_in_place_change_rebuilds():
    _say("case csr cache: in-place change")
    n, H, d = 300, 4, 8
    ei = torch.from_numpy(hub_coo(n, n, 900, seed=4)).cuda()
    q, k, v = _qkv(n, H, d, 2)
    cache = AdjacencyCache()
    sparse_attention(q, k, v, ei, cache=cache)
    ei[1].copy_(torch.flip(ei[1], [0]))  # same tensor, new contents
    x, _ = sparse_attention(q, k, v, ei, cache=cache)
    assert cache.builds == 2
    ref, _ = sparse_attention(q, k, v, ei.clone(), cache=AdjacencyCache())
    assert torch.equal(x.cpu(), ref.cpu())


def test_cache_respects_its_byte_bound():
    _say("case csr cache: byte bound")
    n, H, d = 400, 4, 8
    q, k, v = _qkv(n, H, d, 3)
    probe = AdjacencyCache()
    sparse_attention(q, k, v, torch.from_numpy(hub_coo(n, n, 2000, seed=10)).cuda(), cache=probe)
    one = probe.nbytes()
    cache = AdjacencyCache(capacity=64, max_bytes=int(2.5 * one))
    for s in range(6):
        ei = torch.from_numpy(hub_coo(n, n, 2000 + s, seed=10 + s)).cuda()
        sparse_attention(q, k, v, ei, cache=cache)
        assert cache.nbytes() <= cache.max_bytes or len(cache._d) == 1
    assert cache.builds == 6 and len(cache._d) <= 2
