"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors for its attention path, so these pin
the oracle (and through it the HIP kernels) across machines and torch
versions.  Inputs are seeded; outputs are the oracle's fp32 forward and
autograd backward.  Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as OA  # noqa: E402
from oracle import graph as OG  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def _qkv(n_q, n_k, H, d, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n_q, H, d, generator=g), torch.randn(n_k, H, d, generator=g),
            torch.randn(n_k, H, d, generator=g), torch.randn(n_q, H, d, generator=g))


def sparse_case(name, n_q, n_k, H, d, E, seed, q_mult=1.0):
    rng = np.random.default_rng(seed)
    src = rng.integers(0, n_k, E)
    dst = rng.integers(0, n_q - 2, E)  # the last two query rows stay empty
    src = np.concatenate([src, [3, 3]])  # one duplicated edge
    dst = np.concatenate([dst, [1, 1]])
    ei = np.stack([src, dst]).astype(np.int64)
    q, k, v, go = _qkv(n_q, n_k, H, d, seed)
    q = q * q_mult
    res = OA.sparse_fwd_bwd(q, k, v, torch.from_numpy(ei), go, H, dtype=torch.float32)
    csr = OG.csr_from_coo(ei[0], ei[1], n_q, n_k)
    np.savez_compressed(os.path.join(HERE, f"attn_{name}.npz"), kind="sparse", edge_index=ei,
                        q=q.numpy(), k=k.numpy(), v=v.numpy(), go=go.numpy(),
                        **{n: res[n].numpy() for n in ("x", "node_scores", "dq", "dk", "dv")},
                        **{"csr_" + n: a for n, a in csr.items()})


def dense_case(name, n_q, n_k, H, d, seed):
    q, k, v, go = _qkv(n_q, n_k, H, d, seed)
    res = OA.full_fwd_bwd(q, k, v, go, dtype=torch.float32)
    np.savez_compressed(os.path.join(HERE, f"attn_{name}.npz"), kind="dense", q=q.numpy(),
                        k=k.numpy(), v=v.numpy(), go=go.numpy(),
                        **{n: res[n].numpy() for n in ("x", "node_scores", "dq", "dk", "dv")})


def related_case():
    """Hand-checkable related-node selection with ties (metisPartition.py:397-425)."""
    # 8-node symmetric weighted graph; partition {0, 1, 2}
    edges = {(0, 3): 5, (0, 4): 2, (1, 4): 3, (1, 5): 2, (2, 6): 2, (2, 7): 1, (0, 1): 9,
             (3, 4): 1}
    n = 8
    adj = [[] for _ in range(n)]
    for (a, b), w in sorted(edges.items()):
        adj[a].append((b, w))
        adj[b].append((a, w))
    xadj = np.zeros(n + 1, np.int32)
    adjncy, ew = [], []
    for u in range(n):
        for b, w in sorted(adj[u]):
            adjncy.append(b)
            ew.append(w)
        xadj[u + 1] = len(adjncy)
    part = np.array([2, 0, 1], np.int64)
    outs = {}
    for pct in (0, 25, 50, 60, 100):
        out, n_ext = OG.merge_related_nodes(xadj, adjncy, ew, part, pct)
        outs[f"out_{pct}"] = out
        outs[f"n_ext_{pct}"] = np.int64(n_ext)
    np.savez_compressed(os.path.join(HERE, "related_small.npz"), xadj=xadj,
                        adjncy=np.array(adjncy, np.int32), eweights=np.array(ew, np.int32),
                        partition=part, **outs)


if __name__ == "__main__":
    sparse_case("sparse_h4d8", 24, 24, 4, 8, 150, seed=1)
    sparse_case("sparse_h2d16_nk", 20, 31, 2, 16, 120, seed=2, q_mult=4.0)  # clamp active
    dense_case("dense_h2d8", 12, 17, 2, 8, seed=3)
    related_case()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
