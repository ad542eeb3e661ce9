"""Pure-Python/numpy restatement of APPNP personalised PageRank with per-row
top-k (test oracle only).

NeutronGT/core/ppr_backends/appnp_backend.py:179-310 (SpGEMM in
cusparse_spgemm.cu:65-267): per batch of seeds, ``num_iterations`` times

    state <- topk_K( fp32(1 - alpha) * (state @ P) + alpha * e_seed ),
    P[c, n] = fp32(1 / max(deg(c), 1)).

All arithmetic is float32, in a fixed order: the products state[r, c] * P[c, n]
of one (row, n) are added in the order (state rank of c, CSR position of n),
starting from 0; the sum is scaled, then the teleport added.  Top-k ranks by
value descending, node id ascending.  The reference leaves both orders to
cuSPARSE / an atomic scatter_add / torch.topk; this fixes them the way the
product documents.
"""
from __future__ import annotations

import numpy as np


def transition_csr(edge_index, num_nodes=None):
    """Rows sorted by (src, dst) (appnp_backend.py:37-55).  Returns
    (rowptr int64, col int64, inv_deg float32, n)."""
    ei = np.asarray(edge_index, np.int64)
    n = int(num_nodes) if num_nodes is not None else (int(ei.max()) + 1 if ei.size else 0)
    order = np.lexsort((ei[1], ei[0])) if ei.size else np.zeros(0, np.int64)
    src, dst = ei[0][order], ei[1][order]
    counts = np.bincount(src, minlength=n)
    rowptr = np.zeros(n + 1, np.int64)
    rowptr[1:] = np.cumsum(counts)
    inv = (np.float32(1.0) / np.maximum(counts, 1).astype(np.float32)).astype(np.float32)
    return rowptr, dst, inv, n


def rank(entries, k):
    """Top-k of [(node, value)] by value descending, node ascending."""
    return sorted(entries, key=lambda t: (-float(t[1]), int(t[0])))[:k]


def appnp_row(rowptr, col, inv, seed, alpha, K, num_iterations):
    keep = np.float32(1.0 - alpha)
    a32 = np.float32(alpha)
    state = [(int(seed), np.float32(1.0))]
    for _ in range(num_iterations):
        acc = {}
        for c, v in state:
            w = np.float32(v * inv[c])
            for n in col[rowptr[c]:rowptr[c + 1]].tolist():
                acc[n] = np.float32(acc.get(n, np.float32(0.0)) + w)
        out = {n: np.float32(s * keep) for n, s in acc.items()}
        out[int(seed)] = np.float32(out.get(int(seed), np.float32(0.0)) + a32)
        state = rank(out.items(), K)
    return state


def personal_pagerank_appnp(edge_index, alpha, topk=100, num_iterations=10, num_nodes=None,
                            iter_topk=None, source_start=None, source_end=None):
    """(edge_index [2, nnz], values) with rows in seed order, entries in rank
    order (batching does not change the result: rows are independent)."""
    rowptr, col, inv, n = transition_csr(edge_index, num_nodes)
    start = 0 if source_start is None else max(0, min(int(source_start), n))
    end = n if source_end is None else max(start, min(int(source_end), n))
    topk = min(int(topk), n)
    K = min(topk if iter_topk is None else int(iter_topk), n)
    keep_final = min(topk, K)
    src, dst, val = [], [], []
    for s in range(start, end):
        for node, v in appnp_row(rowptr, col, inv, s, alpha, K, num_iterations)[:keep_final]:
            src.append(s)
            dst.append(node)
            val.append(v)
    return np.array([src, dst], np.int64).reshape(2, -1), np.array(val, np.float32)


def appnp_dense_fp64(edge_index, n, alpha, K, num_iterations, seeds):
    """The same recursion with dense float64 matrices (independent check):
    S <- trunc_K((1 - alpha) S P + alpha E).  Returns S [len(seeds), n]."""
    ei = np.asarray(edge_index, np.int64)
    A = np.zeros((n, n))
    np.add.at(A, (ei[0], ei[1]), 1.0)
    deg = np.maximum(A.sum(1), 1.0)
    P = A / deg[:, None]
    B = len(seeds)
    E = np.zeros((B, n))
    E[np.arange(B), seeds] = 1.0
    S = E.copy()
    for _ in range(num_iterations):
        S = (1.0 - alpha) * (S @ P) + alpha * E
        for r in range(B):
            nz = np.flatnonzero(S[r])
            if nz.size > K:
                order = sorted(nz.tolist(), key=lambda c: (-S[r, c], c))
                S[r, order[K:]] = 0.0
    return S
