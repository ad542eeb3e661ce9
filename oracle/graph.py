"""numpy restatements of the integer window preparation (test oracle only).

Every function returns plain numpy arrays and is bit-exact by construction
(integer arithmetic, stable sorts).

  csr_from_coo              the canonical CSR the kernels consume, built from the
                            window COO of NeutronGT/core/node_level_pipeline/
                            window_state.py:122-140 (rows sorted by (dst, src,
                            edge id); transposed by (src, dst, edge id))
  work_items                degree-binned work list (chunked long rows first)
  merge_related_nodes       NeutronGT/core/metisPartition.py:397-425
  duplicate_rerange         NeutronGT/core/node_level_pipeline/window_state.py:52-73
  dup_cache_metadata        NeutronGT/core/node_level_pipeline/window_state.py:181-205
  assemble_window_features  NeutronGT/core/node_level_pipeline/train_eval.py:234-242
  adj_weights               NeutronGT/core/ppr_preprocess.py:30-71 (weight rule;
                            neighbour order fixed stable, see the docstring)
  subgraph_coo              torch_geometric.utils.subgraph(relabel_nodes=True)
                            semantics as used at window_state.py:127
  subgraph_from_csr         NeutronGT/core/node_level_pipeline/window_state.py:92-119
"""
from __future__ import annotations

import numpy as np


def csr_from_coo(src, dst, n_q: int, n_k: int):
    """Query-major + key-major CSR of a window COO.  Returns a dict of int32
    arrays: rowptr, col, perm, t_rowptr, t_col, t_perm, q2t."""
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    assert src.shape == dst.shape
    assert (src >= 0).all() and (src < n_k).all() and (dst >= 0).all() and (dst < n_q).all()
    perm = np.lexsort((src, dst))  # stable: ties keep edge-id order
    t_perm = np.lexsort((dst, src))
    rowptr = np.zeros(n_q + 1, dtype=np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=n_q))
    t_rowptr = np.zeros(n_k + 1, dtype=np.int64)
    t_rowptr[1:] = np.cumsum(np.bincount(src, minlength=n_k))
    tpos = np.empty(src.shape[0], dtype=np.int64)
    tpos[t_perm] = np.arange(src.shape[0])
    return {
        "rowptr": rowptr.astype(np.int32),
        "col": src[perm].astype(np.int32),
        "perm": perm.astype(np.int32),
        "t_rowptr": t_rowptr.astype(np.int32),
        "t_col": dst[t_perm].astype(np.int32),
        "t_perm": t_perm.astype(np.int32),
        "q2t": tpos[perm].astype(np.int32),
    }


def work_items(rowptr, chunk: int, small: int = 0):
    """Degree-binned work list for one orientation.

    Rows longer than ``chunk`` are cut into chunks (listed first, in row
    order, part slot = item index).  Rows with small < degree <= chunk are one
    item each (part -1) and rows with degree <= small go to the packed list;
    both follow the order of a stable ascending sort by degree, reversed
    (longest first; equal degrees by descending row id).  Requires
    small < chunk (the host clamps it), so no row is both split and packed.
    Returns (items [n,4], splits [m,4], packed [p])."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    deg = np.diff(rowptr)
    split_items, splits = [], []
    for r in range(rowptr.shape[0] - 1):
        b, e = int(rowptr[r]), int(rowptr[r + 1])
        if e - b > chunk:
            n = (e - b + chunk - 1) // chunk
            splits.append((r, len(split_items), n, 0))
            for c in range(n):
                s = len(split_items)
                split_items.append((r, b + c * chunk, min(e, b + (c + 1) * chunk), s))
    order = np.argsort(deg, kind="stable")
    d_sorted = deg[order]
    packed = order[d_sorted <= small][::-1]
    medium = order[(d_sorted > small) & (d_sorted <= chunk)][::-1]
    plain = [(int(r), int(rowptr[r]), int(rowptr[r + 1]), -1) for r in medium]
    items = np.array(split_items + plain, dtype=np.int32).reshape(-1, 4)
    return (items, np.array(splits, dtype=np.int32).reshape(-1, 4),
            np.asarray(packed, dtype=np.int32))


def merge_related_nodes(xadj, adjncy, eweights, partition, topk_percent: int):
    """weightMetis_keepParent._merge_related_nodes (metisPartition.py:397-425),
    restated with the same Python containers (dict insertion order, stable
    ``sorted``)."""
    xadj = np.asarray(xadj, np.int64)
    adjncy = np.asarray(adjncy)
    eweights = np.asarray(eweights)
    part = [int(x) for x in partition]
    partition_set = set(part)
    external = {}
    for node in part:
        start, end = int(xadj[node]), int(xadj[node + 1])
        if end - start == 0:
            continue
        for nb, w in zip(adjncy[start:end].tolist(), eweights[start:end].tolist()):
            if nb not in partition_set:
                external[nb] = external.get(nb, 0) + w
    ranked = sorted(external.items(), key=lambda x: x[1], reverse=True)
    n_select = len(ranked) * topk_percent // 100 if topk_percent > 0 else 0
    selected = {node for node, _ in ranked[:n_select]}
    out = sorted(partition_set | selected)
    return np.array(out, dtype=np.int64), len(external)


def row_orders(rowptr, t_rowptr, n_q, n_k):
    """The rows longest first, ties by descending row id (a stable ascending
    sort by degree, reversed): every query row, and the key rows j <
    min(n_q, n_k).  The schedule order of the library's tiled kernels; it
    changes no result, only which rows share a block."""
    dq = np.diff(np.asarray(rowptr, np.int64))
    dk = np.diff(np.asarray(t_rowptr, np.int64))[: min(n_q, n_k)]
    return (np.argsort(dq, kind="stable")[::-1].astype(np.int32),
            np.argsort(dk, kind="stable")[::-1].astype(np.int32))


def duplicate_rerange(local_partitions):
    """_compute_local_duplicate_nodes (window_state.py:52-73): nodes present in
    >= 2 of the rank's windows go first in each window (original order kept)."""
    parts = [np.asarray(p, dtype=np.int64) for p in local_partitions]
    if not parts:
        return [], []
    all_nodes = np.concatenate(parts) if parts else np.zeros(0, np.int64)
    if all_nodes.size == 0:
        return [p.copy() for p in parts], [np.zeros(0, np.int64) for _ in parts]
    uniq, counts = np.unique(all_nodes, return_counts=True)
    dups = uniq[counts >= 2]
    if dups.size == 0:
        return [p.copy() for p in parts], [np.zeros(0, np.int64) for _ in parts]
    reranged, dup_lists = [], []
    for p in parts:
        m = np.isin(p, dups)
        reranged.append(np.concatenate([p[m], p[~m]]))
        dup_lists.append(p[m])
    return reranged, dup_lists


def dup_cache_metadata(dup_lists):
    """build_dup_cache_metadata (window_state.py:181-205): the cache holds the
    sorted unique duplicate ids; each window indexes it by searchsorted."""
    non_empty = [np.asarray(d, np.int64) for d in dup_lists if len(d) > 0]
    if not non_empty:
        return np.zeros(0, np.int64), [np.zeros(0, np.int64) for _ in dup_lists]
    uniq = np.unique(np.concatenate(non_empty))
    idx = [np.searchsorted(uniq, np.asarray(d, np.int64)) if len(d) else np.zeros(0, np.int64)
           for d in dup_lists]
    return uniq, idx


def assemble_window_features(feature, cache_ids, dup_index, partition):
    """x_i = cat(cache[dup_index], feature[partition[n_dup:]]) (train_eval.py:234-242)."""
    feature = np.asarray(feature)
    cache = feature[np.asarray(cache_ids, np.int64)]
    n_dup = len(dup_index)
    rest = feature[np.asarray(partition, np.int64)[n_dup:]]
    if n_dup == 0:
        return rest
    return np.concatenate([cache[np.asarray(dup_index, np.int64)], rest], axis=0)


def adj_weights(edge_index, ppr_val):
    """build_adj_fromat's weight rule (ppr_preprocess.py:30-71).

    Undirected key min*N+max, unique (sorted), fp32 sum of the PPR values per
    key, w = int32(clamp_min(sum * 1000, 1)) (truncation), both directions.
    The reference orders rows with an unstable argsort; this restatement (and
    the product) fixes the order stable: within row u, the entries coming from
    (u, v>u) keys in ascending v, then the (v<u, u) keys in ascending v.
    Returns (xadj int32 [N+1], adjncy int32, eweights int32).
    """
    ei = np.asarray(edge_index, dtype=np.int64)
    val = np.asarray(ppr_val, dtype=np.float32)
    if ei.size == 0:
        return np.zeros(1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.int32)
    n = int(ei.max()) + 1
    u = np.minimum(ei[0], ei[1])
    v = np.maximum(ei[0], ei[1])
    key = u * n + v
    uniq, inv = np.unique(key, return_inverse=True)
    summed = np.zeros(uniq.shape[0], dtype=np.float32)
    np.add.at(summed, inv, val)
    uu = uniq // n
    vv = uniq % n
    w = np.maximum(summed * np.float32(1000.0), np.float32(1.0)).astype(np.int32)
    u_all = np.concatenate([uu, vv])
    v_all = np.concatenate([vv, uu])
    w_all = np.concatenate([w, w])
    order = np.argsort(u_all, kind="stable")
    deg = np.bincount(u_all, minlength=n)
    xadj = np.zeros(n + 1, dtype=np.int64)
    xadj[1:] = np.cumsum(deg)
    return xadj.astype(np.int32), v_all[order].astype(np.int32), w_all[order].astype(np.int32)


def subgraph_coo(partition, edge_index, num_nodes: int):
    """Induced subgraph with relabelling by position in ``partition``, edges in
    global edge order (torch_geometric subgraph(relabel_nodes=True))."""
    part = np.asarray(partition, np.int64)
    ei = np.asarray(edge_index, np.int64)
    pos = np.full(num_nodes, -1, dtype=np.int64)
    pos[part] = np.arange(part.shape[0])
    keep = (pos[ei[0]] >= 0) & (pos[ei[1]] >= 0)
    return np.stack([pos[ei[0][keep]], pos[ei[1][keep]]])


def subgraph_from_csr(node_set, rowptr, col):
    """_subgraph_from_csr (window_state.py:92-119), restated with numpy: the set
    is sorted once; for each set node in set order, its CSR neighbours are
    looked up by binary search in the sorted set and the matches emitted as
    (position of the row node, original position of the neighbour)."""
    node_set = np.asarray(node_set, np.int64)
    rowptr = np.asarray(rowptr, np.int64)
    col = np.asarray(col, np.int64)
    if node_set.size == 0:
        return np.zeros((2, 0), np.int64)
    sort_order = np.argsort(node_set, kind="stable")
    sorted_nodes = node_set[sort_order]
    rows, cols = [], []
    for local_src, g in enumerate(node_set.tolist()):
        nbrs = col[rowptr[g]:rowptr[g + 1]]
        if nbrs.size == 0:
            continue
        p = np.searchsorted(sorted_nodes, nbrs)
        inb = p < sorted_nodes.size
        matched = np.zeros(nbrs.size, bool)
        matched[inb] = sorted_nodes[p[inb]] == nbrs[inb]
        if not matched.any():
            continue
        local_dst = sort_order[p[matched]]
        rows.append(np.full(local_dst.size, local_src, np.int64))
        cols.append(local_dst.astype(np.int64))
    if not rows:
        return np.zeros((2, 0), np.int64)
    return np.stack([np.concatenate(rows), np.concatenate(cols)])
