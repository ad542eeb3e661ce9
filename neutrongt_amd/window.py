"""Window preparation that feeds the attention core (integer work, bit-exact).

  merge_related_nodes       GPU (ngt_merge_related_nodes); mirrors
                            weightMetis_keepParent._merge_related_nodes,
                            NeutronGT/core/metisPartition.py:397-425
  window_dup_layout         GPU (ngt_window_dup_layout); the two functions below
                            in one pass
  duplicate_rerange         GPU; NeutronGT/core/node_level_pipeline/window_state.py:52-73
  dup_cache_metadata        GPU; NeutronGT/core/node_level_pipeline/window_state.py:181-205
  dup_feature_cache         GPU row gather; window_state.py:204
  assemble_window_features  GPU row gather (ngt_gather_rows); mirrors
                            NeutronGT/core/node_level_pipeline/train_eval.py:234-242
  adj_weights               NeutronGT/core/ppr_preprocess.py:30-71 weight rule,
                            with a stable neighbour order (the reference's
                            argsort at :53 is unstable)
  subgraph                  GPU (ngt_subgraph_coo); torch_geometric subgraph with
                            relabel_nodes=True as called at window_state.py:82,127
                            and metisPartition.py:280,290
  subgraph_from_csr         GPU (ngt_subgraph_csr); window_state.py:92-119
  rebuild_local_windows     a rank's windows: duplicate layout, feature cache and
                            induced subgraphs in one call; window_state.py:223-260

Every step runs as HIP kernels; Python only sizes buffers and reads back
counts.
"""
from __future__ import annotations

import ctypes as C
import functools

import torch

from . import _lib, _streams


def merge_related_nodes(xadj: torch.Tensor, adjncy: torch.Tensor, eweights: torch.Tensor,
                        partition: torch.Tensor, topk_percent: int) -> torch.Tensor:
    """Partition expanded by its top ``topk_percent`` % external neighbours.

    xadj/adjncy/eweights: int32 symmetric CSR of the global graph on the GPU
    (METIS adjacency + edge weights); partition: int64 global ids.  Returns a
    sorted int64 tensor on the GPU (one device->host sync for its length).
    """
    lib = _lib.load()
    dev = partition.device
    if not (xadj.is_cuda and adjncy.is_cuda and eweights.is_cuda and partition.is_cuda):
        raise ValueError("merge_related_nodes: all tensors must be on the GPU")
    xadj = xadj.to(torch.int32).contiguous()
    adjncy = adjncy.to(torch.int32).contiguous()
    eweights = eweights.to(torch.int32).contiguous()
    part = partition.to(torch.int64).contiguous()
    n_nodes = int(xadj.numel()) - 1
    if adjncy.numel() != eweights.numel():
        raise ValueError("adjncy and eweights differ in length")
    # The kernels index adjncy through xadj: reject a malformed CSR up front.
    if n_nodes < 0 or int(xadj[0].item()) != 0 or int(xadj[-1].item()) != adjncy.numel() or \
            bool((xadj[1:] < xadj[:-1]).any().item()):
        raise ValueError("merge_related_nodes: xadj is not a valid CSR row pointer for adjncy")
    out = torch.empty(max(n_nodes, 1), dtype=torch.int64, device=dev)
    status = torch.zeros(3, dtype=torch.int32, device=dev)
    nb = C.c_size_t()
    _lib.check(lib.ngt_related_workspace_bytes(n_nodes, int(part.numel()), C.byref(nb)))
    ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=dev)
    stream = _lib.stream_ptr(dev)
    _lib.check(lib.ngt_merge_related_nodes(xadj.data_ptr(), adjncy.data_ptr(),
                                           eweights.data_ptr(), n_nodes, part.data_ptr(),
                                           int(part.numel()), int(topk_percent), out.data_ptr(),
                                           status.data_ptr(), ws.data_ptr(), nb.value, stream))
    length, _n_ext, bad = (int(x) for x in status.cpu().tolist())
    if bad:
        raise ValueError(f"merge_related_nodes: {bad} invalid node ids / weights")
    return out[:length]


def window_dup_layout(local_partitions, device=None, min_count: int = 2):
    """The duplicate-node layout of a rank's windows in one GPU pass
    (``ngt_window_dup_layout``): _compute_local_duplicate_nodes
    (NeutronGT/core/node_level_pipeline/window_state.py:52-73) followed by
    build_dup_cache_metadata (:181-205).

    ``local_partitions``: the rank's windows, 1-D integer tensors (CPU or GPU).
    A node is a duplicate when it occurs ``min_count`` or more times over all
    of them.  Returns (reranged, dup_nodes_per_partition, cache_ids,
    dup_indices), int64 on ``device`` (default: the current GPU):
    ``reranged[w]`` is window w with its duplicates first, both parts in their
    original order; ``dup_nodes_per_partition[w]`` its leading duplicates;
    ``cache_ids`` the sorted unique duplicates (the rows the feature cache
    holds); ``dup_indices[w]`` the cache position of each of window w's
    duplicates.  One device-to-host read (the counts)."""
    parts = list(local_partitions)
    dev = torch.device(device) if device is not None else torch.device(
        "cuda", torch.cuda.current_device())
    if dev.type != "cuda":
        raise ValueError("window_dup_layout runs on the GPU")
    empty = lambda: torch.empty((0,), dtype=torch.long, device=dev)  # noqa: E731
    if not parts:
        return [], [], empty(), []
    lens = [int(p.numel()) for p in parts]
    T, W = sum(lens), len(parts)
    nodes = (torch.cat([p.reshape(-1).to(device=dev, dtype=torch.long) for p in parts])
             if T else empty())
    ptr = [0]
    for n in lens:
        ptr.append(ptr[-1] + n)
    win_ptr = torch.tensor(ptr, dtype=torch.long).to(dev)
    lib = _lib.load()
    nb = C.c_size_t()
    _lib.check(lib.ngt_window_dup_workspace_bytes(T, C.byref(nb)))
    ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=dev)
    reranged = torch.empty(max(T, 1), dtype=torch.long, device=dev)
    cache_ids = torch.empty(max(T, 1), dtype=torch.long, device=dev)
    dup_index = torch.empty(max(T, 1), dtype=torch.long, device=dev)
    # the counts come back in one copy: info[3] then dup_ptr[W + 1]
    counts = torch.empty(3 + W + 1, dtype=torch.long, device=dev)
    info, dup_ptr = counts[:3], counts[3:]
    _lib.check(lib.ngt_window_dup_layout(
        nodes.data_ptr() if T else None, T, win_ptr.data_ptr(), W, int(min_count),
        reranged.data_ptr(), dup_ptr.data_ptr(), cache_ids.data_ptr(), dup_index.data_ptr(),
        info.data_ptr(), ws.data_ptr(), nb.value, _lib.stream_ptr(dev)))
    host = counts.tolist()
    n_cache, _total, bad = host[:3]
    dptr = host[3:]
    if bad:
        raise ValueError(f"window_dup_layout: {bad} nodes outside the windows (internal error)")
    rer = list(torch.split(reranged[:T], lens)) if T else [empty() for _ in parts]
    dups = [r[: dptr[w + 1] - dptr[w]] for w, r in enumerate(rer)]
    idx = [dup_index[dptr[w]: dptr[w + 1]] for w in range(W)]
    return rer, dups, cache_ids[:n_cache], idx


def duplicate_rerange(local_partitions, device=None):
    """_compute_local_duplicate_nodes (window_state.py:52-73) on the GPU:
    nodes present in >= 2 of a rank's windows move to the front of each
    window (original order kept).  Returns (reranged, dup_nodes_per_partition)
    as int64 GPU tensors."""
    rer, dups, _, _ = window_dup_layout(local_partitions, device=device, min_count=2)
    return rer, dups


def dup_cache_metadata(dup_lists, device=None):
    """build_dup_cache_metadata (window_state.py:181-205) on the GPU:
    (cache_ids = the sorted unique ids of ``dup_lists``, per-window indices
    into it).  Empty ``dup_lists`` give an empty cache and an empty list, as
    the reference's early return does."""
    if not list(dup_lists):
        dev = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        return torch.empty((0,), dtype=torch.long, device=dev), []
    _, _, cache_ids, idx = window_dup_layout(dup_lists, device=device, min_count=1)
    return cache_ids, idx


def dup_feature_cache(feature: torch.Tensor, cache_ids: torch.Tensor) -> torch.Tensor:
    """feature[cache_ids] on the GPU (the reference's
    local_dup_nodes_per_partition_feature, window_state.py:204): the cache of
    duplicate nodes' feature rows that assemble_window_features reads."""
    out, bad = gather_rows(feature, cache_ids.to(feature.device))
    if cache_ids.numel() and int(bad.item()):
        raise IndexError("dup_feature_cache: cache id outside the feature table")
    return out


def gather_rows(src: torch.Tensor, idx: torch.Tensor, out: torch.Tensor | None = None):
    """out[r] = src[idx[r]] on the GPU (bit copy).  Raises IndexError on a bad index."""
    lib = _lib.load()
    if not (src.is_cuda and idx.is_cuda):
        raise ValueError("gather_rows: tensors must be on the GPU")
    src = src.contiguous()
    idx = idx.to(torch.int64).contiguous()
    row_bytes = src[0].numel() * src.element_size() if src.dim() > 1 else src.element_size()
    if out is None:
        out = torch.empty((idx.numel(),) + tuple(src.shape[1:]), dtype=src.dtype, device=src.device)
    bad = torch.zeros(1, dtype=torch.int32, device=src.device)
    if row_bytes % 4:
        raise ValueError("gather_rows: row size must be a multiple of 4 bytes")
    stream = _lib.stream_ptr(src.device)
    _lib.check(lib.ngt_gather_rows(src.data_ptr(), int(src.shape[0]), idx.data_ptr(),
                                   int(idx.numel()), int(row_bytes), out.data_ptr(),
                                   bad.data_ptr(), stream))
    return out, bad


_SUBGRAPH_ERRORS = {1: "node id out of range in the node set", 2: "duplicate node in the node set",
                    4: "edge endpoint out of range", 8: "CSR row outside col"}


def _subgraph_job(call, n_nodes: int, n_edges: int, n_set: int, device, stream, host):
    """Count pass, the count copied into ``host`` (pinned) asynchronously, a
    yield, then the emit pass into an exact [2, n] tensor: a job of
    _streams.run_in_flight."""
    lib = _lib.load()
    nb = C.c_size_t()
    _lib.check(lib.ngt_subgraph_workspace_bytes(n_nodes, n_edges, n_set, C.byref(nb)))
    with torch.cuda.stream(stream):
        ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=device)
        result = torch.zeros(2, dtype=torch.int64, device=device)
    sp = stream.cuda_stream
    _lib.check(call(None, 0, result.data_ptr(), ws.data_ptr(), nb.value, sp))
    with torch.cuda.stream(stream):
        host[:2].copy_(result, non_blocking=True)
    landed = torch.cuda.Event()
    landed.record(stream)
    yield
    landed.synchronize()
    n, err = int(host[0]), int(host[1])
    if err:
        why = ", ".join(m for b, m in _SUBGRAPH_ERRORS.items() if err & b)
        raise IndexError(f"subgraph: {why}")
    with torch.cuda.stream(stream):
        out = torch.empty(2, n, dtype=torch.int64, device=device)
    if n:
        _lib.check(call(out.data_ptr(), n, result.data_ptr(), ws.data_ptr(), nb.value, sp))
    return out


def _coo_call(subset: torch.Tensor, edge_index: torch.Tensor, num_nodes: int):
    lib = _lib.load()
    if not (subset.is_cuda and edge_index.is_cuda):
        raise ValueError("subgraph: tensors must be on the GPU")
    if edge_index.dim() != 2 or edge_index.shape[0] != 2:
        raise ValueError(f"subgraph: edge_index must be [2, E], got {tuple(edge_index.shape)}")
    subset = subset.to(torch.int64).contiguous()
    ei = edge_index.to(torch.int64).contiguous()
    E, n_set = int(ei.shape[1]), int(subset.numel())
    call = lambda out, cap, res, ws, wb, st: lib.ngt_subgraph_coo(  # noqa: E731
        ei.data_ptr(), E, int(num_nodes), subset.data_ptr(), n_set, out, cap, res, ws, wb, st)
    return functools.partial(_subgraph_job, call, int(num_nodes), E, n_set, subset.device)


def _csr_call(node_set: torch.Tensor, rowptr: torch.Tensor, col: torch.Tensor):
    lib = _lib.load()
    if not (node_set.is_cuda and rowptr.is_cuda and col.is_cuda):
        raise ValueError("subgraph_from_csr: tensors must be on the GPU")
    node_set = node_set.to(torch.int64).contiguous()
    rowptr = rowptr.to(torch.int64).contiguous()
    col = col.to(torch.int64).contiguous()
    n_nodes, n_set = int(rowptr.numel()) - 1, int(node_set.numel())
    if n_nodes < 0:
        raise ValueError("subgraph_from_csr: rowptr must have n_nodes + 1 entries")
    call = lambda out, cap, res, ws, wb, st: lib.ngt_subgraph_csr(  # noqa: E731
        rowptr.data_ptr(), col.data_ptr(), int(col.numel()), n_nodes, node_set.data_ptr(), n_set,
        out, cap, res, ws, wb, st)
    return functools.partial(_subgraph_job, call, n_nodes, int(col.numel()), n_set,
                             node_set.device)


def subgraph(subset: torch.Tensor, edge_index: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """torch_geometric.utils.subgraph(subset, edge_index, relabel_nodes=True,
    num_nodes)[0] on the GPU (window_state.py:82,127; metisPartition.py:280,290):
    the edges with both endpoints in ``subset``, in their original order, each
    node renamed to its position in ``subset``.  int64 [2, E_sub].  Raises
    IndexError on ids outside [0, num_nodes) or a repeated subset node."""
    job = _coo_call(subset, edge_index, num_nodes)
    return _streams.run_in_flight([job], subset.device, 1)[0]


def subgraph_from_csr(node_set: torch.Tensor, rowptr: torch.Tensor, col: torch.Tensor) -> torch.Tensor:
    """_subgraph_from_csr (window_state.py:92-119) on the GPU: for each node of
    ``node_set`` in order, its CSR neighbours (CSR order) inside the set, as
    (position of the row node, position of the neighbour).  int64 [2, E_sub]."""
    job = _csr_call(node_set, rowptr, col)
    return _streams.run_in_flight([job], node_set.device, 1)[0]


def subgraphs_from_csr(node_sets, rowptr: torch.Tensor, col: torch.Tensor,
                       streams: int = 4) -> list:
    """subgraph_from_csr for each of ``node_sets``, up to ``streams`` windows
    in flight (each on a stream of its own; same results).  Each window's
    walk touches only its own rows, so on a large graph the windows' count
    read-backs and small passes overlap (the COO form streams the whole edge
    list per window and fills the GPU alone, so it has no such variant)."""
    jobs = [_csr_call(s, rowptr, col) for s in node_sets]
    return _streams.run_in_flight(jobs, rowptr.device, streams) if jobs else []


def assemble_window_features(feature: torch.Tensor, cache: torch.Tensor, dup_index: torch.Tensor,
                             partition: torch.Tensor, check: bool = True) -> torch.Tensor:
    """x_i = cat(cache[dup_index], feature[partition[n_dup:]]) as two GPU
    gathers into one buffer (feature and cache resident in HBM)."""
    n_dup = int(dup_index.numel())
    part = partition.to(feature.device)
    n = int(part.numel())
    out = torch.empty((n,) + tuple(feature.shape[1:]), dtype=feature.dtype, device=feature.device)
    bads = []
    if n_dup:
        _, b = gather_rows(cache, dup_index.to(feature.device), out[:n_dup])
        bads.append(b)
    if n - n_dup:
        _, b = gather_rows(feature, part[n_dup:], out[n_dup:])
        bads.append(b)
    if check and bads and int(sum(b for b in bads).item()):
        raise IndexError("assemble_window_features: index out of range")
    return out


def adj_weights(edge_index: torch.Tensor, ppr_val: torch.Tensor):
    """Symmetric int32 METIS adjacency + weights from a PPR edge list
    (build_adj_fromat, NeutronGT/core/ppr_preprocess.py:30-71), on the GPU
    (``ngt_adj_weights``).

    w = int32(clamp_min(fp32 sum of the PPR values of {u,v} * 1000, 1)), the
    values of a key added in entry order from 0 (fixed, not atomic); rows in
    ascending node order; inside row u the (u, v>u) keys come first in
    ascending v, then the (v<u, u) keys in ascending v (stable order).  The
    node count is max(edge_index) + 1 (one device-to-host read, as in the
    reference).  Returns (xadj, adjncy, eweights) int32 on edge_index's device.
    """
    dev = edge_index.device
    if not edge_index.is_cuda:
        raise ValueError("adj_weights runs on the GPU (edge_index is on the CPU)")
    if edge_index.numel() == 0:
        z = torch.zeros(0, dtype=torch.int32, device=dev)
        return torch.zeros(1, dtype=torch.int32, device=dev), z, z
    ei = edge_index.to(torch.int64).contiguous()
    val = ppr_val.to(device=dev, dtype=torch.float32).contiguous()
    E = int(ei.shape[1])
    if val.numel() != E:
        raise ValueError(f"{val.numel()} PPR values for {E} entries")
    n = int(ei.max().item()) + 1
    lib = _lib.load()
    nb = C.c_size_t()
    _lib.check(lib.ngt_adj_weights_workspace_bytes(E, n, C.byref(nb)))
    ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=dev)
    xadj = torch.empty(n + 1, dtype=torch.int32, device=dev)
    adjncy = torch.empty(2 * E, dtype=torch.int32, device=dev)
    ew = torch.empty(2 * E, dtype=torch.int32, device=dev)
    info = torch.empty(3, dtype=torch.int64, device=dev)
    _lib.check(lib.ngt_adj_weights(ei.data_ptr(), val.data_ptr(), E, n, xadj.data_ptr(),
                                   adjncy.data_ptr(), ew.data_ptr(), info.data_ptr(),
                                   ws.data_ptr(), nb.value, _lib.stream_ptr(dev)))
    u, bad, big = (int(x) for x in info.tolist())
    if bad or big:
        raise ValueError(f"adj_weights: {bad} entries with a negative id, {big} weights >= 2^31")
    return xadj, adjncy[: 2 * u], ew[: 2 * u]


class LocalWindows:
    """A rank's window structures as _rebuild_local_window_structures keeps
    them (NeutronGT/core/node_level_pipeline/window_state.py:223-260), on the
    GPU: ``partitions`` (duplicates first when the cache is used),
    ``dup_nodes`` and ``dup_indices`` per window, ``feature_cache`` (the
    duplicate nodes' feature rows), ``sub_edge_index`` per window (the
    induced subgraph relabelled by position in its partition) and ``timings``
    (seconds, the reference's timing_stats keys; each step synchronised)."""

    def __init__(self, partitions, dup_nodes, dup_indices, feature_cache, sub_edge_index,
                 timings):
        self.partitions = partitions
        self.dup_nodes = dup_nodes
        self.dup_indices = dup_indices
        self.feature_cache = feature_cache
        self.sub_edge_index = sub_edge_index
        self.timings = timings

    def features(self, i: int, feature: torch.Tensor) -> torch.Tensor:
        """x_i of window i (train_eval.py:234-242): its duplicates' rows from
        the cache, the rest from ``feature``; bitwise feature[partition]."""
        idx = self.dup_indices[i] if self.dup_indices else torch.empty(
            (0,), dtype=torch.long, device=feature.device)
        return assemble_window_features(feature, self.feature_cache, idx, self.partitions[i])


def rebuild_local_windows(local_partitions, feature: torch.Tensor, use_cache: bool = True,
                          edge_index: torch.Tensor | None = None, num_nodes: int | None = None,
                          rowptr: torch.Tensor | None = None, col: torch.Tensor | None = None,
                          streams: int = 4):
    """_rebuild_local_window_structures (window_state.py:223-260) for one rank,
    every step on the GPU: with ``use_cache`` the duplicate layout and its
    feature cache (:52-73, :181-205; window_dup_layout), then each window's
    induced subgraph, from the global COO ``edge_index`` (PyG subgraph,
    :122-133) or, without it, from the global CSR ``rowptr``/``col``
    (_subgraph_from_csr, :92-119, 134-140).  ``feature`` [num_nodes, F] on
    the GPU.  The struct_enc spatial positions (:247-256) are not built.
    ``streams``: windows whose CSR-walk subgraphs are built at once, each on
    a stream of its own (same result).  Returns a LocalWindows."""
    import time

    dev = feature.device
    if not feature.is_cuda:
        raise ValueError("rebuild_local_windows: feature must be on the GPU")
    if edge_index is None and (rowptr is None or col is None):
        raise ValueError("rebuild_local_windows: give edge_index (+ num_nodes) or rowptr and col")
    parts = [p.reshape(-1).to(device=dev, dtype=torch.long) for p in local_partitions]
    timings = {"local_dup_cache_rebuild_time": 0.0, "local_subgraph_rebuild_time": 0.0,
               "local_spatial_rebuild_time": 0.0}
    torch.cuda.synchronize(dev)
    t = time.perf_counter()
    if use_cache and parts:
        parts, dups, cache_ids, idx = window_dup_layout(parts, device=dev)
        cache = dup_feature_cache(feature, cache_ids)
    else:
        dups = [torch.empty((0,), dtype=torch.long, device=dev) for _ in parts]
        idx = []
        cache = torch.empty((0,) + tuple(feature.shape[1:]), dtype=feature.dtype, device=dev)
    torch.cuda.synchronize(dev)
    timings["local_dup_cache_rebuild_time"] = time.perf_counter() - t
    t = time.perf_counter()
    if edge_index is not None:
        n = int(num_nodes) if num_nodes is not None else int(feature.shape[0])
        subs = [subgraph(p, edge_index, n) for p in parts]
    else:
        subs = subgraphs_from_csr(parts, rowptr, col, streams=streams)
    torch.cuda.synchronize(dev)
    timings["local_subgraph_rebuild_time"] = time.perf_counter() - t
    return LocalWindows(parts, dups, idx, cache, subs, timings)
