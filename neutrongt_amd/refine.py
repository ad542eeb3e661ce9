"""Window refinement on the GPU: node_out / node_in.

Mirrors weightMetis_keepParent.node_out and node_in
(NeutronGT/core/metisPartition.py:160-287), which the training loop calls when
the loss plateaus (NeutronGT/main_sp_node_level_ppr.py:225-247) with the last
layer's node scores of every window:

  node_out  keeps the top max(int(N*(1-ratio)), 1) nodes of each window by node
            score, rebuilds the window's edge list (induced subgraph,
            ngt_subgraph_coo) and puts the expired nodes in a shared buffer;
  node_in   refills each window with the buffered nodes that receive the most
            PPR mass from it (fp32 sums in PPR-edge order, ngt_segment_sum_f32)
            and rebuilds its edge list from the global graph.

Everything stays on the GPU (int64 node ids, the buffer as a tensor multiset).
Ties: the reference ranks with torch.argsort / torch.topk, whose order among
equal scores is implementation-defined; here the lower window position
(node_out) or the lower node id (node_in) wins, so results are deterministic.
The reference's node_in returns at the first window with nothing to recover
(metisPartition.py:169-172) or no candidate outside it (:180-181); kept, so the
same windows change.
"""
from __future__ import annotations

import torch

from . import _lib
from .window import subgraph


def _segment_sum(vals: torch.Tensor, seg: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    n_seg = int(seg.numel()) - 1
    out = torch.empty(max(n_seg, 0), dtype=torch.float32, device=vals.device)
    bad = torch.zeros(1, dtype=torch.int32, device=vals.device)
    if n_seg > 0:
        _lib.check(lib.ngt_segment_sum_f32(vals.data_ptr(), int(vals.numel()), seg.data_ptr(),
                                           n_seg, out.data_ptr(), bad.data_ptr(),
                                           _lib.stream_ptr(vals.device)))
    return out


def _check_ids(num_nodes: int, *tensors):
    """Node ids index device tables here: reject any outside [0, num_nodes)
    on the host (one sync) instead of letting an index assert fire."""
    parts = [t.reshape(-1) for t in tensors if t.numel()]
    if not parts:
        return
    both = torch.stack([torch.stack([p.min(), p.max()]) for p in parts])
    lo, hi = int(both[:, 0].min()), int(both[:, 1].max())
    if lo < 0 or hi >= num_nodes:
        raise IndexError(f"node id out of range [0, {num_nodes}): min {lo}, max {hi}")


def node_out_window(nodes: torch.Tensor, edge_index: torch.Tensor, node_scores: torch.Tensor,
                    remove_ratio: float = 0.1):
    """One window of node_out (metisPartition.py:224-287).  Returns (kept
    nodes, their relabelled edge_index, expired nodes), all on the GPU."""
    n = int(nodes.numel())
    if node_scores.dim() != 1 or int(node_scores.numel()) != n:
        raise ValueError(f"node score shape {tuple(node_scores.shape)} does not match the window "
                         f"({n} nodes)")
    num_keep = max(int(n * (1 - remove_ratio)), 1)
    order = torch.sort(node_scores.float(), descending=True, stable=True).indices
    keep = torch.sort(order[:num_keep]).values
    expire = torch.sort(order[num_keep:]).values
    return nodes[keep], subgraph(keep, edge_index, n), nodes[expire]


def node_in_window(nodes: torch.Tensor, buffer: torch.Tensor, ppr_edge_index: torch.Tensor,
                   ppr_val: torch.Tensor, num_to_recover: int, edge_index: torch.Tensor,
                   num_nodes: int):
    """One window of node_in (metisPartition.py:160-222).  Returns None when no
    buffered node lies outside the window, else (new sorted nodes, their
    edge_index from the global graph, remaining buffer)."""
    dev = nodes.device
    _check_ids(num_nodes, nodes, buffer, ppr_edge_index)
    in_window = torch.zeros(num_nodes, dtype=torch.bool, device=dev)
    in_window[nodes] = True
    cand = torch.unique(buffer)
    valid = cand[~in_window[cand]]
    if valid.numel() == 0:
        return None
    real_add = min(int(num_to_recover), int(valid.numel()))
    # PPR entries from a window node to a candidate, in PPR-edge order; a
    # position table replaces the reference's two isin passes
    cand_pos = torch.full((num_nodes,), -1, dtype=torch.int64, device=dev)
    cand_pos[valid] = torch.arange(valid.numel(), device=dev)
    pos = cand_pos[ppr_edge_index[1]]
    keep = in_window[ppr_edge_index[0]] & (pos >= 0)
    idx = pos[keep]
    contrib = ppr_val[keep].float()
    # group the contributions per candidate, keeping their PPR-edge order, and
    # add them one by one (the rounding of the reference's index_add_)
    grouped = contrib[torch.sort(idx, stable=True).indices]
    seg = torch.zeros(valid.numel() + 1, dtype=torch.int64, device=valid.device)
    seg[1:] = torch.cumsum(torch.bincount(idx, minlength=valid.numel()), 0)
    scores = _segment_sum(grouped.contiguous(), seg)
    selected = valid[torch.sort(scores, descending=True, stable=True).indices[:real_add]]
    remaining = torch.sort(buffer).values
    keep = torch.ones(remaining.numel(), dtype=torch.bool, device=remaining.device)
    keep[torch.searchsorted(remaining, selected)] = False
    new_nodes = torch.sort(torch.cat([nodes, selected])).values
    return new_nodes, subgraph(new_nodes, edge_index, num_nodes), remaining[keep]


class WindowRefiner:
    """The window state node_out / node_in share in the reference
    (partitioned_results, sub_edge_index_for_partition_results,
    global_expired_node_buffer, partition_expired_node_num), on the GPU."""

    def __init__(self, partitions, sub_edge_indices, edge_index: torch.Tensor, num_nodes: int,
                 ppr_edge_index: torch.Tensor, ppr_val: torch.Tensor):
        self.partitioned_results = [p.to(torch.int64) for p in partitions]
        self.sub_edge_index_for_partition_results = [e.to(torch.int64) for e in sub_edge_indices]
        self.global_edge_index = edge_index.to(torch.int64)
        self.num_nodes = int(num_nodes)
        self.ppr_edge_index = ppr_edge_index.to(torch.int64)
        self.ppr_val = ppr_val
        dev = self.global_edge_index.device
        self.global_expired_node_buffer = torch.zeros(0, dtype=torch.int64, device=dev)
        self.partition_expired_node_num = {}

    def node_out(self, score_of_partition_list, remove_ratio: float = 0.1):
        for i in range(len(self.partitioned_results)):
            nodes, edges, expired = node_out_window(
                self.partitioned_results[i], self.sub_edge_index_for_partition_results[i],
                score_of_partition_list[i], remove_ratio)
            if expired.numel():
                self.partition_expired_node_num[i] = int(expired.numel())
                self.global_expired_node_buffer = torch.cat([self.global_expired_node_buffer,
                                                             expired])
            self.partitioned_results[i] = nodes
            self.sub_edge_index_for_partition_results[i] = edges

    def node_in(self):
        for i in range(len(self.partitioned_results)):
            num = self.partition_expired_node_num.get(i, 0)
            if num <= 0 or self.global_expired_node_buffer.numel() == 0:
                self.partition_expired_node_num[i] = 0
                return
            r = node_in_window(self.partitioned_results[i], self.global_expired_node_buffer,
                               self.ppr_edge_index, self.ppr_val, num, self.global_edge_index,
                               self.num_nodes)
            if r is None:
                return
            (self.partitioned_results[i], self.sub_edge_index_for_partition_results[i],
             self.global_expired_node_buffer) = r
            self.partition_expired_node_num[i] = 0
