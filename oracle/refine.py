"""numpy restatement of window refinement (test oracle only).

weightMetis_keepParent.node_out / node_in, NeutronGT/core/metisPartition.py:160-287,
as driven by the training loop when the loss plateaus
(NeutronGT/main_sp_node_level_ppr.py:225-247).

Only the 1-D node-score form of node_out is restated (the attention core's
node_scores; metisPartition.py:239-242).  Ranking ties: the reference ranks
with torch.argsort(descending=True) (node_out) and torch.topk (node_in), whose
order among equal scores is implementation-defined; this restatement (and the
product) puts the lower window position (node_out) or the lower node id
(node_in) first.  node_in's candidate scores are fp32 sums in PPR-edge order,
which is what the reference's CPU index_add_ computes (np.add.at is the same
sequential, unbuffered accumulation).
"""
from __future__ import annotations

import numpy as np

from .graph import subgraph_coo


def node_out_window(nodes, edge_index, node_scores, remove_ratio: float):
    """One window of node_out (:224-287): keep the top max(int(N*(1-ratio)), 1)
    nodes by score.  Returns (kept nodes, their relabelled edges, expired nodes)."""
    nodes = np.asarray(nodes, np.int64)
    scores = np.asarray(node_scores, np.float32)
    n = nodes.size
    if scores.shape != (n,):
        raise ValueError(f"node score length {scores.shape} != window size {n}")
    num_keep = max(int(n * (1 - remove_ratio)), 1)
    order = np.argsort(-scores, kind="stable")
    keep = np.sort(order[:num_keep])
    expire = np.sort(order[num_keep:])
    return nodes[keep], subgraph_coo(keep, np.asarray(edge_index, np.int64), n), nodes[expire]


def node_in_window(nodes, buffer, ppr_edge_index, ppr_val, num_to_recover: int, edge_index,
                   num_nodes: int):
    """One window of node_in (:160-222) once it has something to recover.
    Returns None when no buffered node is outside the window (the reference
    returns from node_in there, :180-181), else (new nodes, their relabelled
    edges, remaining buffer as a sorted multiset)."""
    nodes = np.asarray(nodes, np.int64)
    buffer = np.asarray(buffer, np.int64)
    cand = np.unique(buffer)
    valid = cand[~np.isin(cand, nodes)]
    if valid.size == 0:
        return None
    real_add = min(int(num_to_recover), valid.size)
    src = np.asarray(ppr_edge_index[0], np.int64)
    dst = np.asarray(ppr_edge_index[1], np.int64)
    val = np.asarray(ppr_val, np.float32)
    mask_src = np.isin(src, nodes)
    dest, vals = dst[mask_src], val[mask_src]
    mask_dst = np.isin(dest, valid)
    scores = np.zeros(valid.size, np.float32)
    if mask_dst.any():
        np.add.at(scores, np.searchsorted(valid, dest[mask_dst]), vals[mask_dst])
    selected = valid[np.argsort(-scores, kind="stable")[:real_add]]
    remaining = np.sort(buffer)
    drop = np.searchsorted(remaining, selected)  # one occurrence of each selected node
    keep = np.ones(remaining.size, bool)
    keep[drop] = False
    new_nodes = np.sort(np.concatenate([nodes, selected]))
    return (new_nodes, subgraph_coo(new_nodes, np.asarray(edge_index, np.int64), num_nodes),
            remaining[keep])


class Refiner:
    """The state node_out / node_in share in the reference: windows, their edge
    lists, the expired-node buffer and the per-window expired counts."""

    def __init__(self, partitions, sub_edges, edge_index, num_nodes, ppr_edge_index, ppr_val):
        self.partitions = [np.asarray(p, np.int64) for p in partitions]
        self.sub_edges = [np.asarray(e, np.int64) for e in sub_edges]
        self.edge_index = np.asarray(edge_index, np.int64)
        self.num_nodes = int(num_nodes)
        self.ppr_edge_index = np.asarray(ppr_edge_index, np.int64)
        self.ppr_val = np.asarray(ppr_val, np.float32)
        self.buffer = np.zeros(0, np.int64)
        self.expired_num = {}

    def node_out(self, scores, remove_ratio=0.1):
        for i in range(len(self.partitions)):
            nodes, edges, expired = node_out_window(self.partitions[i], self.sub_edges[i],
                                                    scores[i], remove_ratio)
            if expired.size:  # the count is only updated when something expired (:268-272)
                self.expired_num[i] = int(expired.size)
                self.buffer = np.concatenate([self.buffer, expired])
            self.partitions[i], self.sub_edges[i] = nodes, edges

    def node_in(self):
        for i in range(len(self.partitions)):
            num = self.expired_num.get(i, 0)
            if num <= 0 or self.buffer.size == 0:
                # the reference returns from node_in at the first such window (:169-172)
                self.expired_num[i] = 0
                return
            r = node_in_window(self.partitions[i], self.buffer, self.ppr_edge_index, self.ppr_val,
                               num, self.edge_index, self.num_nodes)
            if r is None:
                return  # :180-181
            self.partitions[i], self.sub_edges[i], self.buffer = r
            self.expired_num[i] = 0
