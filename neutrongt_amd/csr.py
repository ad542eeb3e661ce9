"""Device-resident window adjacency (CSR + transposed CSR + work lists).

The reference hands the attention core a COO ``edge_index`` [2, E] (row 0 =
key/src, row 1 = query/dst; NeutronGT/core/node_level_pipeline/
window_state.py:122-140) and re-derives the grouping with gathers and scatter
adds on every call (NeutronGT/models/graphormer_dist_node_level.py:75-97).
Here the window's edge_index is converted once on the GPU
(``ngt_csr_build``) and cached (AdjacencyCache): found again by the same
edge_index object (every layer of a window step) or by equal contents (a
fresh device copy of the window's edges each step).
"""
from __future__ import annotations

import ctypes as C
import math
import os
import weakref
from collections import OrderedDict

import torch

from . import _lib

# A work item covers at most this many edges of one row; longer rows are cut
# into chunks whose partial sums a finalize pass adds.  With the kernels'
# 8 edge slots per wave (8 heads per pass) a 256-edge chunk is 32 rounds of a
# wave.
CHUNK_EDGES = 256
CHUNK_EDGES_MIN = 128
CHUNK_EDGES_MAX = 1024


def chunk_for_heads(n_heads: int, n_edges: int = 0) -> int:
    """Edges per work item: 2^floor(log2(n_edges / 2048)) within [128, 1024]
    (256 when n_edges is not given).  Longer chunks mean fewer partials and
    smaller finalize passes, but a hub row's chunk is one wave's serial work,
    which must stay short next to the whole kernel.  Measured on the current
    kernels: the high-degree window (3.67 M edges) 272 / 264 / 322 us per layer
    at 512 / 1024 / 2048; GPH_Large (1.79 M) 16.47 / 16.35 / 16.72 ms per
    12-layer step at 256 / 512 / 1024 (at 256 its key-major pass gains 6 us and
    the query-major pass and the finalizes lose 19); GPH_Slim and the GT arxiv
    window (0.25 M) at 128 / 256 as HIP-graph replays 62.3 / 63.9 and 71.8 /
    75.8 us (their key-major pass is one round of waves, as long as its
    longest chunk; 64 gave no more; 512 and 1024 had cost them 40-120 %).  The head count does not enter; the argument keeps the
    callers' form.  NGT_CHUNK_EDGES overrides the choice."""
    del n_heads
    env = os.environ.get("NGT_CHUNK_EDGES")
    if env and int(env) > 0:
        return int(env)
    if n_edges <= 0:
        return CHUNK_EDGES
    chunk = CHUNK_EDGES_MIN
    while chunk < CHUNK_EDGES_MAX and 2 * chunk * 2048 <= n_edges:
        chunk *= 2
    return chunk


def small_for_heads(n_heads: int) -> int:
    """Rows with at most this many edges are packed one row per edge slot
    (no cross-slot reduction, no per-row work item): 64 / next_pow2(H), the
    slots per wave of an all-heads pass, except 16 at 5-8 heads and 32 from
    H = 32 on.  At 5-8 heads this is the key-major list's threshold, and the
    query-major list's comes from the window's degrees (pack_q_adaptive).  On the 32,768-query window (H = 32, d = 24) raising it from 2
    to 32 took the layer from 1.45 to 1.40 ms.  At H = 8 with 128-edge chunks
    (HIP-graph replays, us per layer at 8 / 12 / 16 / 24 / 32): GPH_Slim
    61.9 / 58.6 / 56.5 / 60.5 / 68.1, the GT arxiv window 72.0 / 69.7 / 66.0 /
    64.4 / 72.7, the high-degree window 312-314 throughout."""
    lanes = 1
    while lanes < n_heads:
        lanes <<= 1
    if n_heads >= 32:
        return 32
    if lanes == 8:
        return 16
    return max(1, 64 // lanes)


def pack_q_adaptive(n_heads: int) -> bool:
    """Whether the query-major packing threshold is read from the window's
    degrees (5-8 heads).  A packed row is walked serially by one edge slot, a
    longer row by a whole wave, and the best threshold follows the degree
    distribution rather than the head count.  HIP-graph replays, us per layer
    at thresholds 8 / 16 / 24 / 32 / 48 (in brackets the share of query rows
    that the chosen threshold packs):
      GT arxiv window,  0 related keys: 51.3 / 49.5 / 53.4 / 54.0 / 62.3 (16: 0.85)
                        4 related keys: 60.5 / 55.9 / 58.7 / 63.6 / 68.4 (16: 0.79)
                        8 related keys: 68.1 / 64.9 / 62.2 / 67.9 / 73.1 (24: 0.85)
                       16 related keys: 78.5 / 78.2 / 81.2 / 75.8 / 81.7 (32: 0.85)
      GPH_Slim, mean degree  8:         47.7 / 48.6 / 52.5 / 54.9 / 63.8 ( 8: 0.82)
                mean degree 14:         58.8 / 56.6 / 60.0 / 64.0 / 72.5 (16: 0.86)
                mean degree 28:         85.1 / 85.3 / 85.9 / 87.8 / 91.1 (24: 0.80)
    The first step that packs at least 78 % of the rows is within 1 % of the
    best threshold on all seven windows; ngt_csr_build applies that rule on
    the device (small_q = NGT_SMALL_FROM_DEGREES) from the degrees it sorts
    anyway, so the choice costs no extra host round trip."""
    return 4 < n_heads <= 8


class WindowAdjacency:
    """Both CSR orientations of one window plus its work lists (int32, on device)."""

    def __init__(self, edge_index: torch.Tensor, n_q: int, n_k: int, chunk: int, small: int = 0,
                 pack_q: bool = False, tiled: bool = True):
        """``tiled``: also build the rows' degree orders (order_q, order_k), which
        let the library run its tiled kernels on dense windows; without them
        every window runs the work-list kernels."""
        if edge_index.dim() != 2 or edge_index.shape[0] != 2:
            raise ValueError(f"edge_index must be [2, E], got {tuple(edge_index.shape)}")
        if not edge_index.is_cuda:
            raise ValueError("edge_index must be on the GPU")
        lib = _lib.load()
        dev = edge_index.device
        ei = edge_index.to(torch.int64).contiguous()
        E = int(ei.shape[1])
        self.edge_index = edge_index  # pins the cache key's storage
        # a later tensor with the same contents (AdjacencyCache): weak reference, version
        self.alias, self.alias_version = None, None
        self.n_q, self.n_k, self.n_edges, self.chunk = int(n_q), int(n_k), E, int(chunk)
        small = int(min(max(small, 0), chunk - 1))
        self.small = small  # key-major threshold (and query-major unless pack_q)
        small_q = _lib.SMALL_FROM_DEGREES if pack_q else small
        miq, msq, mik, msk = (C.c_int32() for _ in range(4))
        _lib.check(lib.ngt_csr_sizes(E, n_q, n_k, chunk, chunk, C.byref(miq), C.byref(msq),
                                     C.byref(mik), C.byref(msk)))
        # every device array of the window lives in one int32 allocation
        # (self.mem, 256-byte aligned slices), so that holding self.mem keeps
        # all memory the ngt_window_csr points into alive
        e1 = max(E, 1)
        layout = (("rowptr", (n_q + 1,)), ("col", (e1,)), ("perm", (e1,)),
                  ("t_rowptr", (n_k + 1,)), ("t_col", (e1,)), ("t_perm", (e1,)), ("q2t", (e1,)),
                  ("items_q", (miq.value, 4)), ("splits_q", (msq.value, 4)),
                  ("items_k", (mik.value, 4)), ("splits_k", (msk.value, 4)),
                  ("packed_q", (max(n_q, 1),)), ("packed_k", (max(n_k, 1),)),
                  ("info_dev", (_lib.INFO_LEN,)))
        if tiled:
            layout = layout + (("order_q", (max(n_q, 1),)),
                               ("order_k", (max(min(n_q, n_k), 1),)))
        offs, total = [], 0
        for _, shape in layout:
            offs.append(total)
            total += -(-math.prod(shape) // 64) * 64
        self.mem = torch.empty(total, dtype=torch.int32, device=dev)
        for (name, shape), o in zip(layout, offs):
            setattr(self, name, self.mem[o:o + math.prod(shape)].view(shape))
        self.info_dev.zero_()
        s = _lib.WindowCSR()
        s.n_q, s.n_k, s.n_edges, s.chunk_q, s.chunk_k = n_q, n_k, E, chunk, chunk
        s.small_q, s.small_k = small_q, small
        for name in ("rowptr", "col", "perm", "t_rowptr", "t_col", "t_perm", "q2t", "items_q",
                     "splits_q", "packed_q", "items_k", "splits_k", "packed_k") + (
                         ("order_q", "order_k") if tiled else ()):
            setattr(s, name, getattr(self, name).data_ptr())
        self.tiled = tiled
        s.info = self.info_dev.data_ptr()
        s.max_items_q, s.max_splits_q = miq.value, msq.value
        s.max_items_k, s.max_splits_k = mik.value, msk.value
        ws_bytes = C.c_size_t()
        with torch.cuda.device(dev):
            _lib.check(lib.ngt_csr_workspace_bytes(E, n_q, n_k, C.byref(ws_bytes)))
            ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=dev)
            stream = _lib.stream_ptr(dev)
            _lib.check(lib.ngt_csr_build(ei.data_ptr() if E else None, C.byref(s), ws.data_ptr(),
                                         ws_bytes.value, stream))
            info = self.info_dev.cpu()  # one sync per window build
        del ws
        self.info = [int(x) for x in info.tolist()]
        self.small_q = self.info[_lib.INFO_SMALL_Q]  # the threshold the build used
        if self.info[_lib.INFO_BAD_EDGES]:
            raise IndexError(f"edge_index has {self.info[_lib.INFO_BAD_EDGES]} entries outside "
                             f"[0, {n_k}) x [0, {n_q}) (src x dst)")
        s.n_items_q = self.info[_lib.INFO_ITEMS_Q]
        s.n_parts_q = self.info[_lib.INFO_PARTS_Q]
        s.n_splits_q = self.info[_lib.INFO_SPLITS_Q]
        s.n_items_k = self.info[_lib.INFO_ITEMS_K]
        s.n_parts_k = self.info[_lib.INFO_PARTS_K]
        s.n_splits_k = self.info[_lib.INFO_SPLITS_K]
        s.n_packed_q = self.info[_lib.INFO_PACKED_Q]
        s.n_packed_k = self.info[_lib.INFO_PACKED_K]
        self.struct = s
        self.dst_end = self.info[_lib.INFO_DST_END]
        self.max_deg_q = self.info[_lib.INFO_MAX_DEG_Q]
        self.max_deg_k = self.info[_lib.INFO_MAX_DEG_K]
        self._ptr = C.byref(self.struct)
        self._ws_bytes = {}
        # the struct's bytes as a CPU tensor, for callers that keep a copy
        # (the C++ autograd node holds it with self.mem until its backward)
        self.csr_bytes = torch.frombuffer(bytearray(bytes(s)), dtype=torch.uint8)

    def ptr(self):
        return self._ptr

    def workspace_bytes(self, n_heads: int, head_dim: int):
        """(forward, backward) workspace bytes of ngt_sparse_fwd/bwd for this
        window and head shape, asked once and kept."""
        key = (int(n_heads), int(head_dim))
        hit = self._ws_bytes.get(key)
        if hit is None:
            fb, bb = C.c_size_t(), C.c_size_t()
            _lib.check(_lib.load().ngt_sparse_workspace_bytes(self._ptr, key[0], key[1],
                                                             C.byref(fb), C.byref(bb)))
            hit = self._ws_bytes[key] = (fb.value, bb.value)
        return hit


class AdjacencyCache:
    """LRU of WindowAdjacency, found by the edge_index tensor or by its contents.

    The same edge_index object (every layer of a window step) is a hit with no
    device work.  A new tensor with the same contents -- the reference's loop
    copies the window's edge_index to the device afresh every step
    (NeutronGT/core/node_level_pipeline/train_eval.py:244) -- is matched by a
    device-side comparison against the cached windows of the same shape (one
    host sync), and is remembered through a weak reference, so the other layers
    of its step hit without comparing again.  An entry whose own edge_index was
    modified in place is dropped.  The cache holds at most ``capacity``
    windows and ``max_bytes`` of device memory (their arenas and the
    edge_index tensors they keep), least recently used first out."""

    def __init__(self, capacity: int = 64, max_bytes: int = 2 << 30):
        self.capacity = capacity
        self.max_bytes = int(max_bytes)
        self._d: OrderedDict = OrderedDict()  # id -> (shape key, adjacency, version)
        self._next = 0
        self.builds = 0  # windows built (a test and bench counter)
        self.content_hits = 0

    @staticmethod
    def _nbytes(adj: WindowAdjacency) -> int:
        return adj.mem.numel() * 4 + adj.edge_index.numel() * adj.edge_index.element_size()

    def nbytes(self) -> int:
        return sum(self._nbytes(a) for _, a, _ in self._d.values())

    def get(self, edge_index: torch.Tensor, n_q: int, n_k: int, chunk: int,
            small: int = 0, pack_q: bool = False) -> WindowAdjacency:
        shape_key = (tuple(edge_index.shape), str(edge_index.device), edge_index.dtype, n_q, n_k,
                     chunk, small, pack_q)
        same_shape = []
        for eid in reversed(self._d):  # most recent first
            key, adj, ver = self._d[eid]
            if key != shape_key:
                continue
            if adj.edge_index._version != ver:
                continue  # stale: dropped below
            if adj.edge_index is edge_index:
                self._d.move_to_end(eid)
                return adj
            alias = adj.alias() if adj.alias is not None else None
            if alias is edge_index and adj.alias_version == edge_index._version:
                self._d.move_to_end(eid)
                return adj
            same_shape.append(eid)
        for eid in [e for e, (_, a, v) in self._d.items() if a.edge_index._version != v]:
            del self._d[eid]
        for eid in same_shape:
            adj = self._d[eid][1]
            if torch.equal(adj.edge_index, edge_index):  # one device compare + sync
                adj.alias = weakref.ref(edge_index)
                adj.alias_version = edge_index._version
                self._d.move_to_end(eid)
                self.content_hits += 1
                return adj
        adj = WindowAdjacency(edge_index, n_q, n_k, chunk, small, pack_q)
        self.builds += 1
        self._d[self._next] = (shape_key, adj, edge_index._version)
        self._next += 1
        total = self.nbytes()
        while len(self._d) > 1 and (len(self._d) > self.capacity or total > self.max_bytes):
            _, (_, old, _) = self._d.popitem(last=False)
            total -= self._nbytes(old)
        return adj

    def clear(self):
        self._d.clear()


# Sized for a training loop that cycles through every window of a graph each
# epoch: with fewer slots than windows, least-recently-used eviction misses on
# every step.  A GPH_Large window (32,768 queries, 1.79 M edges) takes about
# 70 MB with its edge_index, so 8 GiB holds the ~75 windows of an
# ogbn-products-sized graph, under 3 % of an MI355X's memory.
default_cache = AdjacencyCache(capacity=128, max_bytes=8 << 30)
