"""Personalised PageRank preprocessing on the GPU (APPNP propagation with
per-row top-k), the step that feeds related-node selection and the METIS
weights.

``personal_pagerank_appnp`` keeps the signature and return value of the
reference's backend (NeutronGT/core/ppr_backends/appnp_backend.py:227-310):
batches of seed nodes start from their identity rows and are propagated
``num_iterations`` times,

    state <- topk_K( (1 - alpha) * state @ P + alpha * e_seed ),
    P[c, n] = 1 / max(deg(c), 1) for every edge c -> n,

with K = iter_topk (the shipped scripts run topk = iter_topk = 5, alpha 0.85,
10 iterations, batch 8192); the result keeps min(topk, iter_topk) entries per
seed and is returned as (edge_index [2, nnz] = (seed, node), values).  Each
step is ngt_ppr_count, one read-back of the product counts, then
ngt_ppr_step_direct: every (seed, node) sum evaluated where the node first
occurs in the seed's state lists (binary searches in the others, the products
added in the same order), the best K kept per chunk of a row and merged per
row; no product list is written or sorted.  Several batches are in flight at
once, each on a stream of its own, so that one batch's read-back overlaps the
others' kernels.  ``method="sort"`` runs the
product-list form instead (ngt_ppr_step: expansion, radix sort, ordered
segment sums, per-row top-k, on row chunks that bound the step's memory); the
two give the same bits.

Differences from the reference, by design:
  * iter_topk must be positive (1..64): without per-step pruning the state
    grows with the reachable set, which the reference itself warns about;
  * ties in the top-k go to the lower node id, and each (seed, node) sum is
    taken in a fixed order, so the result is deterministic (cuSPARSE plus an
    atomic scatter_add and torch.topk's tie order are not).
"""
from __future__ import annotations

import ctypes as C
import functools

import torch

from . import _lib, _streams

MAX_K = 64


def transition_csr(edge_index: torch.Tensor | None = None, csr_data: dict | None = None,
                   num_nodes: int | None = None, device="cuda"):
    """(rowptr int64, col int64, inv_deg fp32, num_nodes) of the graph, as
    _load_csr_graph / _build_csr_from_edge_index (appnp_backend.py:17-55) build
    it: rows sorted by (src, dst), inv_deg = 1 / max(out-degree, 1) in fp32."""
    dev = torch.device(device)
    if csr_data is not None:
        rowptr = torch.as_tensor(csr_data["rowptr"], dtype=torch.long, device=dev)
        col = torch.as_tensor(csr_data["col"], dtype=torch.long, device=dev)
        n = int(rowptr.numel() - 1)
        if num_nodes is not None and n != int(num_nodes):
            raise ValueError(f"CSR num_nodes mismatch: expected {num_nodes}, got {n}")
        deg = (rowptr[1:] - rowptr[:-1]).clamp_min(1).to(torch.float32)
        return rowptr, _sorted_rows(rowptr, col), 1.0 / deg, n
    if edge_index is None:
        raise ValueError("edge_index must be provided when csr_data is None")
    ei = edge_index.to(dev).long()
    if ei.numel() == 0:
        n = int(num_nodes or 0)
        z = torch.zeros(n + 1, dtype=torch.long, device=dev)
        return z, torch.empty(0, dtype=torch.long, device=dev), torch.ones(n, device=dev), n
    n = int(num_nodes) if num_nodes is not None else int(ei.max().item()) + 1
    order = torch.argsort(ei[0] * max(n, 1) + ei[1], stable=True)
    src, dst = ei[0][order], ei[1][order]
    counts = torch.bincount(src, minlength=n)
    rowptr = torch.zeros(n + 1, dtype=torch.long, device=dev)
    rowptr[1:] = torch.cumsum(counts, 0)
    return rowptr, dst.contiguous(), 1.0 / counts.clamp_min(1).to(torch.float32), n


def _sorted_rows(rowptr: torch.Tensor, col: torch.Tensor) -> torch.Tensor:
    """col with every CSR row's columns in ascending order (a stable sort by
    (row, column) when some row is not).  Sums do not depend on the order
    within a row: repeats of a column in one row carry the same product."""
    if col.numel() < 2:
        return col
    n = rowptr.numel() - 1
    deg = (rowptr[1:] - rowptr[:-1]).clamp_min(0)
    if int(rowptr[0]) != 0 or int(deg.sum()) != col.numel():
        return col  # malformed rows: left to the kernels' own checks
    desc = col[1:] < col[:-1]  # entry i: col[i + 1] below col[i]
    last = rowptr[1:-1] - 1    # a row's last entry may exceed the next row's first
    desc[last[(last >= 0) & (last < desc.numel())]] = False
    if not bool(desc.any()):
        return col
    row = torch.repeat_interleave(torch.arange(n, device=col.device), deg)
    lo = int(col.min())
    span = int(col.max()) - lo + 1
    order = torch.argsort(row * span + (col - lo), stable=True)
    return col[order].contiguous()


def max_repeats(rowptr: torch.Tensor, col: torch.Tensor) -> int:
    """The most times one column repeats within a CSR row whose columns are
    in ascending order (1 without duplicate edges)."""
    if col.numel() < 2:
        return 1
    same = col[1:] == col[:-1]  # entry i: col[i + 1] repeats col[i]
    last = rowptr[1:-1] - 1
    same[last[(last >= 0) & (last < same.numel())]] = False
    if not bool(same.any()):
        return 1
    idx = torch.arange(same.numel(), device=col.device)
    brk = torch.cummax(torch.where(same, torch.full_like(idx, -1), idx), 0).values
    return int((idx - brk).max()) + 1


def _check_status(status: torch.Tensor) -> None:
    bad, disorder = status.tolist()
    if bad:
        raise IndexError(f"personalised PageRank: {bad} node ids out of range")
    if disorder:
        raise ValueError("personalised PageRank: CSR rows must list their columns in ascending "
                         "order for the direct step (transition_csr sorts them), with no column "
                         "repeated more than max_mult times")


def _direct_batch(lib, rowptr, col, inv_deg, n_nodes: int, seeds: torch.Tensor, alpha: float,
                  K: int, num_iterations: int, max_mult: int, stream, host: torch.Tensor):
    """One batch through ngt_ppr_count + ngt_ppr_step_direct, all on
    ``stream``, as a job of _streams.run_in_flight: after each step's count it
    copies the product total into ``host[0]`` (pinned) asynchronously and
    yields; resumed, it waits for the copy and enqueues the step.  Returns
    (cols, vals, cnt, status)."""
    dev = seeds.device
    B = int(seeds.numel())
    sp = stream.cuda_stream
    with torch.cuda.stream(stream):
        st_col = torch.zeros(B, K, dtype=torch.int32, device=dev)
        st_val = torch.zeros(B, K, dtype=torch.float32, device=dev)
        st_col[:, 0] = seeds.to(torch.int32)
        st_val[:, 0] = 1.0
        st_cnt = torch.ones(B, dtype=torch.int32, device=dev)
        nx_col, nx_val, nx_cnt = (torch.empty_like(st_col), torch.empty_like(st_val),
                                  torch.empty_like(st_cnt))
        seeds = seeds.to(torch.int64).contiguous()
        status = torch.zeros(2, dtype=torch.int32, device=dev)
        row_off = torch.empty(B + 1, dtype=torch.int64, device=dev)
        cb = C.c_size_t()
        _lib.check(lib.ngt_ppr_count_workspace_bytes(B, C.byref(cb)))
        cws = torch.empty(cb.value, dtype=torch.uint8, device=dev)
    keep = float(1.0 - alpha)  # rounded to fp32 by ctypes, as fp32_tensor * (1 - alpha) is
    landed = torch.cuda.Event()
    for _ in range(num_iterations):
        _lib.check(lib.ngt_ppr_count(rowptr.data_ptr(), n_nodes, st_col.data_ptr(),
                                     st_cnt.data_ptr(), B, K, row_off.data_ptr(),
                                     status.data_ptr(), cws.data_ptr(), cb.value, sp))
        with torch.cuda.stream(stream):
            host[:1].copy_(row_off[B:], non_blocking=True)
        landed.record(stream)
        yield
        landed.synchronize()
        total = int(host[0])
        sb = C.c_size_t()
        _lib.check(lib.ngt_ppr_step_direct_workspace_bytes(total, B, K, C.byref(sb)))
        with torch.cuda.stream(stream):
            ws = torch.empty(sb.value, dtype=torch.uint8, device=dev)
        _lib.check(lib.ngt_ppr_step_direct(rowptr.data_ptr(), col.data_ptr(), inv_deg.data_ptr(),
                                           n_nodes, st_col.data_ptr(), st_val.data_ptr(),
                                           st_cnt.data_ptr(), seeds.data_ptr(), B, K,
                                           float(alpha), keep, int(max_mult), total,
                                           nx_col.data_ptr(), nx_val.data_ptr(),
                                           nx_cnt.data_ptr(), status.data_ptr(), ws.data_ptr(),
                                           sb.value, sp))
        st_col, nx_col = nx_col, st_col
        st_val, nx_val = nx_val, st_val
        st_cnt, nx_cnt = nx_cnt, st_cnt
    return st_col, st_val, st_cnt, status


def _run_direct(rowptr, col, inv_deg, n_nodes: int, seed_batches, alpha: float, K: int,
                num_iterations: int, max_mult: int, streams: int):
    """Propagates the seed batches through the direct step with up to
    ``streams`` batches in flight, each on a stream of its own (default
    priority; 1 = torch's current stream), and returns per batch (cols, vals,
    cnt), ready on the current stream.  Rows are independent, so the results
    do not depend on ``streams``: it lets the host's wait for one batch's
    product total overlap the other batches' kernels, and small steps of
    different batches share the GPU.  Raises after the last batch if any
    batch flagged an id out of range or a CSR row out of order."""
    lib = _lib.load()
    if not seed_batches:
        return []
    jobs = [functools.partial(_direct_batch, lib, rowptr, col, inv_deg, n_nodes, seeds, alpha, K,
                              num_iterations, max_mult) for seeds in seed_batches]
    results = _streams.run_in_flight(jobs, seed_batches[0].device, streams)
    _check_status(torch.stack([r[3] for r in results]).sum(0))
    return [r[:3] for r in results]


def appnp_batch(rowptr, col, inv_deg, n_nodes: int, seeds: torch.Tensor, alpha: float, K: int,
                num_iterations: int, max_products: int = 1 << 27, method: str = "direct",
                max_mult: int | None = None):
    """Propagates one batch of seed rows.  Returns (cols [B, K] int32,
    vals [B, K] fp32, cnt [B] int32), rows in rank order.  ``method``
    "direct" (ngt_ppr_step_direct; CSR rows must be in ascending column order,
    as transition_csr returns them; ``max_mult`` is max_repeats(rowptr, col),
    found here when None, and 0 turns its pruning off, with the same result)
    or "sort" (ngt_ppr_step), where a step whose product count exceeds
    ``max_products`` runs on consecutive row chunks (rows are independent),
    which bounds the step's workspace."""
    if not 1 <= K <= MAX_K:
        raise ValueError(f"per-step top-k must be in 1..{MAX_K}, got {K}")
    if method not in ("direct", "sort"):
        raise ValueError(f"method must be 'direct' or 'sort', got {method!r}")
    if method == "direct":
        if max_mult is None:
            max_mult = max_repeats(rowptr, col)
        return _run_direct(rowptr, col, inv_deg, n_nodes, [seeds], alpha, K, num_iterations,
                           max_mult, 1)[0]
    lib = _lib.load()
    dev = seeds.device
    B = int(seeds.numel())
    st_col = torch.zeros(B, K, dtype=torch.int32, device=dev)
    st_val = torch.zeros(B, K, dtype=torch.float32, device=dev)
    st_col[:, 0] = seeds.to(torch.int32)
    st_val[:, 0] = 1.0
    st_cnt = torch.ones(B, dtype=torch.int32, device=dev)
    nx_col, nx_val, nx_cnt = torch.empty_like(st_col), torch.empty_like(st_val), torch.empty_like(st_cnt)
    seeds = seeds.to(torch.int64).contiguous()
    status = torch.zeros(2, dtype=torch.int32, device=dev)
    row_off = torch.empty(B + 1, dtype=torch.int64, device=dev)
    cb = C.c_size_t()
    _lib.check(lib.ngt_ppr_count_workspace_bytes(B, C.byref(cb)))
    cws = torch.empty(cb.value, dtype=torch.uint8, device=dev)
    stream = _lib.stream_ptr(dev)
    keep = float(1.0 - alpha)  # rounded to fp32 by ctypes, as fp32_tensor * (1 - alpha) is

    def count(r0, r1, off):
        _lib.check(lib.ngt_ppr_count(rowptr.data_ptr(), n_nodes, st_col[r0:r1].data_ptr(),
                                     st_cnt[r0:r1].data_ptr(), r1 - r0, K, off.data_ptr(),
                                     status.data_ptr(), cws.data_ptr(), cb.value, stream))

    def step(r0, r1, off, total):
        sb = C.c_size_t()
        _lib.check(lib.ngt_ppr_step_workspace_bytes(total, r1 - r0, C.byref(sb)))
        ws = torch.empty(sb.value, dtype=torch.uint8, device=dev)
        _lib.check(lib.ngt_ppr_step(rowptr.data_ptr(), col.data_ptr(), inv_deg.data_ptr(),
                                    n_nodes, st_col[r0:r1].data_ptr(), st_val[r0:r1].data_ptr(),
                                    st_cnt[r0:r1].data_ptr(), seeds[r0:r1].data_ptr(), r1 - r0,
                                    K, float(alpha), keep, off.data_ptr(), total,
                                    nx_col[r0:r1].data_ptr(), nx_val[r0:r1].data_ptr(),
                                    nx_cnt[r0:r1].data_ptr(), status.data_ptr(), ws.data_ptr(),
                                    sb.value, stream))

    for _ in range(num_iterations):
        count(0, B, row_off)
        total = int(row_off[B])
        if total <= max_products:
            step(0, B, row_off, total)
        else:
            offs = row_off.cpu()
            r0 = 0
            while r0 < B:
                r1 = int(torch.searchsorted(offs, offs[r0] + max_products, right=True)) - 1
                r1 = min(max(r1, r0 + 1), B)
                part = torch.empty(r1 - r0 + 1, dtype=torch.int64, device=dev)
                count(r0, r1, part)
                step(r0, r1, part, int(offs[r1] - offs[r0]))
                r0 = r1
        st_col, nx_col = nx_col, st_col
        st_val, nx_val = nx_val, st_val
        st_cnt, nx_cnt = nx_cnt, st_cnt
    _check_status(status)
    return st_col, st_val, st_cnt


def personal_pagerank_appnp(edge_index, alpha, topk=100, num_iterations: int = 10,
                            batch_size: int = 8, device="cuda", csr_data=None,
                            num_nodes: int | None = None, iter_topk: int | None = None,
                            source_start: int | None = None, source_end: int | None = None,
                            method: str = "direct", streams: int = 8):
    """The reference's APPNP backend (appnp_backend.py:227-310) on the GPU.
    Returns (edge_index [2, nnz] int64 = (seed, node), values fp32).
    ``method``: the step's form, "direct" or "sort" (see appnp_batch);
    ``streams``: batches in flight at once with the direct step (each on a
    stream of its own; the result does not depend on it)."""
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("the APPNP backend runs on the GPU")
    batch_size = max(1, int(batch_size))
    num_iterations = max(1, int(num_iterations))
    rowptr, col, inv_deg, n = transition_csr(edge_index, csr_data, num_nodes, dev)
    empty = (torch.empty((2, 0), dtype=torch.long, device=dev),
             torch.empty(0, dtype=torch.float32, device=dev))
    if n == 0:
        return empty
    start = 0 if source_start is None else max(0, min(int(source_start), n))
    end = n if source_end is None else max(start, min(int(source_end), n))
    if start >= end:
        return empty
    topk = min(int(topk), n)
    iter_topk = topk if iter_topk is None else int(iter_topk)
    if iter_topk <= 0:
        raise NotImplementedError("iter_topk <= 0 (no per-step pruning) is not supported: give a "
                                  f"positive per-step top-k (1..{MAX_K})")
    K = min(iter_topk, n)
    final_keep = min(topk, K)
    if not 1 <= K <= MAX_K:
        raise ValueError(f"per-step top-k must be in 1..{MAX_K}, got {K}")
    if method not in ("direct", "sort"):
        raise ValueError(f"method must be 'direct' or 'sort', got {method!r}")
    batches = [torch.arange(s0, min(s0 + batch_size, end), dtype=torch.long, device=dev)
               for s0 in range(start, end, batch_size)]
    if method == "direct":
        outs = _run_direct(rowptr, col, inv_deg, n, batches, alpha, K, num_iterations,
                           max_repeats(rowptr, col), streams)
    else:
        outs = [appnp_batch(rowptr, col, inv_deg, n, seeds, alpha, K, num_iterations,
                            method=method) for seeds in batches]
    # every row's first min(cnt, topk) entries, seeds in order
    cols = torch.cat([o[0] for o in outs])
    vals = torch.cat([o[1] for o in outs])
    cnt = torch.cat([o[2] for o in outs]).clamp(max=final_keep).long()
    mask = torch.arange(K, device=dev)[None, :] < cnt[:, None]
    seeds = torch.arange(start, end, dtype=torch.long, device=dev)
    return torch.stack([seeds.repeat_interleave(cnt), cols[mask].long()]), vals[mask]
