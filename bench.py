#!/usr/bin/env python3
"""Window sparse-attention benchmark on one MI355X.

A step is one pass of the attention path over one synthetic window: for the
default workload (GPH_Large: 32,768-query window + 4 related keys per query,
H=32, d=24, bf16, 12 layers) the forward of all 12 attention layers followed by
their backward, each layer with its own q/k/v, through the drop-in autograd
path (window_attention: C++ autograd node -> libngt_attn.so).  Inputs and the window CSR
are resident in HBM before timing starts (the CSR is built once per window and
reused by every layer and step, as in the training loop).

Prints ONE JSON line: value = masked edges/s (layers x E / step time), the
roofline of the dominant kernel (its share of the layer's compulsory bytes /
its mean launch time, from hipEvents recorded around each launch on its own
stream; its measured L2-to-fabric traffic per launch from
profiles/traffic.json, rocprofv3 FETCH_SIZE and WRITE_SIZE scaled by a device
copy), the whole path's compulsory bytes per second (path_roofline) and the
CPU baseline: the reference's op sequence (the CPU oracle, fp32 torch) timed
on a bounded sample of the same window, on all host threads and on one.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "masked attn edges/sec fwd+bwd per GPU (GPH_Slim, GPH_Large); % HBM peak"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_BF16_TFLOPS = 2500.0
FP32_TFLOPS = 157.3  # published fp32 peak (vector and matrix alike)


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def _elem_bytes(dtype) -> int:
    import torch

    return 4 if dtype == torch.float32 else 2


def sparse_kernel_bytes(name: str, cfg, n_k: int, E: int, adj) -> float:
    """Compulsory HBM bytes of one launch of a sparse kernel: its share of the
    layer's compulsory bytes (every input, output and index array of the path
    that the kernel must touch, counted once).  Intermediates the library
    writes for its own later passes (the per-edge dS, split-row partials,
    work lists) are not counted: a different kernel split would not need them.
    The shares of the forward, rowstat, key-major and query-major passes add
    up to path_bytes."""
    b = _elem_bytes(cfg.dtype)
    H = cfg.n_heads
    D = H * cfg.head_dim
    n_q = cfg.n_q
    if name == "sparse_fwd":  # Q, K, V, O, rowptr, col, rinv, node_score
        return b * D * (2 * n_q + 2 * n_k) + 4 * (n_q + 1) + 4 * E + 4 * n_q * H + 4 * adj.dst_end
    if name == "sparse_rowstat":  # O (dO is counted in the key-major pass)
        return b * D * n_q
    if name == "sparse_bwd_kv":  # Q, dO, K, V, dK, dV, {r, D}, t_rowptr, t_col
        return b * D * (2 * n_q + 4 * n_k) + 8 * n_q * H + 4 * (n_k + 1) + 4 * E
    if name == "sparse_bwd_q":  # dQ, rowptr, col, q2t (K is counted in the key-major pass)
        return b * D * n_q + 4 * (n_q + 1) + 8 * E
    return float("nan")


def dense_kernel_flops(name: str, n_q: int, n_k: int, H: int, d: int) -> float:
    """Matrix-product flops one launch of a dense kernel has to do (2 per
    multiply-add; each N_q x N_k x d product is 2 N_q N_k d per head):
    fwd S = Q K^T, O = P V; scores recomputes S; bwd_kv S, dP^T = V G^T,
    dV = P^T G, dK = dS^T Q; bwd_q S, dP, dQ = dS K."""
    one = 2.0 * n_q * n_k * d * H
    return one * {"dense_fwd": 2, "dense_scores": 1, "dense_bwd_kv": 4,
                  "dense_bwd_q": 3}.get(name, float("nan"))


def path_bytes(cfg, n_k: int, E: int) -> float:
    """Compulsory bytes of one layer's forward + backward (each tensor once):
    fwd Q,O,K,V + CSR + Zinv + node_score; bwd Q,O,dO,K,V + {Zinv,D} + both CSRs
    + perm + dQ,dK,dV."""
    b = _elem_bytes(cfg.dtype)
    H = cfg.n_heads
    D = H * cfg.head_dim
    n_q = cfg.n_q
    fwd = b * D * (2 * n_q + 2 * n_k) + 4 * (n_q + 1) + 4 * E + 4 * n_q * H + 4 * n_q
    bwd = (b * D * (3 * n_q + 2 * n_k) + 8 * n_q * H + 4 * (n_q + 1) + 4 * E + 4 * (n_k + 1)
           + 8 * E + b * D * (n_q + 2 * n_k))
    return float(fwd + bwd)


def measured_traffic(config: str, kernel: str):
    """Bytes per launch of `kernel` between its L2 and the fabric (MALL or
    HBM), measured with rocprofv3 FETCH_SIZE and WRITE_SIZE (profiles/traffic.json,
    scaled by what the same counters read for a plain device copy), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(f"{config}:{kernel}")
    except (OSError, ValueError):
        return None
    if not rec:
        return None
    return float(rec["read_bytes"]) + float(rec["write_bytes"])


def _cpu_model() -> tuple[str, int | None]:
    """(model name, sockets) of the host CPU from lscpu (or /proc/cpuinfo)."""
    import subprocess

    model, sockets = "", None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() == "Model name" and not model:
                model = val.strip()
            elif key.strip() == "Socket(s)":
                try:
                    sockets = int(val.strip())
                except ValueError:
                    pass
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    return model, sockets


def cpu_baseline(cfg, ei_np, n_k, target_s: float = 2.0, reps: int = 5):
    """The reference's op sequence (CPU oracle, fp32) on the in-edges of a
    seeded random subset of the window's query rows, sized so one fwd+bwd
    takes ~target_s: on every host thread this process may use, then on one
    thread (its own, smaller sample).  1 warm-up + median of ``reps`` each.
    Returns the cpu_baseline JSON object (value = the all-threads figure)."""
    import numpy as np
    import torch

    from neutrongt_amd import synthetic as S
    from oracle import attention as OA

    threads = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        threads = min(threads, int(env))
    H = cfg.n_heads
    q, k, v, go = S.make_qkv(cfg, n_k, layer=0, device="cpu")
    # query rows in a seeded random order, so any prefix has the window's
    # degree distribution
    rank = np.empty(cfg.n_q, np.int64)
    rank[np.random.default_rng(S.SEED).permutation(cfg.n_q)] = np.arange(cfg.n_q)
    dst_rank = rank[ei_np[1]]

    def sample(n_rows):
        sub = ei_np[:, dst_rank < n_rows]
        keys, kinv = np.unique(sub[0], return_inverse=True)
        rows = np.argsort(rank)[:n_rows]
        sub_ei = torch.from_numpy(np.stack([kinv, rank[sub[1]]]))
        rows_t = torch.from_numpy(rows)
        return (q[rows_t].float(), k[torch.from_numpy(keys)].float(),
                v[torch.from_numpy(keys)].float(), go[rows_t].float(), sub_ei)

    def run(args):
        t = time.perf_counter()
        OA.sparse_fwd_bwd(args[0], args[1], args[2], args[4], args[3], H, dtype=torch.float32)
        return time.perf_counter() - t

    def measure(n_threads):
        torch.set_num_threads(max(1, n_threads))
        n_rows = min(cfg.n_q, 64)
        args = sample(n_rows)
        run(args)  # first call pays torch's one-time set-up
        t = run(args)
        while t < target_s / 3 and n_rows < cfg.n_q:
            n_rows = min(cfg.n_q, int(n_rows * min(8.0, max(1.5, target_s / max(t, 1e-3)))))
            args = sample(n_rows)
            t = run(args)  # doubles as the warm-up of the final size
        t_med = statistics.median(run(args) for _ in range(reps))
        return int(args[4].shape[1]) / t_med, n_rows, int(args[4].shape[1]), t_med

    prev = torch.get_num_threads()
    try:
        v_all, rows_all, e_all, t_all = measure(threads)
        used = torch.get_num_threads()
        v_one, rows_one, e_one, t_one = measure(1)
    finally:
        torch.set_num_threads(prev)
    model, sockets = _cpu_model()
    kind = "bf16-rounded" if cfg.dtype != torch.float32 else "fp32"
    return {
        "value": v_all,
        "unit": "edges/s",
        "cores": used,
        "kind": "port",
        "sample": (f"one layer fwd+bwd of the reference op sequence (torch CPU oracle in fp32 on "
                   f"{kind} inputs, all {H} heads) on the in-edges of a seeded random choice of "
                   f"query rows: {rows_all} of {cfg.n_q} rows ({e_all} edges) on {used} threads, "
                   f"{t_all:.2f} s per run; median of {reps} after 1 warm-up"),
        "single_thread": {"value": v_one, "unit": "edges/s", "cores": 1,
                          "sample": f"{rows_one} rows ({e_one} edges), {t_one:.2f} s per run, "
                                    f"median of {reps} after 1 warm-up"},
        "cpu_model": model,
        "sockets": sockets,
        "affinity_threads": len(os.sched_getaffinity(0)),
    }


def ppr_bench(args, cfg, dev) -> dict:
    """Personalised-PageRank preprocessing (appnp_backend.py:227-310) with the
    shipped settings (run_NeutronGT.sh: --ppr_topk 5 --ppr_iter_topk 5
    --ppr_alpha 0.85 --ppr_num_iterations 10 --ppr_batch_size 8192) over a
    Chung-Lu graph with cfg's global node count and mean degree.  The oracle's
    restatement is timed on a seeded sample of seeds on one host core."""
    import numpy as np
    import torch

    from neutrongt_amd import ppr as PPR
    from neutrongt_amd import synthetic as S

    n = cfg.n_global
    cap = args.ppr_degree_cap
    t0 = time.perf_counter()
    u, v = S.chung_lu_edges(n, cfg.mean_degree, cfg.gamma, S.SEED, degree_cap=cap)
    if args.ppr_relabel:
        # the same graph under a seeded random node numbering: the generator
        # numbers nodes by decreasing weight, so the top-k's ties (lowest id
        # first) would otherwise always land on the largest hubs
        perm = np.random.default_rng(S.SEED + 1).permutation(n).astype(np.int64)
        u, v = perm[u], perm[v]
    ei = torch.from_numpy(np.stack([np.concatenate([u, v]), np.concatenate([v, u])]))
    _log(f"[bench] ppr: graph drawn in {time.perf_counter() - t0:.1f} s")
    alpha, topk, iters, batch = 0.85, 5, 10, 8192
    rowptr, col, inv_deg, _ = PPR.transition_csr(ei, num_nodes=n, device=dev)
    deg_max = int((rowptr[1:] - rowptr[:-1]).max().item()) if n else 0
    csr = {"rowptr": rowptr, "col": col}
    _log(f"[bench] ppr: graph n={n}, {int(col.numel())} directed edges; topk {topk}, "
         f"{iters} iterations, batches of {batch}")
    # as many batches as run at once as warm-up (so the streams exist), then
    # the whole graph timed
    method = args.ppr_method
    streams = max(1, args.ppr_streams) if method == "direct" else 1  # the sort form: one at a time
    PPR.personal_pagerank_appnp(None, alpha, topk=topk, num_iterations=iters, batch_size=batch,
                                device=dev, csr_data=csr, iter_topk=topk,
                                source_end=streams * batch, method=method, streams=streams)
    torch.cuda.synchronize()
    # all seeds, in chunks of 32 batches with a progress line after each (the
    # rows are independent, so chunking changes nothing but the logging)
    chunk = 32 * batch
    idx_parts, val_parts = [], []
    t = time.perf_counter()
    for s0 in range(0, n, chunk):
        i_c, v_c = PPR.personal_pagerank_appnp(None, alpha, topk=topk, num_iterations=iters,
                                               batch_size=batch, device=dev, csr_data=csr,
                                               iter_topk=topk, source_start=s0,
                                               source_end=min(s0 + chunk, n), method=method,
                                               streams=streams)
        idx_parts.append(i_c)
        val_parts.append(v_c)
        torch.cuda.synchronize()
        _log(f"[bench] ppr: seeds {min(s0 + chunk, n)}/{n} after {time.perf_counter() - t:.1f} s")
    t_gpu = time.perf_counter() - t
    idx, val = torch.cat(idx_parts, dim=1), torch.cat(val_parts)
    _log(f"[bench] ppr: {t_gpu * 1e3:.1f} ms for {n} seeds ({int(idx.shape[1])} entries)")
    cpu = None
    if not args.no_cpu:
        from oracle import ppr as OP

        rp, cl, iv = rowptr.cpu().numpy(), col.cpu().numpy(), inv_deg.cpu().numpy()
        sample = np.random.default_rng(S.SEED).choice(n, 200, replace=False)
        t = time.perf_counter()
        rows = [OP.appnp_row(rp, cl, iv, sd, alpha, topk, iters) for sd in sample.tolist()]
        t_s = time.perf_counter() - t
        # the same seeds' rows of the GPU result, checked against the oracle's
        # (entries in rank order; nodes and fp32 values bit for bit)
        src, dst, vv = idx[0].cpu().numpy(), idx[1].cpu().numpy(), val.cpu().numpy()
        starts = np.searchsorted(src, sample, side="left")
        ends = np.searchsorted(src, sample, side="right")
        exact = sum(
            [int(c) for c, _ in row] == dst[a:b].tolist()
            and np.array([w for _, w in row], np.float32).tobytes() == vv[a:b].tobytes()
            for row, a, b in zip(rows, starts, ends))
        cpu = {"value": t_s / sample.size * n * 1e3, "unit": "ms", "cores": 1, "kind": "port",
               "sample": (f"the oracle's restatement on 200 seeded random seeds ({t_s:.1f} s), "
                          f"scaled to all {n} seeds"),
               "rows_bit_exact": f"{exact}/{sample.size}"}
        _log(f"[bench] ppr cpu baseline {cpu['value'] / 1e3:.1f} s (extrapolated); "
             f"{exact}/{sample.size} sampled rows bit-exact against the oracle")
    return {
        "metric": "personalised PageRank preprocessing time (APPNP, top-5, 10 iterations)",
        "value": t_gpu * 1e3, "unit": "ms", "n_gpus": 1, "steps": 1, "warmup": 1,
        "ms_per_step": t_gpu * 1e3, "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": (f"{cfg.name} global graph: Chung-Lu n={n}, "
                                f"{int(col.numel())} directed edges"
                                + (f" (expected degrees capped at {cap:g})" if cap else "")
                                + (", nodes randomly relabelled" if args.ppr_relabel else "")
                                + f", alpha {alpha}, top-{topk}, {iters} iterations, "
                                f"batches of {batch} seeds"),
                   "entries": int(idx.shape[1]), "degree_cap": cap,
                   "relabelled": bool(args.ppr_relabel), "step": method, "streams": streams,
                   "max_degree": int(deg_max)},
        "cpu_baseline": cpu,
    }


def prep_bench(args, cfg, dev) -> dict:
    """Assembly of one window on the GPU, from the global graph to the
    attention inputs: related-node selection (metisPartition.py:397-425), the
    induced subgraph in both reference orders (window_state.py:92-127), the
    window CSR and schedules, and the feature gather (train_eval.py:234-242).
    The global graph is a Chung-Lu graph with cfg's node count and mean degree,
    drawn on the GPU (duplicate pairs kept); the partition is a seeded random
    set of cfg.n_q nodes, sorted.  The oracle's CPU restatement of the same
    steps (the reference's host path) is timed once on the host beside it."""
    import numpy as np
    import torch

    from neutrongt_amd import chunk_for_heads, pack_q_adaptive, small_for_heads
    from neutrongt_amd import synthetic as S
    from neutrongt_amd import window as W
    from neutrongt_amd.csr import WindowAdjacency

    n = cfg.n_global
    g = torch.Generator(device=dev).manual_seed(S.SEED)
    w = (torch.arange(n, device=dev, dtype=torch.float64) + 1.0) ** (-1.0 / (cfg.gamma - 1.0))
    cdf = torch.cumsum(w / w.sum(), 0)
    cdf[-1] = 1.0
    m = int(n * cfg.mean_degree / 2)
    a = torch.searchsorted(cdf, torch.rand(m, generator=g, device=dev, dtype=torch.float64),
                           right=True)
    b = torch.searchsorted(cdf, torch.rand(m, generator=g, device=dev, dtype=torch.float64),
                           right=True)
    keep = a != b
    rows = torch.cat([a[keep], b[keep]])
    cols = torch.cat([b[keep], a[keep]])
    del a, b, keep, w, cdf
    order = torch.argsort(rows, stable=True)
    rows, col = rows[order], cols[order]
    del cols, order
    rowptr = torch.searchsorted(rows, torch.arange(n + 1, device=dev, dtype=torch.int64))
    coo = torch.stack([rows, col])
    del rows
    xadj = rowptr.to(torch.int32)
    adjncy = col.to(torch.int32)
    eweights = torch.randint(1, 4, (col.numel(),), generator=g, device=dev, dtype=torch.int32)
    part = torch.sort(torch.randperm(n, generator=g, device=dev)[: cfg.n_q]).values
    feat_dim = cfg.feat_dim or 128
    features = torch.randn(n, feat_dim, generator=g, device=dev)
    pct = max(cfg.related_per_query, 1)
    H = cfg.n_heads
    E_glob = int(col.numel())
    _log(f"[bench] prep: global graph n={n} directed entries={E_glob}, window {cfg.n_q} nodes, "
         f"related {pct}%")

    def timed(fn, reps=5):
        out = fn()
        ts = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t = time.perf_counter()
            out = fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t)
        return out, 1e3 * statistics.median(ts)

    win, t_rel = timed(lambda: W.merge_related_nodes(xadj, adjncy, eweights, part, pct))
    sub_csr, t_csr = timed(lambda: W.subgraph_from_csr(win, rowptr, col))
    sub_coo, t_coo = timed(lambda: W.subgraph(win, coo, n))
    n_w = int(win.numel())
    # attention edge_index: row 0 = key (the CSR row node), row 1 = query
    adj, t_adj = timed(lambda: WindowAdjacency(sub_csr, n_w, n_w,
                                               chunk_for_heads(H, int(sub_csr.shape[1])),
                                               small_for_heads(H), pack_q_adaptive(H)))
    (x_i, _), t_gather = timed(lambda: W.gather_rows(features, win))
    # window refinement of this window: node_out with seeded node scores (30 %
    # removed, the training loop's ratio), then node_in refilling it from the
    # expired nodes by PPR mass (8 PPR entries per node of the global graph)
    from neutrongt_amd import refine as RF

    n_ppr = 8 * n
    ppr = torch.stack([torch.randint(0, n, (n_ppr,), generator=g, device=dev),
                       torch.randint(0, n, (n_ppr,), generator=g, device=dev)])
    ppr_val = torch.rand(n_ppr, generator=g, device=dev) * 1e-3
    scores = torch.rand(n_w, generator=g, device=dev)
    # the METIS weights built from that PPR list (build_adj_fromat)
    (_, _, ew_g), t_adjw = timed(lambda: W.adj_weights(ppr, ppr_val))
    (kept, kept_edges, expired), t_out = timed(
        lambda: RF.node_out_window(win, sub_csr, scores, 0.3))
    _, t_in = timed(lambda: RF.node_in_window(kept, expired, ppr, ppr_val, int(expired.numel()),
                                              coo, n))
    # a rank's eight windows (disjoint partitions, each widened by its related
    # nodes, so that they overlap) rebuilt as _rebuild_local_window_structures
    # does: duplicate layout, feature cache, induced subgraphs from the CSR
    perm = torch.randperm(n, generator=g, device=dev)
    n_win = 8 if 8 * cfg.n_q <= n else max(1, n // cfg.n_q)
    rank_wins = [W.merge_related_nodes(xadj, adjncy, eweights,
                                       torch.sort(perm[i * cfg.n_q:(i + 1) * cfg.n_q]).values, pct)
                 for i in range(n_win)]
    lw, t_rank = timed(lambda: W.rebuild_local_windows(rank_wins, features, rowptr=rowptr,
                                                       col=col), reps=3)
    n_dup = int(lw.feature_cache.shape[0])
    # the last run's two phases (each ends in a device sync): the duplicate
    # layout with its feature cache, and the windows' subgraphs
    t_dup = 1e3 * lw.timings["local_dup_cache_rebuild_time"]
    t_subs = 1e3 * lw.timings["local_subgraph_rebuild_time"]
    rank_h = [w.cpu().numpy() for w in rank_wins]
    rank_out = ([w.cpu().numpy() for w in lw.partitions], lw.feature_cache.cpu().numpy())
    del lw, rank_wins, perm
    ops = {"merge_related_nodes_ms": t_rel, "subgraph_from_csr_ms": t_csr,
           "subgraph_coo_ms": t_coo, "window_csr_build_ms": t_adj, "feature_gather_ms": t_gather,
           "node_out_ms": t_out, "node_in_ms": t_in, "adj_weights_ms": t_adjw,
           "rank_windows": n_win,
           "rank_rebuild_ms": t_rank, "rank_dup_cache_ms": t_dup, "rank_subgraphs_ms": t_subs,
           "rank_cached_nodes": n_dup}
    total = t_rel + t_csr + t_adj + t_gather
    _log("[bench] prep: " + ", ".join(f"{k} {v:.3f}" if isinstance(v, float) else f"{k} {v}"
                                      for k, v in ops.items())
         + f"; window {n_w} nodes, {int(sub_csr.shape[1])} edges")

    cpu = None
    if not args.no_cpu:
        from oracle import graph as OG

        xadj_h, adj_h, ew_h = xadj.cpu().numpy(), adjncy.cpu().numpy(), eweights.cpu().numpy()
        part_h, rowptr_h, col_h = part.cpu().numpy(), rowptr.cpu().numpy(), col.cpu().numpy()
        feat_h = features.cpu().numpy()
        t = time.perf_counter()
        win_h, _ = OG.merge_related_nodes(xadj_h, adj_h, ew_h, part_h, pct)
        sub_h = OG.subgraph_from_csr(win_h, rowptr_h, col_h)
        OG.csr_from_coo(sub_h[0], sub_h[1], len(win_h), len(win_h))
        feat_h[win_h]
        t_cpu = time.perf_counter() - t
        if not (np.array_equal(win_h, win.cpu().numpy())
                and np.array_equal(sub_h, sub_csr.cpu().numpy())):
            raise RuntimeError("window assembly differs from the oracle")
        from oracle import refine as OR

        t = time.perf_counter()
        k_h, _, x_h = OR.node_out_window(win_h, sub_h, scores.cpu().numpy(), 0.3)
        OR.node_in_window(k_h, x_h, ppr.cpu().numpy(), ppr_val.cpu().numpy(), x_h.size,
                          coo.cpu().numpy(), n)
        t_ref = time.perf_counter() - t
        # the rank's duplicate layout and feature cache (_compute_local_duplicate_nodes,
        # build_dup_cache_metadata and the cache gather: the reference's host path)
        t = time.perf_counter()
        rer_h, dups_h = OG.duplicate_rerange(rank_h)
        cache_h, _ = OG.dup_cache_metadata(dups_h)
        cache_feat_h = feat_h[cache_h]
        t_dup_cpu = time.perf_counter() - t
        if not (all(np.array_equal(a, b) for a, b in zip(rer_h, rank_out[0]))
                and np.array_equal(cache_feat_h, rank_out[1])):
            raise RuntimeError("rank duplicate layout differs from the oracle")
        # the METIS weights of the same PPR list (numpy unique + ordered adds)
        ppr_h, pv_h = ppr.cpu().numpy(), ppr_val.cpu().numpy()
        t = time.perf_counter()
        _, _, ew_h = OG.adj_weights(ppr_h, pv_h)
        t_adjw_cpu = time.perf_counter() - t
        if not np.array_equal(ew_h, ew_g.cpu().numpy()):
            raise RuntimeError("METIS weights differ from the oracle")
        cpu = {"value": 1e3 * t_cpu, "unit": "ms", "cores": 1, "kind": "port",
               "sample": "the same window once: the oracle's restatement of "
                         "_merge_related_nodes (Python dict loop), _subgraph_from_csr (per-node "
                         "searchsorted loop), the CSR build (numpy lexsort) and the feature gather",
               "refine_ms": 1e3 * t_ref, "rank_dup_cache_ms": 1e3 * t_dup_cpu,
               "adj_weights_ms": 1e3 * t_adjw_cpu}
        _log(f"[bench] prep cpu baseline {1e3 * t_cpu:.1f} ms; node_out+node_in "
             f"{1e3 * t_ref:.1f} ms; rank duplicate layout + cache {1e3 * t_dup_cpu:.1f} ms; "
             f"METIS weights {1e3 * t_adjw_cpu:.1f} ms")
    return {
        "metric": "window assembly time (related nodes, induced subgraph, window CSR, features)",
        "value": total, "unit": "ms", "n_gpus": 1, "steps": 5, "warmup": 1, "ms_per_step": total,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "int64",
        "data": "synthetic",
        "config": {"workload": (f"{cfg.name} window assembly: global Chung-Lu graph n={n}, "
                                f"{E_glob} directed entries; window of {cfg.n_q} nodes + "
                                f"{pct}% related -> {n_w} nodes, {int(sub_csr.shape[1])} edges; "
                                f"features {feat_dim} fp32"),
                   "window_nodes": n_w, "window_edges": int(sub_csr.shape[1])},
        "ops": ops,
        "cpu_baseline": cpu,
    }


def model_step_bench(args, cfg, layers: int, dev) -> dict:
    """The window training step of train_eval.py:255-300 on one GPU: the
    node-level Graphormer, or GT for the GT presets (cfg's hidden size, heads
    and layers; FFN width = hidden as in the presets) over one synthetic window, bf16 autocast,
    NLL over the window's training nodes, backward, AdamW.  Related keys' K/V
    come from a per-layer cache.  The loss is read back every step, as the
    reference's loop does (loss.item())."""
    import numpy as np
    import torch

    from neutrongt_amd import _lib
    from neutrongt_amd import synthetic as S
    from neutrongt_amd.encoder import WindowGraphormer, WindowGT, window_step

    H, d = cfg.n_heads, cfg.head_dim
    hidden = H * d
    n_classes = 47
    feat = cfg.feat_dim or hidden
    ei_np, n_k = S.make_window_edges(cfg)
    E = int(ei_np.shape[1])
    R = n_k - cfg.n_q
    g = torch.Generator(device="cpu").manual_seed(S.SEED)
    x = torch.randn(cfg.n_q, feat, generator=g).to(dev)
    labels = torch.randint(0, n_classes, (cfg.n_q,), generator=g).to(dev)
    train_mask = (torch.rand(cfg.n_q, generator=g) < 0.5).to(dev)
    cache = [tuple((0.05 * torch.randn(R, H, d, generator=g)).to(torch.bfloat16).to(dev)
                   for _ in range(2)) for _ in range(layers)] if R else None
    ei = torch.from_numpy(ei_np).to(dev)
    torch.manual_seed(S.SEED)
    # GT presets run the GT twin (post-LN, MLP readout); the others Graphormer
    family = WindowGT if cfg.name.startswith("gt") else WindowGraphormer
    model = family(layers, H, feat, hidden, n_classes, dropout_rate=0.3,
                   input_dropout_rate=0.1, attention_dropout_rate=0.5,
                   ffn_dim=hidden).to(dev).train()
    n_params = sum(p.numel() for p in model.parameters())
    # torch's single-kernel AdamW (the reference builds the foreach default,
    # main_sp_node_level_ppr.py:164; same update rule)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, weight_decay=0.01,
                            capturable=bool(args.graph), fused=True)
    _log(f"[bench] window step: {layers} layers, hidden {hidden}, {n_params} parameters, "
         f"n_q={cfg.n_q} n_k={n_k} E={E}")

    def step():
        loss, _ = window_step(model, opt, x, ei, labels, train_mask, cache, torch.bfloat16)
        return loss.item()

    if args.tunable:
        # GEMM kernel choice by measurement (hipBLASLt/rocBLAS candidates); a
        # results file that already holds these shapes is only read
        torch.cuda.tunable.enable(True)
        torch.cuda.tunable.set_filename(args.tunable)
        tuned = os.path.exists(args.tunable)
        if tuned:
            torch.cuda.tunable.read_file(args.tunable)
        torch.cuda.tunable.tuning_enable(not tuned)
    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()
    if args.tunable and not tuned:
        torch.cuda.tunable.tuning_enable(False)  # the results file is written at exit
    if args.graph:
        # the whole step (forward, loss, backward, AdamW) as one HIP graph;
        # warm-up on a side stream first, as graph capture requires
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                window_step(model, opt, x, ei, labels, train_mask, cache, torch.bfloat16)
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_loss, _ = window_step(model, opt, x, ei, labels, train_mask, cache,
                                         torch.bfloat16)

        def step():  # noqa: F811
            graph.replay()
            return static_loss.item()

        step()
        torch.cuda.synchronize()
    times, losses = [], []
    for _ in range(args.steps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        losses.append(step())
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t)
    ms = 1e3 * statistics.median(times)
    _lib.timing_enable(True)
    _lib.timing_summary()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    summ = _lib.timing_summary()
    _lib.timing_enable(False)
    attn_ms = sum(v[1] for n, v in summ.items() if n.startswith(("sparse_", "dense_"))) / args.steps
    copies = {}
    if not args.graph:
        # the reference's loop copies the window's edge_index to the device
        # every step (train_eval.py:244): timed with the cache matching the
        # copy by contents, and with the cache emptied first (a CSR rebuild
        # every step, what an identity-keyed cache would do)
        from neutrongt_amd.csr import default_cache

        ei_host = ei.cpu()

        def step_copy():
            loss, _ = window_step(model, opt, x, ei_host.to(dev), labels, train_mask, cache,
                                  torch.bfloat16)
            return loss.item()

        def step_rebuild():
            default_cache.clear()
            return step_copy()

        for name, fn in (("per_step_copy_ms", step_copy), ("per_step_rebuild_ms", step_rebuild)):
            fn()
            ts = []
            for _ in range(args.steps):
                torch.cuda.synchronize()
                t = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                ts.append(time.perf_counter() - t)
            copies[name] = 1e3 * statistics.median(ts)
        _log(f"[bench] window step with a fresh edge_index copy per step: "
             f"{copies['per_step_copy_ms']:.2f} ms (CSR found by contents), "
             f"{copies['per_step_rebuild_ms']:.2f} ms (CSR rebuilt)")
    _log(f"[bench] window step {ms:.2f} ms (median of {args.steps}), attention kernels "
         f"{attn_ms:.2f} ms/step, loss {losses[0]:.4f} -> {losses[-1]:.4f}")
    return {
        "metric": "window training step time (encoder fwd + NLL + bwd + AdamW)",
        "value": ms, "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": (f"{cfg.name} window step: {layers}-layer {family.__name__}, hidden "
                                f"{hidden}, {H} heads, ffn {hidden}, {n_params} parameters, "
                                f"n_q={cfg.n_q}, n_k={n_k}, E={E}, bf16 autocast, AdamW"),
                   "layers": layers, "parameters": n_params, "edges": E,
                   "hip_graph": bool(args.graph)},
        "attention_ms_per_step": attn_ms,
        **copies,
        "edges_per_s_in_step": layers * E / (ms * 1e-3),
        "losses": [losses[0], losses[-1]],
    }


def measure_window(args, cfg, layers: int, dev, graph: bool, calib_copy: bool) -> dict:
    """Time `layers` layers of the window attention fwd+bwd on `cfg` (W warm-up
    steps, then exactly K timed steps between events on the current stream),
    then the same steps again with the library's per-launch hipEvents; returns
    the step time, edges/s, per-kernel times and the dominant kernel's roofline."""
    import torch

    from neutrongt_amd import _lib, chunk_for_heads, pack_q_adaptive, small_for_heads
    from neutrongt_amd import synthetic as S
    from neutrongt_amd.attention import DenseAttentionFunction, window_attention
    from neutrongt_amd.csr import WindowAdjacency

    H, d = cfg.n_heads, cfg.head_dim
    scale = math.sqrt(d)

    t0 = time.perf_counter()
    if cfg.dense:
        ei_np, n_k, E = None, cfg.n_q, cfg.n_q * cfg.n_q
    else:
        ei_np, n_k = S.make_window_edges(cfg)
        E = int(ei_np.shape[1])
    _log(f"[bench] workload {cfg.name}: n_q={cfg.n_q} n_k={n_k} E={E} H={H} d={d} "
         f"layers={layers} ({time.perf_counter() - t0:.1f}s)")
    tensors = []
    for layer in range(layers):
        q, k, v, go = S.make_qkv(cfg, n_k, layer=layer, device=dev)
        tensors.append([t.requires_grad_(True) for t in (q, k, v)] + [go])
    adj = None
    csr_ms = None
    if not cfg.dense:
        ei = torch.from_numpy(ei_np).to(dev)
        # built three times: the first build also pays one-time library and
        # allocator set-up, and a later one can still meet an allocator
        # growth; the faster of the second and third is what a new window
        # costs in a running job
        cold = None
        for _ in range(3):
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            adj = WindowAdjacency(ei, cfg.n_q, n_k, chunk_for_heads(H, E), small_for_heads(H),
                                  pack_q_adaptive(H))
            t_build = (time.perf_counter() - t1) * 1e3
            if cold is None:
                cold = t_build
            else:
                csr_ms = t_build if csr_ms is None else min(csr_ms, t_build)
        _log(f"[bench] csr built in {csr_ms:.2f} ms (first build {cold:.1f} ms; incl. one info "
             f"sync); items q/k "
             f"{adj.struct.n_items_q}/{adj.struct.n_items_k}, packed q/k "
             f"{adj.struct.n_packed_q}/{adj.struct.n_packed_k}, splits q/k "
             f"{adj.struct.n_splits_q}/{adj.struct.n_splits_k}, max deg q/k "
             f"{adj.max_deg_q}/{adj.max_deg_k}")

    def step():
        outs, grads = [], []
        for q, k, v, go in tensors:
            q.grad = k.grad = v.grad = None
            if cfg.dense:
                x, _ = DenseAttentionFunction.apply(q, k, v, scale, True)
            else:
                x, _ = window_attention(q, k, v, adj, scale, -5.0, 5.0, 1e-6)
            outs.append(x)
            grads.append(go)
        torch.autograd.backward(outs, grads)

    if calib_copy:
        src = torch.empty(256 << 20, dtype=torch.int16, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # 512 MiB read + 512 MiB written
        torch.cuda.synchronize()
        del src, dst
    # W untimed steps, then more until the warm-up has run for --min-warmup-ms:
    # three steps of a 1.2 ms workload leave the GPU short of its steady clock
    # (the dense window read 1.24 / 1.18 / 1.14 ms per step after 3 / 10 / 30
    # warm-up steps on one box); the timed region stays exactly K steps.
    t_w = time.perf_counter()
    warm_steps = 0
    while warm_steps < args.warmup or (time.perf_counter() - t_w) * 1e3 < args.min_warmup_ms:
        step()
        warm_steps += 1
        if warm_steps >= args.warmup:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    warm_ms = (time.perf_counter() - t_w) * 1e3
    run = step
    if graph:
        # Same kernels, launched from one captured graph (no per-launch host work).
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
        for _ in range(2):
            run()
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    value = layers * E / (ms_step * 1e-3)
    _log(f"[bench] {args.steps} steps: {ms_step:.3f} ms/step, {value / 1e9:.3f} G edges/s")

    # Kernel-level timing (separate pass of the same steps; hipEvents around
    # every launch of the library, on the launch stream).
    _lib.timing_enable(True)
    _lib.timing_summary()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    summ = _lib.timing_summary()
    _lib.timing_enable(False)
    kernels = {n: {"launches": c, "avg_us": 1e3 * ms / c, "total_ms_per_step": ms / args.steps}
               for n, (c, ms) in summ.items()}
    dom = max(summ, key=lambda n: summ[n][1])
    dom_avg_s = summ[dom][1] / summ[dom][0] * 1e-3
    if cfg.dense:
        flops = dense_kernel_flops(dom, cfg.n_q, n_k, H, d)
        peak = FP32_TFLOPS if cfg.dtype == torch.float32 else MFMA_BF16_TFLOPS
        roof = {"bound": "mfma", "achieved": flops / dom_avg_s / 1e12, "peak": peak,
                "unit": "TFLOP/s", "frac": flops / dom_avg_s / 1e12 / peak,
                "traffic": measured_traffic(cfg.name, dom) if layers == cfg.layers else None,
                "kernel": dom, "flops_per_launch": flops,
                "avg_launch_us": dom_avg_s * 1e6}
        path = None
    else:
        kb = sparse_kernel_bytes(dom, cfg, n_k, E, adj)
        ach = kb / dom_avg_s / 1e9
        traffic = measured_traffic(cfg.name, dom) if layers == cfg.layers else None
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": ach / HBM_PEAK_GBS, "traffic": traffic, "kernel": dom,
                "bytes_per_launch": kb, "avg_launch_us": dom_avg_s * 1e6}
        pb = path_bytes(cfg, n_k, E)
        path = {"algorithmic_bytes_per_layer": pb,
                "achieved_GBs": pb * layers / (ms_step * 1e-3) / 1e9,
                "frac": pb * layers / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS}
    _log(f"[bench] kernels: " + ", ".join(f"{n} {v['avg_us']:.1f}us x{v['launches']}"
                                          for n, v in sorted(kernels.items())))
    return {"ms_step": ms_step, "value": value, "kernels": kernels, "roof": roof, "path": path,
            "n_k": n_k, "E": E, "csr_ms": csr_ms, "warm_steps": warm_steps,
            "warm_ms": warm_ms, "ei_np": ei_np}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--min-warmup-ms", type=float, default=300.0,
                    help="keep taking untimed warm-up steps past --warmup until this much time "
                         "has passed (0: exactly --warmup)")
    ap.add_argument("--config", default="gph_large",
                    help="gph_large (default), gph_slim, gt_arxiv, gt_highdeg, dense_slim, "
                         "dense_slim_f32")
    ap.add_argument("--layers", type=int, default=None, help="override the layer count")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--also", default=None,
                    help="a second window timed the same way and reported under 'also' "
                         "(default: gph_slim when the config is gph_large, the metric's other "
                         "workload; 'none' for no second window)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="run one 512 MiB device copy first (calibrates HBM byte counters)")
    ap.add_argument("--graph", action="store_true",
                    help="capture one step (all layers, fwd+bwd) in a HIP graph and time replays")
    ap.add_argument("--ppr", action="store_true",
                    help="time the personalised-PageRank preprocessing instead (APPNP, top-5, "
                         "10 iterations, batches of 8192 seeds) on the config's global graph")
    ap.add_argument("--ppr-degree-cap", type=float, default=None,
                    help="with --ppr: cap the global graph's expected node degrees (e.g. 17481, "
                         "ogbn-products' largest degree); default uncapped")
    ap.add_argument("--ppr-relabel", action="store_true",
                    help="with --ppr: number the global graph's nodes by a seeded random "
                         "permutation (the generator numbers them by decreasing degree)")
    ap.add_argument("--ppr-method", choices=("direct", "sort"), default="direct",
                    help="with --ppr: the propagation step's form (direct evaluation, or the "
                         "sorted product list); both give the same bits")
    ap.add_argument("--ppr-streams", type=int, default=8,
                    help="with --ppr: seed batches in flight at once, each on a stream of its "
                         "own (the result does not depend on it)")
    ap.add_argument("--prep", action="store_true",
                    help="time the window assembly instead (related nodes, induced subgraph, "
                         "window CSR, feature gather) on the config's global graph")
    ap.add_argument("--tunable", default=None, metavar="CSV",
                    help="with --model: let torch's TunableOp pick the GEMM kernels, reading "
                         "(and, if missing, writing) this results file")
    ap.add_argument("--model", action="store_true",
                    help="time the whole window training step instead (encoder projections, "
                         "LayerNorm, FFN and attention, NLL, backward, AdamW) in bf16 autocast")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build runs the attention path on a single "
              "MI355X (window sharding across GPUs is not part of it); use --gpus 1.",
              file=sys.stderr)
        return 2

    import torch

    from neutrongt_amd import synthetic as S

    cfg = S.CONFIGS[args.config]
    layers = args.layers or cfg.layers
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.ppr:
        if cfg.dense or not cfg.n_global:
            print("--ppr needs a sparse config with a global graph (gt_arxiv, gt_highdeg, "
                  "gph_large)", file=sys.stderr)
            return 2
        print(json.dumps(ppr_bench(args, cfg, dev)), flush=True)
        return 0
    if args.prep:
        if cfg.dense or not cfg.n_global:
            print("--prep needs a sparse config with a global graph (gph_large, gt_arxiv, "
                  "gt_highdeg)", file=sys.stderr)
            return 2
        print(json.dumps(prep_bench(args, cfg, dev)), flush=True)
        return 0
    if args.model:
        if cfg.dense:
            print("--model runs the sparse window encoder; pick a sparse --config", file=sys.stderr)
            return 2
        print(json.dumps(model_step_bench(args, cfg, layers, dev)), flush=True)
        return 0
    r = measure_window(args, cfg, layers, dev, args.graph, args.calib_copy)
    ms_step, value, kernels, roof, path = (r["ms_step"], r["value"], r["kernels"], r["roof"],
                                           r["path"])
    n_k, E, ei_np, H, d = r["n_k"], r["E"], r["ei_np"], cfg.n_heads, cfg.head_dim
    csr_ms, warm_steps, warm_ms = r["csr_ms"], r["warm_steps"], r["warm_ms"]

    also = None
    second = args.also if args.also is not None else ("gph_slim" if args.config == "gph_large"
                                                       and args.layers is None else "none")
    if second != "none":
        cfg2 = S.CONFIGS[second]
        _log(f"[bench] second window: {second}")
        r2 = measure_window(args, cfg2, cfg2.layers, dev, False, False)
        # the same steps replayed from one captured HIP graph: a one-layer step
        # of this size is bound by the host's per-layer autograd cost in eager
        # mode, and the replay shows the kernels' own rate
        r2g = measure_window(args, cfg2, cfg2.layers, dev, True, False)
        also = {second: {
            "value": r2["value"], "unit": "edges/s", "ms_per_step": r2["ms_step"],
            "dtype": "f32" if cfg2.dtype == torch.float32 else "bf16",
            "workload": (f"{cfg2.name}: {cfg2.layers}-layer "
                         f"{'dense' if cfg2.dense else 'sparse'} attention fwd+bwd, window "
                         f"n_q={cfg2.n_q}, n_k={r2['n_k']}, E={r2['E']}, H={cfg2.n_heads}, "
                         f"d={cfg2.head_dim}"),
            "hip_graph_value": r2g["value"], "hip_graph_ms_per_step": r2g["ms_step"],
            "roofline": r2["roof"], "path_roofline": r2["path"],
            "kernels_avg_us": {n: round(v["avg_us"], 2) for n, v in r2["kernels"].items()},
        }}

    cpu = None
    if not args.no_cpu and not cfg.dense:
        _log("[bench] timing the CPU baseline ...")
        cpu = cpu_baseline(cfg, ei_np, n_k)
        _log(f"[bench] cpu baseline {cpu['value'] / 1e6:.3f} M edges/s on {cpu['cores']} threads, "
             f"{cpu['single_thread']['value'] / 1e6:.3f} M edges/s on 1 ({cpu['cpu_model']}, "
             f"{cpu['sockets']} sockets)")

    dtype = "f32" if cfg.dtype == torch.float32 else "bf16"
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": {
            "workload": (f"{cfg.name}: {layers}-layer {'dense' if cfg.dense else 'sparse'} "
                         f"attention fwd+bwd, window n_q={cfg.n_q}, n_k={n_k}, E={E}, H={H}, "
                         f"d={d}, {dtype}"),
            "n_q": cfg.n_q, "n_k": n_k, "edges": E, "heads": H, "head_dim": d,
            "layers": layers, "csr_build_ms": csr_ms, "hip_graph": bool(args.graph),
            "warmup_steps_run": warm_steps, "warmup_ms": round(warm_ms, 1),
        },
        "roofline": roof,
        "path_roofline": path,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "also": also,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
