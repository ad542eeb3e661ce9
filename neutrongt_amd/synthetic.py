"""Seeded synthetic windows for parity tests and the benchmark.

A window is a Chung-Lu power-law graph over the window's query nodes (the
partition's induced subgraph), with self-loops, plus per-query "related" keys
drawn from outside the window with probability proportional to degree (the
PPR halo that NeutronGT merges into each window,
NeutronGT/core/metisPartition.py:397-425).  Related keys get key rows
N_q .. N_k-1 (their K/V come from the feature cache in the reference).

Values: features ~ N(0,1) projected by seeded Xavier-uniform Q/K/V weights
(bias 0), or Q/K/V ~ N(0,1) directly; upstream gradient ~ N(0,1).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np
import torch

SEED = 42  # the reference's default seed (NeutronGT/utils/parser_node_level.py:51)


@dataclasses.dataclass(frozen=True)
class WindowConfig:
    name: str
    n_q: int                 # query nodes in the window
    mean_degree: float       # target in-window mean degree (undirected, before self-loops)
    n_heads: int
    head_dim: int
    dtype: torch.dtype
    related_per_query: int = 0
    n_global: int = 0        # nodes of the whole graph (pool for related keys)
    feat_dim: int = 0        # 0: Q/K/V ~ N(0,1); else project N(0,1) features
    gamma: float = 2.1
    layers: int = 1
    dense: bool = False      # all-pairs full-window attention

    @property
    def hidden(self) -> int:
        return self.n_heads * self.head_dim


# The five workloads of the attention path (sizes from NeutronGT's GPH_Slim,
# GT and GPH_Large presets, NeutronGT/scripts/run_NeutronGT.sh:70-154).
CONFIGS = {
    "gph_slim": WindowConfig("gph_slim", 16384, 14.0, 8, 8, torch.float32, feat_dim=128),
    "gt_arxiv": WindowConfig("gt_arxiv", 10584, 13.8, 8, 16, torch.bfloat16, related_per_query=8,
                             n_global=169343, feat_dim=128),
    "dense_slim": WindowConfig("dense_slim", 16000, 0.0, 8, 8, torch.bfloat16, dense=True),
    # the same all-pairs window in fp32, the dtype the reference's ablation trains in
    "dense_slim_f32": WindowConfig("dense_slim_f32", 16000, 0.0, 8, 8, torch.float32,
                                   dense=True),
    "gph_large": WindowConfig("gph_large", 32768, 50.5, 32, 24, torch.bfloat16,
                              related_per_query=4, n_global=2449029, feat_dim=100, layers=12),
    "gt_highdeg": WindowConfig("gt_highdeg", 7280, 490.0, 8, 16, torch.bfloat16,
                               related_per_query=10, n_global=232965, feat_dim=602),
}


def chung_lu_edges(n: int, mean_degree: float, gamma: float = 2.1, seed: int = SEED,
                   tol: float = 0.02, max_iter: int = 12, degree_cap: float | None = None):
    """Undirected Chung-Lu graph: weights (i+1)^(-1/(gamma-1)); m endpoint pairs
    drawn i.i.d. proportional to weight, self pairs dropped, deduplicated; m is
    recalibrated until the realised mean degree is within ``tol`` of the target
    (or max_iter).  ``degree_cap`` flattens the largest weights so that no node
    expects more than about that many neighbours (None: uncapped, the default).
    Returns (u, v) int64 arrays with u < v, sorted."""
    if n <= 1 or mean_degree <= 0:
        z = np.zeros(0, np.int64)
        return z, z
    rng = np.random.default_rng(seed)
    w = (np.arange(n, dtype=np.float64) + 1.0) ** (-1.0 / (gamma - 1.0))
    # at most half of the n(n-1)/2 possible pairs: beyond that the dedup
    # saturates and the recalibration below would grow m without bound
    target = min(n * mean_degree / 2.0, n * (n - 1) / 4.0)
    if degree_cap is not None and 2.0 * target * w[0] / w.sum() > degree_cap:
        # node i expects about 2 m w_i / sum(w) endpoints: find the weight
        # ceiling c that gives the heaviest node degree_cap (monotone in c)
        lo, hi = 0.0, float(w[0])
        for _ in range(100):
            c = 0.5 * (lo + hi)
            if 2.0 * target * c / np.minimum(w, c).sum() > degree_cap:
                hi = c
            else:
                lo = c
        w = np.minimum(w, lo)
    cdf = np.cumsum(w / w.sum())
    cdf[-1] = 1.0
    m = max(int(target), 1)
    m_cap = 64 * m + 1024
    best = None
    for _ in range(max_iter):
        a = np.searchsorted(cdf, rng.random(m), side="right")
        b = np.searchsorted(cdf, rng.random(m), side="right")
        keep = a != b
        u = np.minimum(a[keep], b[keep])
        v = np.maximum(a[keep], b[keep])
        key = np.unique(u * n + v)
        got = key.shape[0]
        if best is None or abs(got - target) < abs(best.shape[0] - target):
            best = key
        if abs(got - target) <= tol * target:
            break
        m = int(m * target / max(got, 1) * 1.02) if got < target else int(m * target / got)
        m = min(max(m, 1), m_cap)
    return best // n, best % n


def related_keys(n_q: int, k: int, n_pool: int, gamma: float = 2.1, seed: int = SEED):
    """Per query, k distinct out-of-window node ids drawn proportional to
    Chung-Lu weight over a pool of n_pool nodes.  Returns (R sorted unique
    pool ids, per-query [n_q, k] pool ids)."""
    if k <= 0 or n_pool <= 0:
        return np.zeros(0, np.int64), np.zeros((n_q, 0), np.int64)
    k = min(k, n_pool)
    rng = np.random.default_rng(seed + 1)
    w = (np.arange(n_pool, dtype=np.float64) + 1.0) ** (-1.0 / (gamma - 1.0))
    cdf = np.cumsum(w / w.sum())
    cdf[-1] = 1.0
    out = np.empty((n_q, k), np.int64)
    cand = np.searchsorted(cdf, rng.random((n_q, 4 * k)), side="right")
    for i in range(n_q):
        row = cand[i]
        _, first = np.unique(row, return_index=True)
        picked = row[np.sort(first)][:k]
        while picked.shape[0] < k:
            extra = np.searchsorted(cdf, rng.random(4 * k), side="right")
            row = np.concatenate([picked, extra])
            _, first = np.unique(row, return_index=True)
            picked = row[np.sort(first)][:k]
        out[i] = picked
    return np.unique(out), out


def make_window_edges(cfg: WindowConfig, seed: int = SEED):
    """COO edge_index [2, E] (row 0 = key/src, row 1 = query/dst) and N_k.

    In-window edges are listed source-major (the order a CSR-derived global
    edge list gives the induced subgraph), both directions plus self-loops,
    followed by the related-key edges (key row N_q + rank in R -> query)."""
    n = cfg.n_q
    u, v = chung_lu_edges(n, cfg.mean_degree, cfg.gamma, seed)
    src = np.concatenate([u, v, np.arange(n)])
    dst = np.concatenate([v, u, np.arange(n)])
    order = np.lexsort((dst, src))
    src, dst = src[order], dst[order]
    n_k = n
    if cfg.related_per_query > 0:
        pool = max(cfg.n_global - n, cfg.related_per_query)
        R, per_q = related_keys(n, cfg.related_per_query, pool, cfg.gamma, seed)
        rows = n + np.searchsorted(R, per_q)  # [n_q, k]
        src = np.concatenate([src, rows.reshape(-1)])
        dst = np.concatenate([dst, np.repeat(np.arange(n), per_q.shape[1])])
        n_k = n + R.shape[0]
    return np.stack([src, dst]).astype(np.int64), n_k


def make_qkv(cfg: WindowConfig, n_k: int, seed: int = SEED, layer: int = 0, device="cpu"):
    """q [N_q,H,d], k/v [N_k,H,d] in cfg.dtype, plus grad_out [N_q,H,d].

    Random draws are made on the CPU (seeded); the feature projection runs on
    ``device`` (fp32), so the values depend on that device's matmul rounding."""
    g = torch.Generator(device="cpu").manual_seed(seed * 1000 + layer)
    H, d = cfg.n_heads, cfg.head_dim
    D = H * d
    if cfg.feat_dim > 0:
        x = torch.randn(n_k, cfg.feat_dim, generator=g).to(device)
        bound = math.sqrt(6.0 / (cfg.feat_dim + D))
        ws = [((torch.rand(cfg.feat_dim, D, generator=g) * 2 - 1) * bound).to(device)
              for _ in range(3)]
        q = (x[: cfg.n_q] @ ws[0]).view(cfg.n_q, H, d)
        k = (x @ ws[1]).view(n_k, H, d)
        v = (x @ ws[2]).view(n_k, H, d)
    else:
        q = torch.randn(cfg.n_q, H, d, generator=g)
        k = torch.randn(n_k, H, d, generator=g)
        v = torch.randn(n_k, H, d, generator=g)
    go = torch.randn(cfg.n_q, H, d, generator=g)
    cast = lambda t: t.to(cfg.dtype).contiguous().to(device)
    return cast(q), cast(k), cast(v), cast(go)


def small_config(name: str = "small", n_q: int = 300, mean_degree: float = 6.0, n_heads: int = 4,
                 head_dim: int = 8, dtype=torch.float32, related: int = 0, n_global: int = 0,
                 feat_dim: int = 0) -> WindowConfig:
    return WindowConfig(name, n_q, mean_degree, n_heads, head_dim, dtype, related_per_query=related,
                        n_global=n_global, feat_dim=feat_dim)
