"""Hypothesis strategies: random windows of the benchmark's kind (Chung-Lu
power-law graphs over the window's nodes, both directions, optional
self-loops) with related key rows after the window's own, duplicate edges and
the edge list in random order -- of varying size and density."""
from __future__ import annotations

import dataclasses

import numpy as np
from hypothesis import strategies as st

from neutrongt_amd import synthetic as S


@dataclasses.dataclass(frozen=True)
class Window:
    edge_index: np.ndarray  # [2, E] int64: row 0 = key (src), row 1 = query (dst)
    n_q: int
    n_k: int
    desc: str


def make_window(n_q: int, mean_degree: float, gamma: float, self_loops: bool, n_related: int,
                related_per_query: int, dup_frac: float, seed: int) -> Window:
    rng = np.random.default_rng(seed)
    if n_q > 1 and mean_degree > 0:
        u, v = S.chung_lu_edges(n_q, mean_degree, gamma, seed)
    else:
        u = v = np.zeros(0, np.int64)
    src = [u, v]
    dst = [v, u]
    if self_loops:
        src.append(np.arange(n_q))
        dst.append(np.arange(n_q))
    n_k = n_q + n_related
    if n_related and related_per_query:
        src.append(n_q + rng.integers(0, n_related, n_q * related_per_query))
        dst.append(np.repeat(np.arange(n_q), related_per_query))
    src = np.concatenate(src).astype(np.int64)
    dst = np.concatenate(dst).astype(np.int64)
    n_dup = int(dup_frac * src.shape[0])
    if n_dup:
        pick = rng.integers(0, src.shape[0], n_dup)
        src = np.concatenate([src, src[pick]])
        dst = np.concatenate([dst, dst[pick]])
    order = rng.permutation(src.shape[0])
    ei = np.stack([src[order], dst[order]]).astype(np.int64)
    desc = (f"n_q={n_q} n_k={n_k} E={ei.shape[1]} mean_deg={mean_degree:.2f} gamma={gamma:.2f} "
            f"self_loops={self_loops} related={related_per_query}/{n_related} dup={dup_frac:.2f} "
            f"seed={seed}")
    return Window(ei, n_q, n_k, desc)


def windows(max_n: int = 40, max_degree: float = 12.0, max_related: int = 16):
    return st.builds(
        make_window,
        n_q=st.integers(1, max_n),
        mean_degree=st.floats(0.0, max_degree, allow_nan=False),
        gamma=st.floats(2.0, 3.0, allow_nan=False),
        self_loops=st.booleans(),
        n_related=st.integers(0, max_related),
        related_per_query=st.integers(0, 3),
        dup_frac=st.sampled_from([0.0, 0.0, 0.05, 0.3]),
        seed=st.integers(0, 2**31 - 1),
    )
