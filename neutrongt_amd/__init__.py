"""neutrongt_amd -- MI355X (gfx950) window attention for NeutronGT.

Public API
----------
CoreAttention            drop-in for NeutronGT's CoreAttention (sparse + full)
install(model)           swap a model's local_attn modules for CoreAttention
sparse_attention(...)    functional masked attention over a window edge_index
window_attention(...)    the same over a built WindowAdjacency (C++ autograd node)
dense_attention(...)     functional full-window attention
WindowAdjacency          device CSR/transposed CSR/work lists of one window
"""
from .attention import (CoreAttention, DenseAttentionBiasFunction, DenseAttentionFunction,
                        SparseAttentionBiasFunction, SparseAttentionFunction, dense_attention,
                        dense_attention_bias, install, sparse_attention, window_attention)
from .csr import (AdjacencyCache, WindowAdjacency, chunk_for_heads, default_cache, pack_q_adaptive,
                  small_for_heads)

__all__ = [
    "CoreAttention",
    "install",
    "sparse_attention",
    "window_attention",
    "dense_attention",
    "SparseAttentionFunction",
    "SparseAttentionBiasFunction",
    "DenseAttentionFunction",
    "DenseAttentionBiasFunction",
    "dense_attention_bias",
    "WindowAdjacency",
    "AdjacencyCache",
    "chunk_for_heads",
    "pack_q_adaptive",
    "small_for_heads",
    "default_cache",
]
