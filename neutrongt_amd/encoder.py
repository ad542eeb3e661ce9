"""The window encoder around the HIP attention core: the caller side of the path.

Mirrors NeutronGT's node-level Graphormer with its sparse attention
(NeutronGT/models/graphormer_dist_node_level.py): ``FeedForwardNetwork``
(:18-30), ``MultiHeadAttention`` (:128-173), ``EncoderLayer`` (:176-206) and
``Graphormer.forward`` without the structural encodings (:242-381; the shipped
scripts run with ``struct_enc`` False).  Sub-module and parameter names are the
reference's, so a reference ``state_dict`` loads with ``strict=False`` (the
unused centrality/attention-bias embeddings are the only extra keys).

Projections, LayerNorm, GELU and the FFN are plain library GEMMs and
elementwise ops (hipBLASLt through torch); run them under
``torch.autocast("cuda", dtype=torch.bfloat16)`` for the bf16 window step.  The
attention core is ``CoreAttention`` (HIP kernels only).

Related keys.  A window's queries may also attend to out-of-window related
nodes whose K/V come from a cache (one ``(k, v)`` pair of ``[R, H, d]`` tensors
per layer, detached).  They are appended after the window's own key rows, so
edge_index key ids ``>= N`` address them; queries are the window's N nodes.
The reference's ``dup_nodes_kv_cache`` (a detached K/V prefix replacing the
first rows, :148-168) is the same mechanism placed in front of the window's
rows; it is dead in the reference's training loop and is not offered here.
``window_step`` mirrors one iteration of ``train_epoch``
(NeutronGT/core/node_level_pipeline/train_eval.py:255-300) on one GPU.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import CoreAttention


def init_params(module: nn.Module, n_layers: int) -> None:
    """Linear weights ~ N(0, 0.02/sqrt(n_layers)), zero bias; embeddings
    N(0, 0.02) (graphormer_dist_node_level.py:10-15)."""
    if isinstance(module, nn.Linear):
        nn.init.normal_(module.weight, mean=0.0, std=0.02 / math.sqrt(n_layers))
        if module.bias is not None:
            nn.init.zeros_(module.bias)
    elif isinstance(module, nn.Embedding):
        nn.init.normal_(module.weight, mean=0.0, std=0.02)


class FeedForwardNetwork(nn.Module):
    """Linear -> GELU -> Linear (:18-30)."""

    def __init__(self, hidden_size: int, ffn_size: int, dropout_rate: float = 0.0):
        super().__init__()
        self.layer1 = nn.Linear(hidden_size, ffn_size)
        self.gelu = nn.GELU()
        self.layer2 = nn.Linear(ffn_size, hidden_size)

    def forward(self, x):
        return self.layer2(self.gelu(self.layer1(x)))


class MultiHeadAttention(nn.Module):
    """Q/K/V projections, the attention core, output projection (:128-173).

    forward(x [1, N, hidden], edge_index, attn_type, kv_cache=None)
      -> (y [1, N, hidden], node_score, [k, v])
    ``kv_cache``: optional ``(k_r, v_r)``, each ``[R, H, d]``, appended after
    the window's own keys (related nodes; no gradient flows into them).
    """

    def __init__(self, hidden_size: int, attention_dropout_rate: float, num_heads: int):
        super().__init__()
        if hidden_size % num_heads:
            raise ValueError(f"hidden size {hidden_size} is not a multiple of {num_heads} heads")
        self.num_heads = num_heads
        self.att_size = hidden_size // num_heads
        self.linear_q = nn.Linear(hidden_size, num_heads * self.att_size)
        self.linear_k = nn.Linear(hidden_size, num_heads * self.att_size)
        self.linear_v = nn.Linear(hidden_size, num_heads * self.att_size)
        self.local_attn = CoreAttention(hidden_size, attention_dropout_rate, num_heads)
        self.output_layer = nn.Linear(num_heads * self.att_size, hidden_size)

    def forward(self, x, edge_index=None, attn_type="sparse", kv_cache=None):
        b, n, _ = x.shape
        H, d = self.num_heads, self.att_size
        q = self.linear_q(x).view(b, n, H, d)
        k = self.linear_k(x).view(b, n, H, d)
        v = self.linear_v(x).view(b, n, H, d)
        k_all, v_all = k, v
        if kv_cache is not None:
            k_r, v_r = kv_cache
            if k_r.shape != v_r.shape or tuple(k_r.shape[1:]) != (H, d):
                raise ValueError(f"kv_cache rows must be [R, {H}, {d}], got {tuple(k_r.shape)}")
            k_all = torch.cat([k, k_r.detach().to(k.dtype).unsqueeze(0)], dim=1)
            v_all = torch.cat([v, v_r.detach().to(v.dtype).unsqueeze(0)], dim=1)
        # the core needs one dtype for q, k, v (autocast gives bf16 for all three)
        y, score = self.local_attn(q, k_all, v_all, None, edge_index, attn_type)
        y = self.output_layer(y)
        if y.shape != x.shape:
            raise RuntimeError(f"attention output {tuple(y.shape)} != input {tuple(x.shape)}")
        return y, score, [k, v]


class EncoderLayer(nn.Module):
    """Pre-LN block: x + Drop(MHA(LN(x))), then x + Drop(FFN(LN(x))) (:176-206)."""

    def __init__(self, hidden_size: int, ffn_size: int, dropout_rate: float,
                 attention_dropout_rate: float, num_heads: int):
        super().__init__()
        self.self_attention_norm = nn.LayerNorm(hidden_size)
        self.self_attention = MultiHeadAttention(hidden_size, attention_dropout_rate, num_heads)
        self.self_attention_dropout = nn.Dropout(dropout_rate)
        self.ffn_norm = nn.LayerNorm(hidden_size)
        self.ffn = FeedForwardNetwork(hidden_size, ffn_size, dropout_rate)
        self.ffn_dropout = nn.Dropout(dropout_rate)

    def forward(self, x, edge_index=None, attn_type="sparse", kv_cache=None):
        y, score, kv = self.self_attention(self.self_attention_norm(x), edge_index, attn_type,
                                           kv_cache)
        x = x + self.self_attention_dropout(y)
        x = x + self.ffn_dropout(self.ffn(self.ffn_norm(x)))
        return x, score, kv


class WindowGraphormer(nn.Module):
    """Node-level Graphormer over one window (:242-381, struct_enc False).

    forward(x [N, input_dim], edge_index [2, E], attn_type="sparse",
            kv_cache=None (list of per-layer (k_r, v_r)))
      -> (log_probs [N, output_dim], per-layer node scores (detached))
    """

    def __init__(self, n_layers: int, num_heads: int, input_dim: int, hidden_dim: int,
                 output_dim: int, dropout_rate: float = 0.0, input_dropout_rate: float = 0.0,
                 attention_dropout_rate: float = 0.0, ffn_dim: int | None = None):
        super().__init__()
        ffn_dim = ffn_dim or hidden_dim
        self.num_heads = num_heads
        self.n_layers = n_layers
        self.node_encoder = nn.Linear(input_dim, hidden_dim)
        self.input_dropout = nn.Dropout(input_dropout_rate)
        self.layers = nn.ModuleList([
            EncoderLayer(hidden_dim, ffn_dim, dropout_rate, attention_dropout_rate, num_heads)
            for _ in range(n_layers)])
        self.final_ln = nn.LayerNorm(hidden_dim)
        self.downstream_out_proj = nn.Linear(hidden_dim, output_dim)
        self.apply(lambda m: init_params(m, n_layers))

    def forward(self, x, edge_index, attn_type="sparse", kv_cache=None):
        if kv_cache is not None and len(kv_cache) != self.n_layers:
            raise ValueError(f"kv_cache has {len(kv_cache)} entries for {self.n_layers} layers")
        h = self.input_dropout(self.node_encoder(x.unsqueeze(0)))
        scores = []
        for i, layer in enumerate(self.layers):
            h, score, _ = layer(h, edge_index, attn_type,
                                kv_cache[i] if kv_cache is not None else None)
            scores.append(score.detach() if score is not None else None)
        h = self.final_ln(h)
        out = self.downstream_out_proj(h[0])
        return F.log_softmax(out.float(), dim=1), scores


def window_step(model: nn.Module, optimizer, x, edge_index, labels, train_mask,
                kv_cache=None, autocast_dtype=None):
    """One window iteration of train_eval.py:255-300 on one GPU: forward, NLL
    over the window's training nodes, backward, optimizer step.  Returns
    (loss tensor, last layer's node scores).  ``autocast_dtype`` (e.g.
    torch.bfloat16) runs the forward under torch.autocast."""
    if autocast_dtype is not None:
        with torch.autocast("cuda", dtype=autocast_dtype):
            out, scores = model(x, edge_index, "sparse", kv_cache)
    else:
        out, scores = model(x, edge_index, "sparse", kv_cache)
    loss = F.nll_loss(out[train_mask], labels[train_mask])
    optimizer.zero_grad(set_to_none=True)
    loss.backward()
    optimizer.step()
    return loss.detach(), scores[-1]
