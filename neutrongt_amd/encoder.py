"""The window encoders around the HIP attention core: the caller side of the path.

Two model families, as in NeutronGT's node-level pipeline (struct_enc False,
the shipped setting):

  WindowGraphormer  NeutronGT/models/graphormer_dist_node_level.py: pre-LN
                    ``EncoderLayer`` (:176-206) with ``MultiHeadAttention``
                    (:128-173, output projection inside) and the GELU
                    ``FeedForwardNetwork`` (:18-30); final LayerNorm and a
                    linear readout (``Graphormer.forward``, :242-381).
  WindowGT          NeutronGT/models/gt_dist_node_level_single_window.py:
                    post-LN ``EncoderLayer`` (:305-353) whose attention block
                    has no output projection (:230-302), ReLU FFN of width
                    2*hidden, and the ``MLPReadout`` head (``GT_SW``, :505-680).

Sub-module and parameter names are the reference's, so a reference
``state_dict`` loads with ``strict=False`` (the unused structural-encoding
embeddings are the only extra keys).  Projections, activations and the FFN are
library GEMMs and elementwise ops (hipBLASLt through torch); the linear layers'
weight and bias gradients run through ``WgradLinear`` (a row-split GEMM and the
library's column sums) and the LayerNorms through ``FusedLayerNorm`` (the
library's fused kernels).  Run them under
``torch.autocast("cuda", dtype=torch.bfloat16)`` for the bf16 window step.
The attention core is ``CoreAttention`` (HIP kernels only).

Related keys.  A window's queries may also attend to out-of-window related
nodes whose K/V come from a cache (one ``(k, v)`` pair of ``[R, H, d]`` tensors
per layer, detached).  They are appended after the window's own key rows, so
edge_index key ids ``>= N`` address them; queries are the window's N nodes.
The reference's ``dup_nodes_kv_cache`` (a detached K/V prefix replacing the
first rows, graphormer_dist_node_level.py:148-168) is the same mechanism placed
in front of the window's rows; it is dead in the reference's training loop and
is not offered here.  ``window_step`` mirrors one iteration of ``train_epoch``
(NeutronGT/core/node_level_pipeline/train_eval.py:255-300) on one GPU.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import CoreAttention
from .layernorm import FusedLayerNorm, add_dropout_layernorm
from .linear import WgradLinear, groupable, project


def init_params(module: nn.Module, n_layers: int) -> None:
    """Linear weights ~ N(0, 0.02/sqrt(n_layers)), zero bias; embeddings
    N(0, 0.02) (graphormer_dist_node_level.py:10-15; the GT twin's :22-28)."""
    if isinstance(module, nn.Linear):
        nn.init.normal_(module.weight, mean=0.0, std=0.02 / math.sqrt(n_layers))
        if module.bias is not None:
            nn.init.zeros_(module.bias)
    elif isinstance(module, nn.Embedding):
        nn.init.normal_(module.weight, mean=0.0, std=0.02)


class FeedForwardNetwork(nn.Module):
    """Linear -> GELU -> Linear (graphormer_dist_node_level.py:18-30)."""

    def __init__(self, hidden_size: int, ffn_size: int, dropout_rate: float = 0.0):
        super().__init__()
        self.layer1 = WgradLinear(hidden_size, ffn_size)
        self.gelu = nn.GELU()
        self.layer2 = WgradLinear(ffn_size, hidden_size)

    def forward(self, x):
        return self.layer2(self.gelu(self.layer1(x)))


class _Attention(nn.Module):
    """Q/K/V projections and the attention core, shared by both families.

    attend(x [1, N, hidden], edge_index, attn_type, kv_cache=None)
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
        self.linear_q = WgradLinear(hidden_size, num_heads * self.att_size)
        self.linear_k = WgradLinear(hidden_size, num_heads * self.att_size)
        self.linear_v = WgradLinear(hidden_size, num_heads * self.att_size)
        self.local_attn = CoreAttention(hidden_size, attention_dropout_rate, num_heads)

    def attend(self, x, edge_index, attn_type, kv_cache):
        b, n, _ = x.shape
        H, d = self.num_heads, self.att_size
        lins = (self.linear_q, self.linear_k, self.linear_v)
        # one projection node, and the sparse core hands back dQ, dK, dV as
        # column blocks of one matrix for its backward
        interleave = (groupable(x, *lins) and attn_type == "sparse"
                      and isinstance(self.local_attn, CoreAttention))
        extra = {"interleave_grads": True} if interleave else {}
        q, k, v = project(x, *lins)
        q, k, v = q.view(b, n, H, d), k.view(b, n, H, d), v.view(b, n, H, d)
        if kv_cache is None:
            y, score = self.local_attn(q, k, v, None, edge_index, attn_type, **extra)
            return y, score, [k, v]
        k_r, v_r = kv_cache
        if k_r.shape != v_r.shape or tuple(k_r.shape[1:]) != (H, d):
            raise ValueError(f"kv_cache rows must be [R, {H}, {d}], got {tuple(k_r.shape)}")
        # the core needs one dtype for q, k, v (autocast gives bf16 for all three)
        k_r, v_r = k_r.detach().to(k.dtype), v_r.detach().to(v.dtype)
        if isinstance(self.local_attn, CoreAttention):
            # read from the cache's own buffers: no concatenation, no gradient
            y, score = self.local_attn(q, k, v, None, edge_index, attn_type, kv_ext=(k_r, v_r),
                                       **extra)
        else:  # another core (e.g. the reference's) takes the concatenated keys
            y, score = self.local_attn(q, torch.cat([k, k_r.unsqueeze(0)], dim=1),
                                       torch.cat([v, v_r.unsqueeze(0)], dim=1), None,
                                       edge_index, attn_type)
        return y, score, [k, v]


class MultiHeadAttention(_Attention):
    """Graphormer attention block: projections, core, output projection
    (graphormer_dist_node_level.py:128-173)."""

    def __init__(self, hidden_size: int, attention_dropout_rate: float, num_heads: int):
        super().__init__(hidden_size, attention_dropout_rate, num_heads)
        self.output_layer = WgradLinear(num_heads * self.att_size, hidden_size)

    def forward(self, x, edge_index=None, attn_type="sparse", kv_cache=None):
        y, score, kv = self.attend(x, edge_index, attn_type, kv_cache)
        y = self.output_layer(y)
        if y.shape != x.shape:
            raise RuntimeError(f"attention output {tuple(y.shape)} != input {tuple(x.shape)}")
        return y, score, kv


class GTMultiHeadAttention(_Attention):
    """GT attention block: projections and core, no output projection (the
    layer's ``O`` follows it; gt_dist_node_level_single_window.py:230-302)."""

    def forward(self, x, edge_index=None, attn_type="sparse", kv_cache=None):
        y, score, kv = self.attend(x, edge_index, attn_type, kv_cache)
        if y.shape != x.shape:
            raise RuntimeError(f"attention output {tuple(y.shape)} != input {tuple(x.shape)}")
        return y, score, kv


class EncoderLayer(nn.Module):
    """Pre-LN block: x + Drop(MHA(LN(x))), then x + Drop(FFN(LN(x)))
    (graphormer_dist_node_level.py:176-206)."""

    def __init__(self, hidden_size: int, ffn_size: int, dropout_rate: float,
                 attention_dropout_rate: float, num_heads: int):
        super().__init__()
        # pre-LN: both norms feed only bf16 linear layers (bf16 output under autocast)
        self.self_attention_norm = FusedLayerNorm(hidden_size, out_bf16=True)
        self.self_attention = MultiHeadAttention(hidden_size, attention_dropout_rate, num_heads)
        self.self_attention_dropout = nn.Dropout(dropout_rate)
        self.ffn_norm = FusedLayerNorm(hidden_size, out_bf16=True)
        self.ffn = FeedForwardNetwork(hidden_size, ffn_size, dropout_rate)
        self.ffn_dropout = nn.Dropout(dropout_rate)

    def forward(self, x, edge_index=None, attn_type="sparse", kv_cache=None):
        x, f, score, kv = self.forward_open(x, self.self_attention_norm(x), edge_index,
                                            attn_type, kv_cache)
        return x + self.ffn_dropout(f), score, kv

    def forward_open(self, x, x_norm, edge_index=None, attn_type="sparse", kv_cache=None):
        """The block from x and its LayerNorm x_norm = self_attention_norm(x)
        on, with the FFN's residual add left open: returns (x', f, score, kv),
        the block's output being x' + ffn_dropout(f).  A stack closes it
        together with the next LayerNorm (add_dropout_layernorm)."""
        y, score, kv = self.self_attention(x_norm, edge_index, attn_type, kv_cache)
        # x + Drop(y) and the FFN's LayerNorm of it: one fused pass under bf16 autocast
        x, h = add_dropout_layernorm(x, y, self.ffn_norm, self.self_attention_dropout)
        return x, self.ffn(h), score, kv


class GTEncoderLayer(nn.Module):
    """GT post-LN block (gt_dist_node_level_single_window.py:305-353):
    y = O(Drop(MHA(x))); x = LN1(x + y); then the FFN (hidden -> 2*hidden ->
    hidden, ReLU, dropout in between) is applied to y -- not to x -- and
    x = LN2(x + FFN(y)).  The FFN input is the reference's as written (its own
    comment questions it); kept so the layer computes the same function."""

    def __init__(self, hidden_size: int, ffn_size: int, dropout_rate: float,
                 attention_dropout_rate: float, num_heads: int):
        super().__init__()
        self.self_attention_norm = nn.LayerNorm(hidden_size)  # declared, unused (as in the reference)
        self.self_attention = GTMultiHeadAttention(hidden_size, attention_dropout_rate, num_heads)
        self.self_attention_dropout = nn.Dropout(dropout_rate)
        self.O = WgradLinear(hidden_size, hidden_size)
        self.layer_norm1 = FusedLayerNorm(hidden_size)  # the residual stream: fp32 as autocast
        self.FFN_layer1 = WgradLinear(hidden_size, hidden_size * 2)
        self.FFN_layer2 = WgradLinear(hidden_size * 2, hidden_size)
        self.layer_norm2 = FusedLayerNorm(hidden_size)

    def forward(self, x, edge_index=None, attn_type="sparse", kv_cache=None):
        y, score, kv = self.self_attention(x, edge_index, attn_type, kv_cache)
        y = self.O(self.self_attention_dropout(y))
        x = self.layer_norm1(x + y)
        y = self.FFN_layer2(self.self_attention_dropout(F.relu(self.FFN_layer1(y))))
        x = self.layer_norm2(x + y)
        return x, score, kv


class MLPReadout(nn.Module):
    """hidden -> hidden/2 -> hidden/4 -> output, ReLU between
    (gt_dist_node_level_single_window.py:356-372)."""

    def __init__(self, input_dim: int, output_dim: int, L: int = 2):
        super().__init__()
        dims = [input_dim // 2 ** i for i in range(L + 1)]
        self.FC_layers = nn.ModuleList(
            [WgradLinear(dims[i], dims[i + 1]) for i in range(L)] + [WgradLinear(dims[L], output_dim)])
        self.L = L

    def forward(self, x):
        for i in range(self.L):
            x = F.relu(self.FC_layers[i](x))
        return self.FC_layers[self.L](x)


class _WindowModel(nn.Module):
    """node_encoder -> input dropout -> layers -> readout -> log_softmax.

    forward(x [N, input_dim], edge_index [2, E], attn_type="sparse",
            kv_cache=None (list of per-layer (k_r, v_r)))
      -> (log_probs [N, output_dim], per-layer node scores (detached))
    """

    def forward(self, x, edge_index, attn_type="sparse", kv_cache=None):
        if kv_cache is not None and len(kv_cache) != self.n_layers:
            raise ValueError(f"kv_cache has {len(kv_cache)} entries for {self.n_layers} layers")
        h = self.input_dropout(self.node_encoder(x.unsqueeze(0)))
        scores = []
        if isinstance(self, WindowGraphormer) and self.n_layers > 0:
            # pre-LN stack: each block's FFN residual add + dropout and the
            # LayerNorm after it (the next block's, or final_ln) are one pass
            h_norm = self.layers[0].self_attention_norm(h)
            for i, layer in enumerate(self.layers):
                x_res, f, score, _ = layer.forward_open(
                    h, h_norm, edge_index, attn_type,
                    kv_cache[i] if kv_cache is not None else None)
                scores.append(score.detach() if score is not None else None)
                ln = (self.layers[i + 1].self_attention_norm if i + 1 < self.n_layers
                      else self.final_ln)
                h, h_norm = add_dropout_layernorm(x_res, f, ln, layer.ffn_dropout)
            logits = self.downstream_out_proj(h_norm[0])
            return F.log_softmax(logits.float(), dim=1), scores
        for i, layer in enumerate(self.layers):
            h, score, _ = layer(h, edge_index, attn_type,
                                kv_cache[i] if kv_cache is not None else None)
            scores.append(score.detach() if score is not None else None)
        return F.log_softmax(self.readout(h[0]).float(), dim=1), scores


class WindowGraphormer(_WindowModel):
    """Node-level Graphormer over one window (graphormer_dist_node_level.py:242-381)."""

    def __init__(self, n_layers: int, num_heads: int, input_dim: int, hidden_dim: int,
                 output_dim: int, dropout_rate: float = 0.0, input_dropout_rate: float = 0.0,
                 attention_dropout_rate: float = 0.0, ffn_dim: int | None = None):
        super().__init__()
        ffn_dim = ffn_dim or hidden_dim
        self.num_heads = num_heads
        self.n_layers = n_layers
        self.node_encoder = WgradLinear(input_dim, hidden_dim)
        self.input_dropout = nn.Dropout(input_dropout_rate)
        self.layers = nn.ModuleList([
            EncoderLayer(hidden_dim, ffn_dim, dropout_rate, attention_dropout_rate, num_heads)
            for _ in range(n_layers)])
        self.final_ln = FusedLayerNorm(hidden_dim, out_bf16=True)  # feeds the readout linear
        self.downstream_out_proj = WgradLinear(hidden_dim, output_dim)
        self.apply(lambda m: init_params(m, n_layers))

    def readout(self, h):
        return self.downstream_out_proj(self.final_ln(h))


class WindowGT(_WindowModel):
    """Node-level GT over one window (GT_SW, gt_dist_node_level_single_window.py:505-680).
    ``ffn_dim`` is accepted and unused: the GT layer's FFN is 2*hidden wide."""

    def __init__(self, n_layers: int, num_heads: int, input_dim: int, hidden_dim: int,
                 output_dim: int, dropout_rate: float = 0.0, input_dropout_rate: float = 0.0,
                 attention_dropout_rate: float = 0.0, ffn_dim: int | None = None):
        super().__init__()
        self.num_heads = num_heads
        self.n_layers = n_layers
        self.node_encoder = WgradLinear(input_dim, hidden_dim)
        self.input_dropout = nn.Dropout(input_dropout_rate)
        self.layers = nn.ModuleList([
            GTEncoderLayer(hidden_dim, ffn_dim or hidden_dim, dropout_rate,
                           attention_dropout_rate, num_heads) for _ in range(n_layers)])
        self.MLP_layer = MLPReadout(hidden_dim, output_dim)
        self.downstream_out_proj = WgradLinear(hidden_dim, output_dim)  # declared, unused
        self.apply(lambda m: init_params(m, n_layers))

    def readout(self, h):
        return self.MLP_layer(h)


def window_step(model: nn.Module, optimizer, x, edge_index, labels, train_mask,
                kv_cache=None, autocast_dtype=None):
    """One window iteration of train_eval.py:255-300 on one GPU: forward, NLL
    over the window's training nodes, backward, optimizer step.  Returns
    (loss tensor, last layer's node scores).  ``autocast_dtype`` (e.g.
    torch.bfloat16) runs the forward under torch.autocast.

    Nothing here synchronises with the host, so the whole step can be captured
    in a HIP graph (with a capturable optimizer): the masked mean is a
    weighted sum, not a boolean selection (same value as the reference's
    ``loss[mask_train].mean()``)."""
    if autocast_dtype is not None:
        capturing = torch.cuda.is_current_stream_capturing()
        with torch.autocast("cuda", dtype=autocast_dtype, cache_enabled=not capturing):
            out, scores = model(x, edge_index, "sparse", kv_cache)
    else:
        out, scores = model(x, edge_index, "sparse", kv_cache)
    w = train_mask.to(out.dtype)
    loss = (F.nll_loss(out, labels, reduction="none") * w).sum() / w.sum()
    optimizer.zero_grad(set_to_none=True)
    loss.backward()
    optimizer.step()
    return loss.detach(), scores[-1]
