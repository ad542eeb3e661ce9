"""CPU restatement of NeutronGT's two window encoders (test oracle only).

Functional torch code over a ``state_dict`` (parameter tensors by name), so
that it shares nothing with the product's module classes but the parameter
names, which are the reference's.  Eval mode: every dropout is the identity.
Structural encodings off (``struct_enc`` False, the shipped setting) and no
``dup_nodes_kv_cache`` (dead in the reference's training loop), so the window
is square: every node is a query and a key.

  graphormer_forward   Graphormer.forward (NeutronGT/models/graphormer_dist_node_level.py:
                       291-381) over pre-LN EncoderLayer (:176-206), MultiHeadAttention
                       (:128-173, output projection inside), FeedForwardNetwork
                       (:18-30, GELU), final_ln and downstream_out_proj.
  gt_forward           GT_SW.forward (NeutronGT/models/gt_dist_node_level_single_window.py:
                       569-680) over the post-LN EncoderLayer (:305-353: y = O(MHA(x));
                       x = LN1(x + y); the FFN reads y, not x; x = LN2(x + FFN(y))),
                       MultiHeadAttention without output projection (:230-302) and
                       MLPReadout (:356-372).

The attention core is ``oracle.attention.sparse_attention_bias`` (sparse) or
``full_attention`` (full), the restatements of CoreAttention.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import attention as OA

LN_EPS = 1e-5  # nn.LayerNorm's default, used by every LayerNorm of both encoders


def _linear(p, name, x):
    return F.linear(x, p[name + ".weight"], p.get(name + ".bias"))


def _ln(p, name, x):
    return F.layer_norm(x, (x.shape[-1],), p[name + ".weight"], p[name + ".bias"], LN_EPS)


def _attention_core(q, k, v, edge_index, num_heads, attn_type):
    """CoreAttention.forward (graphormer_dist_node_level.py:107-127) for the
    sparse and full branches: returns (x [1, N, H*d], score)."""
    b, n = q.shape[0], q.shape[1]
    if attn_type == "sparse":
        x, score = OA.sparse_attention_bias(q, k, v, edge_index, num_heads)
    else:
        x, score = OA.full_attention(q, k, v)
    return x.reshape(b, n, -1), score


def _qkv(p, prefix, x, num_heads):
    b = x.shape[0]
    hidden = x.shape[-1]
    d = hidden // num_heads
    q = _linear(p, prefix + "linear_q", x).view(b, -1, num_heads, d)
    k = _linear(p, prefix + "linear_k", x).view(b, -1, num_heads, d)
    v = _linear(p, prefix + "linear_v", x).view(b, -1, num_heads, d)
    return q, k, v


def graphormer_layer(p, i, h, edge_index, num_heads, attn_type="sparse"):
    """EncoderLayer.forward (graphormer_dist_node_level.py:187-206), eval mode:
    y = LN(x); y = MHA(y); x = x + y; y = LN(x); y = FFN(y); x = x + y."""
    pre = f"layers.{i}."
    y = _ln(p, pre + "self_attention_norm", h)
    q, k, v = _qkv(p, pre + "self_attention.", y, num_heads)
    y, score = _attention_core(q, k, v, edge_index, num_heads, attn_type)
    y = _linear(p, pre + "self_attention.output_layer", y)
    h = h + y
    y = _ln(p, pre + "ffn_norm", h)
    y = _linear(p, pre + "ffn.layer2", F.gelu(_linear(p, pre + "ffn.layer1", y)))
    return h + y, score


def graphormer_forward(p, x, edge_index, n_layers, num_heads, attn_type="sparse"):
    """Graphormer.forward (graphormer_dist_node_level.py:291-381): x [N, F] ->
    (log_softmax logits [N, C], per-layer node scores)."""
    h = _linear(p, "node_encoder", x.unsqueeze(0))
    scores = []
    for i in range(n_layers):
        h, score = graphormer_layer(p, i, h, edge_index, num_heads, attn_type)
        scores.append(score.detach())
    h = _ln(p, "final_ln", h)
    out = _linear(p, "downstream_out_proj", h[0])
    return F.log_softmax(out, dim=1), scores


def gt_layer(p, i, h, edge_index, num_heads, attn_type="sparse"):
    """EncoderLayer.forward of the GT twin (gt_dist_node_level_single_window.py:
    322-353), eval mode, including its FFN-on-y: the FFN's input is the
    attention branch y, not the normalised residual stream x."""
    pre = f"layers.{i}."
    q, k, v = _qkv(p, pre + "self_attention.", h, num_heads)
    y, score = _attention_core(q, k, v, edge_index, num_heads, attn_type)
    y = _linear(p, pre + "O", y)
    h = _ln(p, pre + "layer_norm1", h + y)
    y = _linear(p, pre + "FFN_layer2", F.relu(_linear(p, pre + "FFN_layer1", y)))
    h = _ln(p, pre + "layer_norm2", h + y)
    return h, score


def mlp_readout(p, x, L=2):
    """MLPReadout.forward (gt_dist_node_level_single_window.py:366-372)."""
    for i in range(L):
        x = F.relu(_linear(p, f"MLP_layer.FC_layers.{i}", x))
    return _linear(p, f"MLP_layer.FC_layers.{L}", x)


def gt_forward(p, x, edge_index, n_layers, num_heads, attn_type="sparse"):
    """GT_SW.forward (gt_dist_node_level_single_window.py:590-680): x [N, F] ->
    (log_softmax logits [N, C], per-layer node scores)."""
    h = _linear(p, "node_encoder", x.unsqueeze(0))
    scores = []
    for i in range(n_layers):
        h, score = gt_layer(p, i, h, edge_index, num_heads, attn_type)
        scores.append(score.detach())
    out = mlp_readout(p, h[0])
    return F.log_softmax(out, dim=1), scores
