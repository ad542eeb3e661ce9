"""Literal CPU restatement of NeutronGT's attention core (test oracle only).

Follows, op for op, the reference's torch code:
  sparse:  NeutronGT/models/graphormer_dist_node_level.py:67-98
           (twin NeutronGT/models/gt_dist_node_level_single_window.py:112-179)
  dense:   NeutronGT/models/graphormer_dist_node_level.py:42-65
           (twin NeutronGT/models/gt_dist_node_level_single_window.py:56-109)
torch_scatter 2.1.1's ``scatter(src, index, dim=0, out=..., reduce='add')`` is
restated as its published algorithm: broadcast the index over ``src`` and call
``Tensor.scatter_add_``; without ``out`` the result has ``index.max() + 1`` rows.

Also holds two independent formulations used to pin the restatement:
``sparse_bruteforce_fp64`` (dense masked matrix form, float64) and
``sparse_backward_closed_form`` (hand-derived gradients).
"""
from __future__ import annotations

import math

import torch

CLAMP_LO = -5.0
CLAMP_HI = 5.0
EPS = 1e-6


def _scatter_add(src: torch.Tensor, index: torch.Tensor, out: torch.Tensor | None = None):
    """torch_scatter.scatter(..., dim=0, reduce='add') (scatter_sum)."""
    idx = index.to(torch.long).view(-1, *([1] * (src.dim() - 1))).expand_as(src)
    if out is None:
        size = int(index.max()) + 1 if index.numel() > 0 else 0
        out = src.new_zeros((size,) + tuple(src.shape[1:]))
    return out.scatter_add_(0, idx, src)


def sparse_attention_bias(q, k, v, edge_index, num_heads, attn_bias=None, scale=None):
    """CoreAttention.sparse_attention_bias (graphormer_dist_node_level.py:67-98).

    q: [1, N_q, H, d]; k, v: [1, N_k, H, d] with N_q <= N_k (the queries are the
    first N_q window rows; rows N_q.. have no in-edges).  Returns
    (x [N_k, H, d] -- the reference's full wV/(Z+eps), node_scores [max(dst)+1]).
    """
    head_dim = q.shape[-1]
    if scale is None:
        scale = math.sqrt(head_dim)  # sqrt(hidden_size // num_heads)
    batch_size, node_num = k.size(0), k.size(1)
    q = q.reshape(-1, num_heads, head_dim)
    k = k.reshape(-1, num_heads, head_dim)
    v = v.reshape(-1, num_heads, head_dim)
    src = k[edge_index[0].to(torch.long)]
    dest = q[edge_index[1].to(torch.long)]
    score = torch.mul(src, dest)
    score = score / scale
    score = score.sum(-1, keepdim=True).clamp(CLAMP_LO, CLAMP_HI)
    if attn_bias is not None:
        attn_bias = attn_bias.permute(0, 2, 3, 1).contiguous().unsqueeze(2).repeat(1, 1, batch_size, 1, 1)
        attn_bias = attn_bias.view(batch_size * node_num, batch_size * node_num, num_heads)
        score = score + attn_bias[edge_index[0].to(torch.long), edge_index[1].to(torch.long), :].unsqueeze(2)
    score = torch.exp(score)
    msg = v[edge_index[0].to(torch.long)] * score
    wv = torch.zeros_like(v)
    _scatter_add(msg, edge_index[1], out=wv)
    z = score.new_zeros(v.size(0), num_heads, 1)
    _scatter_add(score, edge_index[1], out=z)
    x = wv / (z + EPS)
    node_scores = score.mean(dim=1).squeeze(-1)
    node_scores = _scatter_add(node_scores, edge_index[1])
    return x, node_scores


def full_attention(q, k, v, scale=None, attn_bias=None, mask=None, pruning_mask=None):
    """CoreAttention.full_attention (graphormer_dist_node_level.py:42-65), dropout p = 0.

    q: [1, N_q, H, d]; k, v: [1, N_k, H, d].  Returns (x [1, N_q, H, d],
    node_scores [N_k]).  Note the reference MULTIPLIES q by sqrt(d).
    """
    if scale is None:
        scale = math.sqrt(q.shape[-1])
    q = q.transpose(1, 2)
    v = v.transpose(1, 2)
    k = k.transpose(1, 2).transpose(2, 3)
    q = q * scale
    x = torch.matmul(q, k)
    score = x
    if attn_bias is not None:
        x = x + attn_bias
    if pruning_mask is not None:
        x = x + pruning_mask
    if mask is not None:
        mask = mask.to(x.device).unsqueeze(0).unsqueeze(0)
        mask = mask.repeat(1, x.shape[1], 1, 1)
        x = x.masked_fill(mask, -1e9)
    x = torch.softmax(x, dim=3)
    x = x.matmul(v)
    x = x.transpose(1, 2).contiguous()
    node_scores = torch.abs(score).mean(dim=1).squeeze(0).sum(dim=0)
    return x, node_scores


# --------------------------------------------------------------- pinning forms
def sparse_bruteforce_fp64(q, k, v, edge_index, scale=None, lo=CLAMP_LO, hi=CLAMP_HI, eps=EPS):
    """Dense masked-matrix form in float64: C[i,j] = #edges j->i,
    P = C * exp(clamp(Q K^T / scale)), X = P V / (rowsum P + eps)."""
    q = q.reshape(q.shape[-3], q.shape[-2], q.shape[-1]).double()
    k = k.reshape(k.shape[-3], k.shape[-2], k.shape[-1]).double()
    v = v.reshape(v.shape[-3], v.shape[-2], v.shape[-1]).double()
    n_q, n_k, d = q.shape[0], k.shape[0], q.shape[-1]
    if scale is None:
        scale = math.sqrt(d)
    cnt = torch.zeros(n_q, n_k, dtype=torch.float64)
    ei = edge_index.to(torch.long)
    cnt.index_put_((ei[1], ei[0]), torch.ones(ei.shape[1], dtype=torch.float64), accumulate=True)
    s = torch.einsum("ihc,jhc->hij", q, k) / scale
    p = cnt.unsqueeze(0) * torch.exp(s.clamp(lo, hi))
    z = p.sum(-1)  # [H, n_q]
    x = torch.einsum("hij,jhc->ihc", p, v) / (z.t().unsqueeze(-1) + eps)
    return x, z.t()  # x [n_q, H, d], Z [n_q, H]


def sparse_backward_closed_form(q, k, v, edge_index, grad_x, scale=None, lo=CLAMP_LO,
                                hi=CLAMP_HI, eps=EPS):
    """Hand-derived gradients of x = wV/(Z+eps) (fp64, edge loop vectorised).

    dp_e = r_i (G_i . V_j - D_i) with r = 1/(Z+eps), D_i = G_i . X_i;
    da_e = dp_e p_e [lo <= a_e <= hi];  dQ_i += da K_j/s;  dK_j += da Q_i/s;
    dV_j += p r_i G_i.
    """
    q = q.reshape(q.shape[-3], q.shape[-2], q.shape[-1]).double()
    k = k.reshape(k.shape[-3], k.shape[-2], k.shape[-1]).double()
    v = v.reshape(v.shape[-3], v.shape[-2], v.shape[-1]).double()
    n_q, h, d = q.shape
    g = grad_x.reshape(-1, h, d)[:n_q].double()
    if scale is None:
        scale = math.sqrt(d)
    j = edge_index[0].to(torch.long)
    i = edge_index[1].to(torch.long)
    a = (k[j] * q[i]).sum(-1) / scale  # [E, H]
    p = torch.exp(a.clamp(lo, hi))
    z = torch.zeros(n_q, h, dtype=torch.float64).index_add_(0, i, p)
    wv = torch.zeros(n_q, h, d, dtype=torch.float64).index_add_(0, i, p.unsqueeze(-1) * v[j])
    r = 1.0 / (z + eps)
    x = wv * r.unsqueeze(-1)
    dd = (g * x).sum(-1)  # [n_q, H]
    dp = r[i] * ((g[i] * v[j]).sum(-1) - dd[i])
    inside = ((a >= lo) & (a <= hi)).double()
    da = dp * p * inside
    dq = torch.zeros_like(q).index_add_(0, i, da.unsqueeze(-1) * k[j] / scale)
    dk = torch.zeros_like(k).index_add_(0, j, da.unsqueeze(-1) * q[i] / scale)
    dv = torch.zeros_like(v).index_add_(0, j, (p * r[i]).unsqueeze(-1) * g[i])
    return dq, dk, dv


def full_attention_fp64(q, k, v, scale=None):
    """softmax((q*scale) k^T) v per head in float64; also returns sum_i mean_h |S|."""
    q = q.reshape(q.shape[-3], q.shape[-2], q.shape[-1]).double()
    k = k.reshape(k.shape[-3], k.shape[-2], k.shape[-1]).double()
    v = v.reshape(v.shape[-3], v.shape[-2], v.shape[-1]).double()
    if scale is None:
        scale = math.sqrt(q.shape[-1])
    s = torch.einsum("ihc,jhc->hij", q * scale, k)
    p = torch.softmax(s, dim=-1)
    x = torch.einsum("hij,jhc->ihc", p, v)
    ns = s.abs().mean(0).sum(0)
    return x, ns


# --------------------------------------------------------- autograd wrappers
def sparse_fwd_bwd(q, k, v, edge_index, grad_x, num_heads, dtype=torch.float32):
    """Runs the restatement forward + autograd backward on CPU in ``dtype``.

    q [N_q,H,d], k/v [N_k,H,d] (any float dtype; cast to ``dtype``), grad_x
    [N_q,H,d].  Returns dict(x [N_q,H,d], node_scores, dq, dk, dv).
    """
    n_q = q.shape[0]
    n_k = k.shape[0]
    n = max(n_q, n_k)  # the reference's square window: padded rows have no edges
    qf = torch.zeros(n, *q.shape[1:], dtype=dtype)
    qf[:n_q] = q.to(dtype)
    kf = torch.zeros(n, *k.shape[1:], dtype=dtype)
    kf[:n_k] = k.to(dtype)
    vf = torch.zeros(n, *v.shape[1:], dtype=dtype)
    vf[:n_k] = v.to(dtype)
    for t in (qf, kf, vf):
        t.requires_grad_(True)
    x, ns = sparse_attention_bias(qf.unsqueeze(0), kf.unsqueeze(0), vf.unsqueeze(0), edge_index,
                                  num_heads)
    g = torch.zeros_like(x)
    g[:n_q] = grad_x.to(dtype)
    x.backward(g)
    return {
        "x": x.detach()[:n_q],
        "node_scores": ns.detach(),
        "dq": qf.grad[:n_q],
        "dk": kf.grad[:n_k],
        "dv": vf.grad[:n_k],
    }


def full_fwd_bwd(q, k, v, grad_x, dtype=torch.float32):
    """full_attention forward + autograd backward on CPU; q [N_q,H,d], k/v [N_k,H,d]."""
    qf = q.to(dtype).clone().unsqueeze(0).requires_grad_(True)
    kf = k.to(dtype).clone().unsqueeze(0).requires_grad_(True)
    vf = v.to(dtype).clone().unsqueeze(0).requires_grad_(True)
    x, ns = full_attention(qf, kf, vf)
    x.backward(grad_x.to(dtype).unsqueeze(0))
    return {
        "x": x.detach()[0],
        "node_scores": ns.detach(),
        "dq": qf.grad[0],
        "dk": kf.grad[0],
        "dv": vf.grad[0],
    }
