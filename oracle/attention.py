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

Dropout of the dense path (the reference's ``self.att_dropout(x)`` after the
softmax, and ``F.dropout(..., training=True)`` in the flash branch's
naive_attention, graphormer_dist_node_level.py:100-105) draws torch's Philox
stream, which no other implementation reproduces; the product replaces it by
a hash of (seed, head, query, key).  ``dropout_multiplier`` restates that
hash so a test can hand the same mask to this restatement; the mask's own
statistics (keep rate, independence) are what ties it to the reference.
"""
from __future__ import annotations

import math

import numpy as np
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


def _mix32(x):
    """lowbias32 (C. Wellons, hash-prospector) on a uint32 array."""
    x = x ^ (x >> np.uint32(16))
    x = x * np.uint32(0x7FEB352D)
    x = x ^ (x >> np.uint32(15))
    x = x * np.uint32(0x846CA68B)
    x = x ^ (x >> np.uint32(16))
    return x


def dropout_params(p):
    """(threshold, scale) of the product's mask for probability p (passed to
    the library as fp32): keep iff the 16-bit draw >= round(p * 65536), kept
    values scaled by fp32(1 / (1 - p)); p = 1 keeps all with scale 0."""
    p32 = float(np.float32(p))
    if p32 >= 1.0:
        return 0, np.float32(0.0)
    return int(np.rint(p32 * 65536.0)), np.float32(1.0 / (1.0 - p32))


def dropout_multiplier(seed, H, n_q, n_k, p):
    """[H, n_q, n_k] float32: the multiplier (0 or 1/(1-p)) that the product's
    dense kernels apply to P[h, i, j] for dropout probability p and a 64-bit
    seed.  One 32-bit word per key pair of a (head, query) row:
      word = mix32((i * ceil(n_k/2) + j // 2) ^ head_key),
      head_key = mix32(lo32(seed) ^ mix32(hi32(seed) + 0x9e3779b9 * (h + 1))),
    16-bit half j % 2 of the word compared with the threshold."""
    thr, scale = dropout_params(p)
    with np.errstate(over="ignore"):
        s_lo = np.uint32(seed & 0xFFFFFFFF)
        s_hi = np.uint32((seed >> 32) & 0xFFFFFFFF)
        i = np.arange(n_q, dtype=np.uint32)[:, None]
        j = np.arange(n_k, dtype=np.uint32)[None, :]
        n_kp = np.uint32((n_k + 1) // 2)
        out = np.empty((H, n_q, n_k), np.float32)
        heads = np.arange(1, H + 1, dtype=np.uint32)
        head_keys = _mix32(s_lo ^ _mix32(s_hi + np.uint32(0x9E3779B9) * heads))
        for h in range(H):
            w = _mix32((i * n_kp + (j >> np.uint32(1))) ^ head_keys[h])
            half = np.where((j & np.uint32(1)) != 0, w >> np.uint32(16), w & np.uint32(0xFFFF))
            out[h] = np.where(half >= thr, scale, np.float32(0.0))
    return out


def full_attention(q, k, v, scale=None, attn_bias=None, mask=None, pruning_mask=None,
                   dropout_mult=None):
    """CoreAttention.full_attention (graphormer_dist_node_level.py:42-65).

    q: [1, N_q, H, d]; k, v: [1, N_k, H, d].  Returns (x [1, N_q, H, d],
    node_scores [N_k]).  Note the reference MULTIPLIES q by sqrt(d).
    ``dropout_mult`` ([H, N_q, N_k], from dropout_multiplier) stands for
    self.att_dropout in training mode; None is eval mode / p = 0.
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
    if dropout_mult is not None:
        x = x * torch.as_tensor(dropout_mult, dtype=x.dtype).unsqueeze(0)
    x = x.matmul(v)
    x = x.transpose(1, 2).contiguous()
    node_scores = torch.abs(score).mean(dim=1).squeeze(0).sum(dim=0)
    return x, node_scores


def naive_attention(q, k, v, dropout_mult=None):
    """CoreAttention.naive_attention (graphormer_dist_node_level.py:100-105),
    the "flash" branch, on [b, N, H, d] inputs: softmax(q k^T / sqrt(d)),
    dropout (always applied there), times v.  Returns x [b, N_q, H, d]."""
    d = q.shape[-1]
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    s = torch.matmul(qt, kt.transpose(-2, -1)) / (d ** 0.5)
    p = torch.softmax(s, dim=-1)
    if dropout_mult is not None:
        p = p * torch.as_tensor(dropout_mult, dtype=p.dtype).unsqueeze(0)
    return torch.matmul(p, vt).transpose(1, 2).contiguous()


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


def full_attention_fp64(q, k, v, scale=None, dropout_mult=None):
    """softmax((q*scale) k^T) [o dropout_mult] v per head in float64; also
    returns sum_i mean_h |S|."""
    q = q.reshape(q.shape[-3], q.shape[-2], q.shape[-1]).double()
    k = k.reshape(k.shape[-3], k.shape[-2], k.shape[-1]).double()
    v = v.reshape(v.shape[-3], v.shape[-2], v.shape[-1]).double()
    if scale is None:
        scale = math.sqrt(q.shape[-1])
    s = torch.einsum("ihc,jhc->hij", q * scale, k)
    p = torch.softmax(s, dim=-1)
    if dropout_mult is not None:
        p = p * torch.as_tensor(dropout_mult, dtype=torch.float64)
    x = torch.einsum("hij,jhc->ihc", p, v)
    ns = s.abs().mean(0).sum(0)
    return x, ns


# --------------------------------------------------------- autograd wrappers
def sparse_fwd_bwd(q, k, v, edge_index, grad_x, num_heads, dtype=torch.float32, attn_bias=None):
    """Runs the restatement forward + autograd backward on CPU in ``dtype``.

    q [N_q,H,d], k/v [N_k,H,d] (any float dtype; cast to ``dtype``), grad_x
    [N_q,H,d].  Returns dict(x [N_q,H,d], node_scores, dq, dk, dv).  With
    ``attn_bias`` [H, N_k, N_q] (indexed [h, src, dst]) the reference's square
    [1, H, N, N] bias is that block zero-padded, and the dict also holds
    dbias [H, N_k, N_q].
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
    ab = None
    if attn_bias is not None:
        ab = torch.zeros(1, num_heads, n, n, dtype=dtype)
        ab[0, :, :n_k, :n_q] = attn_bias.to(dtype)
        ab.requires_grad_(True)
    x, ns = sparse_attention_bias(qf.unsqueeze(0), kf.unsqueeze(0), vf.unsqueeze(0), edge_index,
                                  num_heads, attn_bias=ab)
    g = torch.zeros_like(x)
    g[:n_q] = grad_x.to(dtype)
    x.backward(g)
    res = {
        "x": x.detach()[:n_q],
        "node_scores": ns.detach(),
        "dq": qf.grad[:n_q],
        "dk": kf.grad[:n_k],
        "dv": vf.grad[:n_k],
    }
    if ab is not None:
        res["dbias"] = ab.grad[0, :, :n_k, :n_q]
    return res


def full_fwd_bwd(q, k, v, grad_x, dtype=torch.float32, dropout_mult=None, flash=False,
                 attn_bias=None, pruning_mask=None, mask=None, flash_half=False):
    """full_attention (or, flash=True, naive_attention) forward + autograd
    backward on CPU; q [N_q,H,d], k/v [N_k,H,d].  attn_bias / pruning_mask
    ([1, H, N_q, N_k] or broadcastable) get their gradients in the dict as
    "dbias" / "dpruning"; mask is a bool [N_q, N_k].  flash_half=True runs
    the flash branch as the reference's forward does (graphormer_dist_node_
    level.py:111-122): q, k, v cast to fp16, naive_attention in fp16, the
    result cast back to ``dtype``."""
    qf = q.to(dtype).clone().unsqueeze(0).requires_grad_(True)
    kf = k.to(dtype).clone().unsqueeze(0).requires_grad_(True)
    vf = v.to(dtype).clone().unsqueeze(0).requires_grad_(True)
    ab = attn_bias.to(dtype).clone().requires_grad_(True) if attn_bias is not None else None
    pm = pruning_mask.to(dtype).clone().requires_grad_(True) if pruning_mask is not None else None
    if flash and flash_half:
        x = naive_attention(qf.half(), kf.half(), vf.half(), dropout_mult=dropout_mult).to(dtype)
        ns = torch.empty(0)
    elif flash:
        x, ns = naive_attention(qf, kf, vf, dropout_mult=dropout_mult), torch.empty(0)
    else:
        x, ns = full_attention(qf, kf, vf, attn_bias=ab, pruning_mask=pm, mask=mask,
                               dropout_mult=dropout_mult)
    x.backward(grad_x.to(dtype).unsqueeze(0))
    res = {
        "x": x.detach()[0],
        "node_scores": ns.detach(),
        "dq": qf.grad[0],
        "dk": kf.grad[0],
        "dv": vf.grad[0],
    }
    if ab is not None:
        res["dbias"] = ab.grad
    if pm is not None:
        res["dpruning"] = pm.grad
    return res
