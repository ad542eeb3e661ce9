"""nn.Linear with a split-K weight gradient and a HIP bias gradient under
bf16 autocast.

The encoder's projections (NeutronGT/models/graphormer_dist_node_level.py:
130-206, the GT twin's :230-302) multiply [32,768 x 768] activations by
768 x 768 weights.  Their weight gradient dW = dY^T X has a 768 x 768 output
and a 32,768-long reduction, and autocast's single GEMM for it ran at 190 us
(few output tiles, no split of the reduction).  ``WgradLinear`` keeps
nn.Linear's parameters, names and forward (the same bf16 GEMM autocast runs)
and in the backward computes
  dX = dY W                          (torch GEMM, bf16, as autocast does),
  dW = sum_c dY_c^T X_c              (one batched library GEMM over 16 row
                                      chunks with fp32 output, then a sum in
                                      chunk order, ngt_chunk_sum_f32),
  db = column sums of dY             (ngt_colsum_bf16, fp32, fixed order).
dW and db are fp32 (autocast's own backward rounds dW to bf16 first).
Outside bf16 autocast or without gradients it is a plain nn.Linear.  Any
widths: the node encoder (100 -> 768) and a 47-class readout take the same
path (autocast's GEMM for the readout's dW ran at 111 us and torch's column
sum for its db at 150 us).  ``project(x, lin_q, lin_k, lin_v)``
runs several such layers on one input as one autograd node whose backward
sums dX inside the GEMMs.
"""
from __future__ import annotations

import ctypes as C

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib

_CHUNK = 2048      # rows per split of the weight-gradient reduction
_MAX_SPLITS = 16   # 16 x 2048 rows measured fastest for 32,768 x 768 x 768


def colsum_bf16(dy: torch.Tensor) -> torch.Tensor:
    """fp32 column sums of a bf16 [K, n] GPU matrix (fixed summation order)."""
    lib = _lib.load()
    if dy.dtype != torch.bfloat16 or not dy.is_cuda or dy.dim() != 2:
        raise TypeError("colsum_bf16 takes a 2-D bf16 GPU tensor")
    if not dy.is_contiguous():
        dy = dy.contiguous()
    K, n = dy.shape
    out = torch.empty(n, dtype=torch.float32, device=dy.device)
    nb = C.c_size_t()
    _lib.check(lib.ngt_colsum_workspace_bytes(K, n, C.byref(nb)))
    ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=dy.device)
    _lib.check(lib.ngt_colsum_bf16(dy.data_ptr(), K, n, out.data_ptr(), ws.data_ptr(), nb.value,
                                   _lib.stream_ptr(dy.device)))
    return out


def chunk_sum(parts: torch.Tensor) -> torch.Tensor:
    """Sum over dim 0 of an fp32 GPU tensor, the slices added in order
    (ngt_chunk_sum_f32)."""
    lib = _lib.load()
    if parts.dtype != torch.float32 or not parts.is_cuda or parts.dim() < 2:
        raise TypeError("chunk_sum takes an fp32 GPU tensor with a leading chunk dimension")
    parts = parts.contiguous()
    out = torch.empty(parts.shape[1:], dtype=torch.float32, device=parts.device)
    _lib.check(lib.ngt_chunk_sum_f32(parts.data_ptr(), parts.shape[0], out.numel(),
                                     out.data_ptr(), _lib.stream_ptr(parts.device)))
    return out


def weight_grad(x: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    """dY^T X in fp32 for bf16 x [K, n_in], dy [K, n_out], split over rows.
    Outputs of 1.5 M elements or more (the stacked Q/K/V gradient, 2,304 x
    768) take at most 8 splits: their GEMM has tiles enough at 8, and the
    chunk sum reads half as much (146 against 154 us with the sum)."""
    K = x.shape[0]
    most = _MAX_SPLITS if dy.shape[1] * x.shape[1] < 1_500_000 else _MAX_SPLITS // 2
    splits = max(1, min(most, K // _CHUNK))
    c = K // splits
    main = splits * c
    with torch.autocast("cuda", enabled=False):
        if splits == 1:
            return torch.mm(dy.t(), x, out_dtype=torch.float32)
        # left operand transposed, right operand contiguous row chunks
        dw = chunk_sum(torch.bmm(dy[:main].view(splits, c, -1).transpose(1, 2),
                                 x[:main].view(splits, c, -1), out_dtype=torch.float32))
        if main < K:
            dw += torch.mm(dy[main:].t(), x[main:], out_dtype=torch.float32)
    return dw


class _WgradLinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        x16 = x.to(torch.bfloat16)
        w16 = weight.to(torch.bfloat16)
        b16 = bias.to(torch.bfloat16) if bias is not None else None
        with torch.autocast("cuda", enabled=False):
            y = F.linear(x16, w16, b16)
        ctx.save_for_backward(x16, w16)
        ctx.has_bias = bias is not None
        return y

    @staticmethod
    def backward(ctx, gy):
        x16, w16 = ctx.saved_tensors
        n_out, n_in = w16.shape
        g2 = gy.to(torch.bfloat16).reshape(-1, n_out).contiguous()
        gx = dw = db = None
        if ctx.needs_input_grad[0]:
            with torch.autocast("cuda", enabled=False):
                gx = (g2 @ w16).view(*x16.shape)
        if ctx.needs_input_grad[1]:
            dw = weight_grad(x16.reshape(-1, n_in).contiguous(), g2)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = colsum_bf16(g2)
        return gx, dw, db


def _joint_rows(gys, n_out: int):
    """The [M, len(gys) * n_out] bf16 matrix whose column blocks are the
    gradients gys, when they are views of one buffer laid out that way (the
    attention core's interleaved dQ/dK/dV); else None."""
    if len(gys) < 2 or any(g is None for g in gys):
        return None
    g0 = gys[0]
    if g0.dtype != torch.bfloat16 or any(g.shape != g0.shape or g.dtype != g0.dtype for g in gys):
        return None
    width = n_out * len(gys)
    try:
        rows = [g.view(-1, n_out) for g in gys]
    except RuntimeError:
        return None
    es = g0.element_size()
    base = g0.untyped_storage().data_ptr()
    for i, r in enumerate(rows):
        if (r.stride() != (width, 1) or r.data_ptr() != g0.data_ptr() + i * n_out * es
                or r.untyped_storage().data_ptr() != base):
            return None
    m = rows[0].shape[0]
    if (g0.storage_offset() + m * width) * es > g0.untyped_storage().nbytes():
        return None
    return torch.as_strided(g0, (m, width), (width, 1))


class _ProjectionGroupFn(torch.autograd.Function):
    """Several projections of one input, y_i = x W_i^T + b_i, as one node.

    Forward: one GEMM per projection, as ``_WgradLinearFn``.  Backward: when
    the output gradients are column blocks of one [M, k * n_out] matrix (the
    attention core's interleaved dQ/dK/dV), one GEMM each for dX (against the
    stacked weights), dW (split-K, fp32) and db (one column sum).  Otherwise
    dX is accumulated by the GEMMs themselves (dX = dY_0 W_0, then dX +=
    dY_i W_i with the library's beta = 1), where separate nodes would leave
    autograd to add their bf16 dX tensors with elementwise kernels (two extra
    passes over a [32,768 x 768] tensor for Q/K/V); dW and db per projection
    as ``_WgradLinearFn``."""

    @staticmethod
    def forward(ctx, x, *params):
        x16 = x.to(torch.bfloat16)
        n = len(params) // 2
        ws = [params[2 * i].to(torch.bfloat16) for i in range(n)]
        bs = [params[2 * i + 1] for i in range(n)]
        ys = []
        with torch.autocast("cuda", enabled=False):
            for w16, b in zip(ws, bs):
                ys.append(F.linear(x16, w16, b.to(torch.bfloat16) if b is not None else None))
        ctx.save_for_backward(x16, *ws)
        ctx.has_bias = [b is not None for b in bs]
        ctx.set_materialize_grads(False)  # an unused output: no GEMMs, no weight gradient
        return tuple(ys)

    @staticmethod
    def backward(ctx, *gys):
        x16, *ws = ctx.saved_tensors
        n_in = x16.shape[-1]
        n_out = ws[0].shape[0]
        joint = None
        if (all(w.shape[0] == n_out for w in ws) and all(ctx.needs_input_grad[1::2])
                and (all(ctx.has_bias) and all(ctx.needs_input_grad[2::2])
                     or not any(ctx.has_bias))):
            joint = _joint_rows(gys, n_out)
        if joint is not None:
            gx = None
            if ctx.needs_input_grad[0]:
                with torch.autocast("cuda", enabled=False):
                    gx = (joint @ torch.cat(ws, 0)).view(*x16.shape)
            dw = weight_grad(x16.reshape(-1, n_in).contiguous(), joint)
            db = colsum_bf16(joint) if ctx.has_bias[0] else None
            grads = []
            for i in range(len(ws)):
                grads += [dw[i * n_out:(i + 1) * n_out],
                          db[i * n_out:(i + 1) * n_out] if db is not None else None]
            return (gx, *grads)
        x2 = None
        gx = None
        grads = []
        for i, (gy, w16) in enumerate(zip(gys, ws)):
            if gy is None:
                grads += [None, None]
                continue
            g2 = gy.to(torch.bfloat16).reshape(-1, w16.shape[0]).contiguous()
            if ctx.needs_input_grad[0]:
                with torch.autocast("cuda", enabled=False):
                    if gx is None:
                        gx = g2 @ w16
                    else:
                        gx.addmm_(g2, w16)
            dw = db = None
            if ctx.needs_input_grad[1 + 2 * i]:
                if x2 is None:
                    x2 = x16.reshape(-1, n_in).contiguous()
                dw = weight_grad(x2, g2)
            if ctx.has_bias[i] and ctx.needs_input_grad[2 + 2 * i]:
                db = colsum_bf16(g2)
            grads += [dw, db]
        if gx is not None:
            gx = gx.view(*x16.shape)
        return (gx, *grads)


def _fast_path(lin: nn.Linear, x: torch.Tensor) -> bool:
    return (x.is_cuda and torch.is_grad_enabled() and lin.weight.requires_grad
            and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.bfloat16)


def groupable(x: torch.Tensor, *lins: nn.Linear) -> bool:
    """Whether project(x, *lins) runs them as one node."""
    return len(lins) > 1 and all(isinstance(l, WgradLinear) and _fast_path(l, x) for l in lins)


def project(x: torch.Tensor, *lins: nn.Linear):
    """(lin(x) for lin in lins), with the backward's dX summed inside the
    GEMMs (and, for gradients that arrive as column blocks of one matrix, dW
    and db as one GEMM and one column sum) when all of them take the bf16
    autocast path; otherwise each module's own forward."""
    if groupable(x, *lins):
        params = []
        for l in lins:
            params += [l.weight, l.bias]
        return _ProjectionGroupFn.apply(x, *params)
    return tuple(l(x) for l in lins)


class WgradLinear(nn.Linear):
    """nn.Linear (same parameters and state-dict names) with the split-K
    weight gradient and the HIP bias gradient under bf16 autocast."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _fast_path(self, x):
            return _WgradLinearFn.apply(x, self.weight, self.bias)
        return super().forward(x)
