"""nn.LayerNorm on the library's fused kernels under bf16 autocast.

The encoder's LayerNorms (graphormer_dist_node_level.py:176-206 pre-LN
``self_attention_norm`` / ``ffn_norm`` and ``final_ln``; the GT twin's post-LN
``layer_norm1/2``, gt_dist_node_level_single_window.py:305-353).  Under bf16
autocast torch computes each as: cast the bf16 input to fp32, LayerNorm in
fp32 (fp32 output), and, where a linear layer consumes it, a cast back to
bf16; the backward takes three more kernels.  ``FusedLayerNorm`` keeps
nn.LayerNorm's parameters and state-dict names and runs ``ngt_layernorm_fwd``
/ ``ngt_layernorm_bwd``: one wave per row, fp32 math on the fp32 or bf16
input, the output written in fp32 (autocast's type) or, with
``out_bf16=True`` for a norm whose only consumers are bf16 linear layers,
directly in bf16 (the rounding the consumer's cast would apply).  dgamma and
dbeta are fp32 column sums added in a fixed order.  Outside bf16 autocast or
for unsupported shapes it is a plain nn.LayerNorm.
"""
from __future__ import annotations

import ctypes as C

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .attention import draw_seed

_CODES = {torch.float32: _lib.NGT_F32, torch.bfloat16: _lib.NGT_BF16}


def _rows(t: torch.Tensor, n_cols: int) -> torch.Tensor:
    """[n, n_cols] contiguous view (or copy) whose base meets the kernels'
    alignment: 16 bytes for fp32 rows, 8 for bf16 (4 elements per access)."""
    t = t.reshape(-1, n_cols)
    if not t.is_contiguous() or t.data_ptr() % (16 if t.dtype == torch.float32 else 8):
        t = t.clone(memory_format=torch.contiguous_format)
    return t


class _LayerNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, eps, out_bf16):
        lib = _lib.load()
        n_cols = weight.numel()
        x2 = _rows(x, n_cols)
        n = x2.shape[0]
        dev = x.device
        y = torch.empty(n, n_cols, device=dev,
                        dtype=torch.bfloat16 if out_bf16 else torch.float32)
        mean = torch.empty(n, device=dev, dtype=torch.float32)
        rstd = torch.empty(n, device=dev, dtype=torch.float32)
        w = weight.detach().float().contiguous()
        b = bias.detach().float().contiguous()
        _lib.check(lib.ngt_layernorm_fwd(_CODES[x2.dtype], x2.data_ptr(), n, n_cols, w.data_ptr(),
                                         b.data_ptr(), float(eps), _CODES[y.dtype], y.data_ptr(),
                                         mean.data_ptr(), rstd.data_ptr(),
                                         _lib.stream_ptr(dev)))
        ctx.save_for_backward(x2, w, mean, rstd)
        ctx.in_shape = x.shape
        return y.view(*x.shape)

    @staticmethod
    def backward(ctx, gy):
        x2, w, mean, rstd = ctx.saved_tensors
        lib = _lib.load()
        n, n_cols = x2.shape
        dev = x2.device
        if gy.dtype not in _CODES:
            gy = gy.float()
        g2 = _rows(gy, n_cols)
        dx = torch.empty_like(x2)
        dw = torch.empty(n_cols, device=dev, dtype=torch.float32)
        db = torch.empty(n_cols, device=dev, dtype=torch.float32)
        nb = C.c_size_t()
        _lib.check(lib.ngt_layernorm_bwd_workspace_bytes(n, n_cols, C.byref(nb)))
        ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=dev)
        _lib.check(lib.ngt_layernorm_bwd(_CODES[x2.dtype], x2.data_ptr(), _CODES[g2.dtype],
                                         g2.data_ptr(), n, n_cols, w.data_ptr(),
                                         mean.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
                                         dw.data_ptr(), db.data_ptr(), ws.data_ptr(), nb.value,
                                         _lib.stream_ptr(dev)))
        return dx.view(*ctx.in_shape), dw, db, None, None


class FusedLayerNorm(nn.LayerNorm):
    """nn.LayerNorm (same parameters and names) on the fused kernels under
    bf16 autocast; ``out_bf16`` writes the output in bf16 for bf16 consumers."""

    def __init__(self, normalized_shape, eps: float = 1e-5, out_bf16: bool = False, **kw):
        super().__init__(normalized_shape, eps=eps, **kw)
        self.out_bf16 = bool(out_bf16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n_cols = self.normalized_shape[-1]
        if (x.is_cuda and len(self.normalized_shape) == 1 and self.elementwise_affine
                and self.bias is not None and x.dtype in _CODES
                and torch.is_autocast_enabled("cuda")
                and torch.get_autocast_dtype("cuda") == torch.bfloat16
                and n_cols % 4 == 0 and 4 <= n_cols <= 2048):
            return _LayerNormFn.apply(x, self.weight, self.bias, self.eps, self.out_bf16)
        return super().forward(x)


def _fused_ok(x: torch.Tensor, ln: nn.LayerNorm) -> bool:
    n_cols = ln.normalized_shape[-1]
    return (isinstance(ln, FusedLayerNorm) and x.is_cuda and len(ln.normalized_shape) == 1
            and ln.elementwise_affine and ln.bias is not None and x.dtype in _CODES
            and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.bfloat16
            and n_cols % 4 == 0 and 4 <= n_cols <= 2048)


class _AddLayerNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, weight, bias, eps, p, seed, out_bf16, seed_t=None):
        lib = _lib.load()
        n_cols = weight.numel()
        x2, y2 = _rows(x, n_cols), _rows(y, n_cols)
        n = x2.shape[0]
        dev = x.device
        s = torch.empty_like(x2)
        out = torch.empty(n, n_cols, device=dev,
                          dtype=torch.bfloat16 if out_bf16 else torch.float32)
        mean = torch.empty(n, device=dev, dtype=torch.float32)
        rstd = torch.empty(n, device=dev, dtype=torch.float32)
        w = weight.detach().float().contiguous()
        b = bias.detach().float().contiguous()
        _lib.check(lib.ngt_add_layernorm_fwd(
            _CODES[x2.dtype], x2.data_ptr(), y2.data_ptr(), n, n_cols, float(p), int(seed),
            seed_t.data_ptr() if seed_t is not None else None, w.data_ptr(), b.data_ptr(),
            float(eps), s.data_ptr(), _CODES[out.dtype], out.data_ptr(), mean.data_ptr(),
            rstd.data_ptr(), _lib.stream_ptr(dev)))
        if seed_t is not None:
            ctx.save_for_backward(s, w, mean, rstd, seed_t)
        else:
            ctx.save_for_backward(s, w, mean, rstd)
        ctx.p, ctx.seed, ctx.shape = float(p), int(seed), x.shape
        return s.view(*x.shape), out.view(*x.shape)

    @staticmethod
    def backward(ctx, g_s, g_out):
        s, w, mean, rstd = ctx.saved_tensors[:4]
        seed_t = ctx.saved_tensors[4] if len(ctx.saved_tensors) == 5 else None
        lib = _lib.load()
        n, n_cols = s.shape
        dev = s.device
        if g_out is None:
            g_out = torch.zeros(n, n_cols, device=dev, dtype=torch.float32)
        g_out2 = _rows(g_out if g_out.dtype in _CODES else g_out.float(), n_cols)
        g_s2 = _rows(g_s.to(s.dtype), n_cols) if g_s is not None else None
        dx = torch.empty_like(s)
        dy = torch.empty_like(s)
        dw = torch.empty(n_cols, device=dev, dtype=torch.float32)
        db = torch.empty(n_cols, device=dev, dtype=torch.float32)
        nb = C.c_size_t()
        _lib.check(lib.ngt_layernorm_bwd_workspace_bytes(n, n_cols, C.byref(nb)))
        ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=dev)
        _lib.check(lib.ngt_add_layernorm_bwd(
            _CODES[s.dtype], s.data_ptr(), _CODES[g_out2.dtype], g_out2.data_ptr(),
            g_s2.data_ptr() if g_s2 is not None else None, n, n_cols, ctx.p, ctx.seed,
            seed_t.data_ptr() if seed_t is not None else None, w.data_ptr(), mean.data_ptr(),
            rstd.data_ptr(), dx.data_ptr(), dy.data_ptr(),
            dw.data_ptr(), db.data_ptr(), ws.data_ptr(), nb.value,
            _lib.stream_ptr(dev)))
        return dx.view(*ctx.shape), dy.view(*ctx.shape), dw, db, None, None, None, None, None


def add_dropout_layernorm(x: torch.Tensor, y: torch.Tensor, ln: nn.LayerNorm,
                          dropout: nn.Dropout):
    """(s, ln(s)) with s = x + dropout(y): the residual add and the LayerNorm
    that follows it, as one pass of ``ngt_add_layernorm_fwd`` under bf16
    autocast (the dropout mask then comes from this library's hash, with a
    seed drawn on the device from torch's generator, so that every replay of a
    captured graph draws a new mask); otherwise the unfused torch ops."""
    p = dropout.p if dropout.training else 0.0
    if (_fused_ok(x, ln) and y.dtype == x.dtype and y.shape == x.shape and p < 1.0
            and torch.is_grad_enabled()):
        seed_t = draw_seed(x.device) if p > 0 else None
        return _AddLayerNormFn.apply(x, y, ln.weight, ln.bias, ln.eps, p, 0, ln.out_bf16, seed_t)
    s = x + F.dropout(y, p, dropout.training) if p > 0 else x + y
    return s, ln(s)
