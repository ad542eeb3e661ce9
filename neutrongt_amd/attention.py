"""Drop-in replacement of NeutronGT's attention core backed by HIP kernels.

``CoreAttention`` keeps the reference class's constructor, attributes and
methods (NeutronGT/models/graphormer_dist_node_level.py:33-127; twin
NeutronGT/models/gt_dist_node_level_single_window.py:30-227) so it can be
installed as ``MultiHeadAttention.local_attn`` (graphormer_dist_node_level.py:138,
call at :170; gt_dist_node_level_single_window.py:243-244, call at :292) or as
``DistributedAttentionNodeLevel.local_attn`` (NeutronGT/gt_sp/gt_layer.py:276-286).

Every compute call goes through libngt_attn.so; there is no PyTorch/CPU
fallback (CPU tensors raise).
"""
from __future__ import annotations

import ctypes as C
import math

import torch
import torch.nn as nn

from . import _lib
from .csr import AdjacencyCache, chunk_for_heads, default_cache, pack_q_adaptive, small_for_heads

CLAMP_LO = -5.0
CLAMP_HI = 5.0
EPS = 1e-6

_DTYPES = {torch.float32: _lib.NGT_F32, torch.bfloat16: _lib.NGT_BF16}


def _dtype_code(t: torch.Tensor) -> int:
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {t.dtype} (float32 or bfloat16)")
    return code


def _prep(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the attention core has no CPU path)")
    if not t.is_contiguous() or t.data_ptr() % 16:
        t = t.contiguous() if not t.is_contiguous() else t.clone()
    return t


def _stream(dev) -> int:
    return _lib.stream_ptr(dev)


def _workspace(nbytes: int, dev) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


# ------------------------------------------------------------------- sparse
class SparseAttentionFunction(torch.autograd.Function):
    """out, node_score = masked attention over a WindowAdjacency.

    q [N_q, H, d], k/v [N_k, H, d] (same dtype, fp32 or bf16).  node_score is
    returned without gradient (the reference's caller detaches it,
    graphormer_dist_node_level.py:345).  Optional k_ext/v_ext [R, H, d] are
    further key rows N_k .. N_k+R-1 read from their own buffers (a detached
    cache of related keys, so the caller need not concatenate); they receive
    no gradient.  ``interleave_grads`` (with N_q == N_k): dQ, dK and dV come
    back as views of one [N, 3, H, d] buffer (ngt_sparse_bwd_strided), which a
    caller of three projections of one input can multiply as one matrix.
    """

    @staticmethod
    def forward(ctx, q, k, v, adj, scale, lo, hi, eps, k_ext=None, v_ext=None,
                interleave_grads=False):
        lib = _lib.load()
        n_q, H, d = q.shape
        dev = q.device
        out = torch.empty_like(q)
        rinv = torch.empty(n_q, H, dtype=torch.float32, device=dev)
        ns = torch.empty(adj.dst_end, dtype=torch.float32, device=dev)
        fwd_bytes, bwd_bytes = adj.workspace_bytes(H, d)
        ws = _workspace(fwd_bytes, dev)
        ext = k_ext is not None
        _lib.check(lib.ngt_sparse_fwd_ext(
            _dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            k_ext.data_ptr() if ext else None, v_ext.data_ptr() if ext else None, k.shape[0],
            adj.ptr(), H, d, scale, lo, hi, eps, out.data_ptr(), rinv.data_ptr(),
            ns.data_ptr() if ns.numel() else None, int(ns.numel()), ws.data_ptr(), fwd_bytes,
            _stream(dev)))
        if ext:
            ctx.save_for_backward(q, k, v, out, rinv, k_ext, v_ext)
        else:
            ctx.save_for_backward(q, k, v, out, rinv)
        ctx.adj, ctx.scale, ctx.lo, ctx.hi, ctx.bwd_bytes = adj, scale, lo, hi, bwd_bytes
        ctx.interleave = bool(interleave_grads) and q.shape[0] == k.shape[0]
        ctx.mark_non_differentiable(ns)
        # the node scores have no gradient: let the engine pass None for them
        # instead of filling a zero tensor (a kernel launch per layer)
        ctx.set_materialize_grads(False)
        return out, ns

    @staticmethod
    def backward(ctx, g_out, g_ns):
        saved = ctx.saved_tensors
        q, k, v, out, rinv = saved[:5]
        k_ext, v_ext = saved[5:] if len(saved) == 7 else (None, None)
        if g_out is None:  # the output was not used by the loss
            return (None,) * 11
        lib = _lib.load()
        n_q, H, d = q.shape
        dev = q.device
        g = g_out.to(q.dtype)
        if not g.is_contiguous() or g.data_ptr() % 16:
            g = g.contiguous() if not g.is_contiguous() else g.clone()
        if ctx.interleave:  # one [N, 3, H, d] buffer: dQ, dK, dV of a row side by side
            buf = torch.empty(n_q, 3, H, d, dtype=q.dtype, device=dev)
            gq, gk, gv = buf.unbind(1)
            ldg = 3 * H * d
        else:
            gq = torch.empty_like(q)
            gk = torch.empty_like(k)
            gv = torch.empty_like(v)
            ldg = 0
        ws = _workspace(ctx.bwd_bytes, dev)
        ext = k_ext is not None
        _lib.check(lib.ngt_sparse_bwd_strided(
            _dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            k_ext.data_ptr() if ext else None, v_ext.data_ptr() if ext else None, k.shape[0],
            out.data_ptr(), g.data_ptr(), rinv.data_ptr(), ctx.adj.ptr(), H, d, ctx.scale, ctx.lo,
            ctx.hi, gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), ldg, ws.data_ptr(),
            ctx.bwd_bytes, _stream(dev)))
        return gq, gk, gv, None, None, None, None, None, None, None, None


class SparseAttentionBiasFunction(torch.autograd.Function):
    """SparseAttentionFunction with the reference's optional per-pair bias
    (attn_bias, graphormer_dist_node_level.py:81-84): ``bias`` [H, Ns, Nd]
    fp32 on the GPU, any strides, indexed [h, src, dst] (Ns >= N_k, Nd >= N_q),
    added to each edge's clamped score: p_e = exp(clamp(a_e) + bias[h, j, i]).
    The bias gets a gradient when it requires one: the score gradient of each
    edge (no clamp mask), summed over duplicate edges in a fixed order."""

    @staticmethod
    def forward(ctx, q, k, v, bias, adj, scale, lo, hi, eps, k_ext=None, v_ext=None):
        lib = _lib.load()
        n_q, H, d = q.shape
        dev = q.device
        if (bias.dim() != 3 or bias.dtype != torch.float32 or not bias.is_cuda
                or bias.shape[0] != H or bias.shape[1] < adj.n_k or bias.shape[2] < adj.n_q):
            raise ValueError(f"bias must be an fp32 GPU tensor [{H}, >= {adj.n_k}, >= {adj.n_q}] "
                             f"(indexed [h, src, dst]), got {tuple(bias.shape)} {bias.dtype}")
        st = _stream(dev)
        E = adj.n_edges
        eb_q = torch.empty(max(E, 1), H, dtype=torch.float32, device=dev)
        eb_t = torch.empty(max(E, 1), H, dtype=torch.float32, device=dev)
        _lib.check(lib.ngt_edge_bias_gather(adj.ptr(), H, bias.data_ptr(), *bias.stride(),
                                            eb_q.data_ptr(), eb_t.data_ptr(), st))
        out = torch.empty_like(q)
        rinv = torch.empty(n_q, H, dtype=torch.float32, device=dev)
        ns = torch.empty(adj.dst_end, dtype=torch.float32, device=dev)
        fwd_bytes, bwd_bytes = adj.workspace_bytes(H, d)
        ws = _workspace(fwd_bytes, dev)
        ext = k_ext is not None
        _lib.check(lib.ngt_sparse_fwd_bias(
            _dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            k_ext.data_ptr() if ext else None, v_ext.data_ptr() if ext else None, k.shape[0],
            adj.ptr(), H, d, scale, lo, hi, eps, eb_q.data_ptr(), out.data_ptr(),
            rinv.data_ptr(), ns.data_ptr() if ns.numel() else None, int(ns.numel()),
            ws.data_ptr(), fwd_bytes, st))
        saved = [q, k, v, out, rinv, eb_t] + ([k_ext, v_ext] if ext else [])
        ctx.save_for_backward(*saved)
        ctx.adj, ctx.scale, ctx.lo, ctx.hi, ctx.bwd_bytes = adj, scale, lo, hi, bwd_bytes
        ctx.bias_shape = tuple(bias.shape)
        ctx.mark_non_differentiable(ns)
        ctx.set_materialize_grads(False)
        return out, ns

    @staticmethod
    def backward(ctx, g_out, g_ns):
        saved = ctx.saved_tensors
        q, k, v, out, rinv, eb_t = saved[:6]
        k_ext, v_ext = saved[6:] if len(saved) == 8 else (None, None)
        if g_out is None:
            return (None,) * 11
        lib = _lib.load()
        n_q, H, d = q.shape
        dev = q.device
        st = _stream(dev)
        g = g_out.to(q.dtype)
        if not g.is_contiguous() or g.data_ptr() % 16:
            g = g.contiguous() if not g.is_contiguous() else g.clone()
        gq = torch.empty_like(q)
        gk = torch.empty_like(k)
        gv = torch.empty_like(v)
        want_bias = ctx.needs_input_grad[3]
        deb = torch.empty_like(eb_t) if want_bias else None
        ws = _workspace(ctx.bwd_bytes, dev)
        ext = k_ext is not None
        _lib.check(lib.ngt_sparse_bwd_bias(
            _dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            k_ext.data_ptr() if ext else None, v_ext.data_ptr() if ext else None, k.shape[0],
            out.data_ptr(), g.data_ptr(), rinv.data_ptr(), ctx.adj.ptr(), H, d, ctx.scale,
            ctx.lo, ctx.hi, eb_t.data_ptr(), deb.data_ptr() if want_bias else None,
            gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), ws.data_ptr(), ctx.bwd_bytes, st))
        gb = None
        if want_bias:
            gb = torch.zeros(ctx.bias_shape, dtype=torch.float32, device=dev)
            _lib.check(lib.ngt_edge_bias_grad(ctx.adj.ptr(), H, deb.data_ptr(), gb.data_ptr(),
                                              *gb.stride(), st))
        return gq, gk, gv, gb, None, None, None, None, None, None, None


def window_attention(q, k, v, adj, scale, lo=CLAMP_LO, hi=CLAMP_HI, eps=EPS, k_ext=None,
                     v_ext=None, interleave_grads=False):
    """SparseAttentionFunction's operation over a built WindowAdjacency, run by
    the C++ autograd node (ngt_autograd.so) when it is built -- the same
    library calls without a Python frame or ctypes conversion per layer and
    without the GIL on the autograd engine's device thread -- else by
    SparseAttentionFunction.  q/k/v (and k_ext/v_ext) as that function takes
    them: contiguous, 16-byte aligned, on the GPU.  ``interleave_grads``: see
    SparseAttentionFunction."""
    ext = _lib.autograd_ext()
    if ext is None:
        return SparseAttentionFunction.apply(q, k, v, adj, scale, lo, hi, eps, k_ext, v_ext,
                                             interleave_grads)
    H, d = q.shape[1], q.shape[2]
    fwd_bytes, bwd_bytes = adj.workspace_bytes(H, d)
    return ext.sparse_attention(q, k, v, k_ext, v_ext, adj.csr_bytes, adj.mem, adj.dst_end,
                                float(scale), float(lo), float(hi), float(eps), fwd_bytes,
                                bwd_bytes, bool(interleave_grads))


def sparse_attention(q, k, v, edge_index, num_heads=None, scale=None, cache: AdjacencyCache = None,
                     lo=CLAMP_LO, hi=CLAMP_HI, eps=EPS, kv_ext=None, attn_bias=None,
                     interleave_grads=False):
    """Functional form.  q [.., N_q, H, d] -> (x [N_q, H, d], node_scores [max(dst)+1]).

    ``edge_index`` [2, E]: row 0 = key (src) index < N_k, row 1 = query (dst)
    index < N_q.  The reference requires N_q == N_k; N_q < N_k (extra key rows,
    e.g. related nodes served from the cache) is also accepted.  ``kv_ext``
    = (k_r, v_r), each [R, H, d], supplies key rows N_k .. N_k+R-1 from their
    own buffers without a concatenation; they get no gradient (a detached cache).
    ``attn_bias`` [1, H, Ns, Nd] (the reference's dense per-pair bias, indexed
    [0, h, src, dst], Ns >= N_k and Nd >= N_q) is added to each edge's clamped
    score and receives a gradient when it requires one.  ``interleave_grads``
    (N_q == N_k, no bias): dQ, dK, dV as views of one [N, 3, H, d] buffer.
    """
    H, d = q.shape[-2], q.shape[-1]
    if num_heads is not None and num_heads != H:
        raise ValueError(f"q has {H} heads, expected {num_heads}")
    q = _prep(q.reshape(-1, H, d), "q")
    k = _prep(k.reshape(-1, H, d), "k")
    v = _prep(v.reshape(-1, H, d), "v")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    _dtype_code(q)
    if k.shape != v.shape or k.shape[1:] != q.shape[1:]:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    k_ext = v_ext = None
    n_k = k.shape[0]
    if kv_ext is not None:
        k_ext = _prep(kv_ext[0].detach().reshape(-1, H, d), "k_ext")
        v_ext = _prep(kv_ext[1].detach().reshape(-1, H, d), "v_ext")
        if k_ext.shape != v_ext.shape or k_ext.dtype != q.dtype or v_ext.dtype != q.dtype:
            raise ValueError(f"kv_ext must be two [R, {H}, {d}] tensors of dtype {q.dtype}")
        n_k += k_ext.shape[0]
    if q.shape[0] > n_k:
        raise ValueError(f"N_q={q.shape[0]} exceeds N_k={n_k}")
    if scale is None:
        scale = math.sqrt(d)
    cache = cache or default_cache
    adj = cache.get(edge_index, q.shape[0], n_k, chunk_for_heads(H, int(edge_index.shape[-1])),
                    small_for_heads(H), pack_q_adaptive(H))
    if attn_bias is not None:
        if (attn_bias.dim() != 4 or attn_bias.shape[0] != 1 or attn_bias.shape[1] != H
                or attn_bias.shape[2] < n_k or attn_bias.shape[3] < q.shape[0]):
            raise ValueError(f"attn_bias must be [1, {H}, >= {n_k}, >= {q.shape[0]}] "
                             f"(indexed [0, h, src, dst]), got {tuple(attn_bias.shape)}")
        if not attn_bias.is_cuda:
            raise ValueError("attn_bias must be a GPU tensor")
        bias = attn_bias[0].to(torch.float32)
        return SparseAttentionBiasFunction.apply(q, k, v, bias, adj, float(scale), float(lo),
                                                 float(hi), float(eps), k_ext, v_ext)
    return window_attention(q, k, v, adj, float(scale), float(lo), float(hi), float(eps), k_ext,
                            v_ext, interleave_grads)


# -------------------------------------------------------------------- dense
class DenseAttentionFunction(torch.autograd.Function):
    """out = dropout_p(softmax((q*scale) k^T)) v per head,
    node_score[j] = sum_i mean_h |S|.  With dropout_p > 0 the keep mask is a
    hash of (seed, head, query, key) (the C-ABI's ngt_dense_fwd documents it);
    the backward regenerates it from the same seed.  ``seed_t`` (an int64
    device tensor of one element, or None) supplies the seed from device
    memory instead of the host integer ``seed``."""

    @staticmethod
    def forward(ctx, q, k, v, scale, want_scores, dropout_p=0.0, seed=0, seed_t=None):
        lib = _lib.load()
        n_q, H, d = q.shape
        n_k = k.shape[0]
        dev = q.device
        dt = _dtype_code(q)
        out = torch.empty_like(q)
        # bf16: an fp32 copy of out feeds the backward's D = G . out
        out32 = (torch.empty(n_q, H, d, dtype=torch.float32, device=dev)
                 if q.dtype != torch.float32 else None)
        lse = torch.empty(H, n_q, dtype=torch.float32, device=dev)
        want = bool(want_scores and n_k)
        ns = torch.empty(n_k if want_scores else 0, dtype=torch.float32, device=dev)
        fb, bb = C.c_size_t(), C.c_size_t()
        _lib.check(lib.ngt_dense_workspace_bytes(dt, n_q, n_k, H, d, int(want), C.byref(fb),
                                                 C.byref(bb)))
        ws = _workspace(fb.value, dev) if fb.value else None
        sp = seed_t.data_ptr() if seed_t is not None else None
        _lib.check(lib.ngt_dense_fwd(dt, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                     n_q, n_k, H, d, scale, dropout_p, seed, sp, out.data_ptr(),
                                     out32.data_ptr() if out32 is not None else None,
                                     lse.data_ptr(), ns.data_ptr() if want else None,
                                     ws.data_ptr() if ws is not None else None, fb.value,
                                     _stream(dev)))
        if seed_t is not None:
            ctx.save_for_backward(q, k, v, out if out32 is None else out32, lse, seed_t)
        else:
            ctx.save_for_backward(q, k, v, out if out32 is None else out32, lse)
        ctx.scale, ctx.bwd_bytes, ctx.dropout_p, ctx.seed = scale, bb.value, dropout_p, seed
        ctx.mark_non_differentiable(ns)
        ctx.set_materialize_grads(False)  # no zero tensor for the node scores' gradient
        return out, ns

    @staticmethod
    def backward(ctx, g_out, g_ns):
        saved = ctx.saved_tensors
        q, k, v, out, lse = saved[:5]
        seed_t = saved[5] if len(saved) == 6 else None
        if g_out is None:
            return None, None, None, None, None, None, None, None
        lib = _lib.load()
        n_q, H, d = q.shape
        n_k = k.shape[0]
        dev = q.device
        g = g_out.to(q.dtype)
        if not g.is_contiguous() or g.data_ptr() % 16:
            g = g.contiguous() if not g.is_contiguous() else g.clone()
        gq = torch.empty_like(q)
        gk = torch.empty_like(k)
        gv = torch.empty_like(v)
        ws = _workspace(ctx.bwd_bytes, dev)
        f32_out = out.dtype != q.dtype  # the fp32 copy saved for a bf16 forward
        _lib.check(lib.ngt_dense_bwd(_dtype_code(q), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                     None if f32_out else out.data_ptr(),
                                     out.data_ptr() if f32_out else None, g.data_ptr(),
                                     lse.data_ptr(), n_q, n_k, H, d,
                                     ctx.scale, ctx.dropout_p, ctx.seed,
                                     seed_t.data_ptr() if seed_t is not None else None,
                                     gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), ws.data_ptr(),
                                     ctx.bwd_bytes, _stream(dev)))
        return gq, gk, gv, None, None, None, None, None


# Bytes of [n_q, n_k] fp32 matrices that the materialized dense path may hold
# at once for its head chunks (S, P, P o M, dL/d(P o M) and dS per head); a
# window runs as many heads per chunk as fit, at least one.
DENSE_BIAS_BUDGET_BYTES = 4 << 30
_DENSE_BIAS_MATS_PER_HEAD = 5


def dense_bias_head_chunk(H: int, n_q: int, n_k: int, budget: int = None) -> int:
    """Heads per chunk of the materialized dense path: as many as keep
    5 [n_q, n_k] fp32 matrices per head within ``budget`` bytes (default
    DENSE_BIAS_BUDGET_BYTES) and the softmax launches within 2^24 rows, at
    least one and at most H."""
    budget = DENSE_BIAS_BUDGET_BYTES if budget is None else int(budget)
    per_head = _DENSE_BIAS_MATS_PER_HEAD * 4 * max(n_q, 1) * max(n_k, 1)
    c = max(1, min(H, budget // per_head))
    return max(1, min(c, (1 << 24) // max(n_q, 1)))


def _f32_contig(*ts):
    for t in ts:
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise RuntimeError(f"internal: dense-bias operand is {t.dtype}, contiguous="
                               f"{t.is_contiguous()} (needs contiguous float32)")


class DenseAttentionBiasFunction(torch.autograd.Function):
    """full_attention with the reference's optional terms
    (graphormer_dist_node_level.py:51-58): out = dropout_p(softmax(z)) v with
    z = mask ? -1e9 : (q*scale) k^T + bias per head, node_score[j] =
    sum_i mean_h |(q*scale) k^T|.  ``bias`` [H, N_q, N_k] fp32 (attn_bias +
    pruning_mask, or None), ``mask`` [N_q, N_k] uint8 (nonzero = filled, or
    None).  The products run as library GEMMs in fp32, one head at a time
    (the reference's own materialized form: a dense bias is O(N_q N_k H)
    whatever the kernel); logits, mask, softmax, dropout (the fused kernels'
    hash mask for the same seed), the softmax backward and the node scores
    are the library's ngt_dense_bias_* / ngt_dense_abs_* kernels.  The heads
    run ``head_chunk`` at a time and the backward recomputes S and P per
    chunk, so no [H, N_q, N_k] intermediate is kept; each head's arithmetic
    is the same whatever the chunk, so every chunk size gives the same bits.
    Autocast is off inside (every operand is fp32).  ``bias`` gets dS as its
    gradient (zero where masked)."""

    @staticmethod
    def _chunk_softmax(lib, st, qh, khT, bias, mask, scale, h0, h1, dropout_p, seed, seed_t,
                       lse=None):
        """S, P and P o M (or None) of heads h0 .. h1-1."""
        n_q, n_k = qh.shape[1], khT.shape[2]
        hc = h1 - h0
        s = torch.empty(hc, n_q, n_k, dtype=torch.float32, device=qh.device)
        for h in range(h0, h1):
            torch.mm(qh[h], khT[h], out=s[h - h0])
        p = torch.empty_like(s)
        pd = torch.empty_like(s) if dropout_p > 0.0 else None
        b = bias[h0:h1] if bias is not None else None
        _f32_contig(s, b)
        _lib.check(lib.ngt_dense_bias_softmax_fwd(
            hc, h0, n_q, n_k, s.data_ptr(), scale, b.data_ptr() if b is not None else None,
            mask.data_ptr() if mask is not None else None, dropout_p, seed,
            seed_t.data_ptr() if seed_t is not None else None, p.data_ptr(),
            pd.data_ptr() if pd is not None else None,
            lse[h0:h1].data_ptr() if lse is not None else None, st))
        return s, p, pd

    @staticmethod
    def forward(ctx, q, k, v, bias, mask, scale, want_scores, dropout_p=0.0, seed=0, seed_t=None,
                head_chunk=None):
        with torch.autocast("cuda", enabled=False):
            lib = _lib.load()
            n_q, H, d = q.shape
            n_k = k.shape[0]
            dev = q.device
            st = _stream(dev)
            c = int(head_chunk) if head_chunk else dense_bias_head_chunk(H, n_q, n_k)
            c = max(1, min(c, H))
            qh = q.permute(1, 0, 2).float().contiguous()  # [H, n_q, d]
            kh = k.permute(1, 0, 2).float().contiguous()
            vh = v.permute(1, 0, 2).float().contiguous()
            khT = kh.transpose(1, 2).contiguous()  # [H, d, n_k]
            _f32_contig(qh, kh, vh, khT, bias)
            ns = torch.zeros(n_k if want_scores else 0, dtype=torch.float32, device=dev)
            scores = bool(want_scores and n_k and n_q)
            m = torch.empty(n_q, n_k, dtype=torch.float32, device=dev) if scores else None
            o = torch.empty(H, n_q, d, dtype=torch.float32, device=dev)
            lse = torch.empty(H, n_q, dtype=torch.float32, device=dev)
            for h0 in range(0, H, c):
                h1 = min(H, h0 + c)
                s, p, pd = DenseAttentionBiasFunction._chunk_softmax(
                    lib, st, qh, khT, bias, mask, scale, h0, h1, dropout_p, seed, seed_t, lse)
                if scores:
                    _lib.check(lib.ngt_dense_abs_head_sum(h1 - h0, n_q, n_k, s.data_ptr(), scale,
                                                          int(h0 > 0), m.data_ptr(), st))
                del s
                pm = pd if pd is not None else p
                for h in range(h0, h1):
                    torch.mm(pm[h - h0], vh[h], out=o[h])
                del p, pd, pm
            if scores:
                wb = C.c_size_t()
                _lib.check(lib.ngt_dense_abs_colsum_workspace_bytes(n_k, C.byref(wb)))
                ws = _workspace(wb.value, dev)
                _lib.check(lib.ngt_dense_abs_colsum(H, n_q, n_k, m.data_ptr(), ns.data_ptr(),
                                                    ws.data_ptr(), wb.value, st))
                del m
            out = o.permute(1, 0, 2).to(q.dtype).contiguous()
        ctx.save_for_backward(qh, khT, vh, bias, mask, seed_t)
        ctx.scale, ctx.dropout_p, ctx.seed, ctx.chunk = scale, dropout_p, seed, c
        ctx.dtypes = (q.dtype, k.dtype, v.dtype)
        ctx.mark_non_differentiable(ns)
        ctx.set_materialize_grads(False)
        return out, ns

    @staticmethod
    def backward(ctx, g_out, g_ns):
        qh, khT, vh, bias, mask, seed_t = ctx.saved_tensors
        if g_out is None:
            return (None,) * 11
        with torch.autocast("cuda", enabled=False):
            lib = _lib.load()
            H, n_q, d = qh.shape
            n_k = khT.shape[2]
            dev = qh.device
            st = _stream(dev)
            c = ctx.chunk
            gh = g_out.permute(1, 0, 2).float().contiguous()  # [H, n_q, d]
            _f32_contig(gh)
            dq = torch.empty(H, n_q, d, dtype=torch.float32, device=dev)
            dk = torch.empty(H, n_k, d, dtype=torch.float32, device=dev)
            dv = torch.empty(H, n_k, d, dtype=torch.float32, device=dev)
            want_bias = ctx.needs_input_grad[3]
            dbias = torch.empty(H, n_q, n_k, dtype=torch.float32, device=dev) if want_bias else None
            for h0 in range(0, H, c):
                h1 = min(H, h0 + c)
                # S and P again, with the forward's calls (the same bits)
                s, p, pd = DenseAttentionBiasFunction._chunk_softmax(
                    lib, st, qh, khT, bias, mask, ctx.scale, h0, h1, ctx.dropout_p, ctx.seed,
                    seed_t)
                del s
                pm = pd if pd is not None else p
                dpd = torch.empty(h1 - h0, n_q, n_k, dtype=torch.float32, device=dev)
                for h in range(h0, h1):
                    torch.mm(gh[h], vh[h].t(), out=dpd[h - h0])
                    torch.mm(pm[h - h0].t(), gh[h], out=dv[h])
                del pd, pm
                ds = dbias[h0:h1] if want_bias else torch.empty_like(dpd)
                _f32_contig(p, dpd, ds)
                _lib.check(lib.ngt_dense_bias_softmax_bwd(
                    h1 - h0, h0, n_q, n_k, p.data_ptr(), dpd.data_ptr(),
                    mask.data_ptr() if mask is not None else None, ctx.dropout_p, ctx.seed,
                    seed_t.data_ptr() if seed_t is not None else None, ds.data_ptr(), st))
                del p, dpd
                for h in range(h0, h1):
                    torch.mm(ds[h - h0], khT[h].t(), out=dq[h])
                    torch.mm(ds[h - h0].t(), qh[h], out=dk[h])
                del ds
            dq.mul_(ctx.scale)
            dk.mul_(ctx.scale)
            tq, tk, tv = ctx.dtypes
            return (dq.permute(1, 0, 2).to(tq), dk.permute(1, 0, 2).to(tk),
                    dv.permute(1, 0, 2).to(tv), dbias, None, None, None, None, None, None, None)


def dense_attention_bias(q, k, v, scale, attn_bias=None, pruning_mask=None, mask=None,
                         node_scores=True, dropout_p=0.0, seed=None, head_chunk=None):
    """full_attention with attn_bias / pruning_mask / mask as the reference
    applies them (graphormer_dist_node_level.py:51-58): q [1, N_q, H, d],
    k/v [1, N_k, H, d]; attn_bias and pruning_mask broadcast to
    [1, H, N_q, N_k] and added after the scaling; mask (bool, [N_q, N_k])
    fills with -1e9.  Returns (x [N_q, H, d], node_scores [N_k]).
    ``head_chunk``: heads per chunk (default: dense_bias_head_chunk, from
    DENSE_BIAS_BUDGET_BYTES); the result does not depend on it."""
    H, d = q.shape[-2], q.shape[-1]
    q = _prep(q.reshape(-1, H, d), "q")
    k = _prep(k.reshape(-1, H, d), "k")
    v = _prep(v.reshape(-1, H, d), "v")
    n_q, n_k = q.shape[0], k.shape[0]
    bias = None
    if attn_bias is not None or pruning_mask is not None:
        for t in (attn_bias, pruning_mask):
            try:
                ok = t is None or torch.broadcast_shapes(t.shape, (1, H, n_q, n_k)) == (1, H, n_q, n_k)
            except RuntimeError:
                ok = False
            if not ok:
                raise ValueError(f"attn_bias/pruning_mask must broadcast to [1, {H}, {n_q}, {n_k}], "
                                 f"got {tuple(t.shape)}")
        bias = torch.zeros(1, H, n_q, n_k, dtype=torch.float32, device=q.device)
        for t in (attn_bias, pruning_mask):
            if t is not None:
                bias = bias + t.to(device=q.device, dtype=torch.float32)
        bias = bias[0]
        if not bias.is_contiguous():
            bias = bias.contiguous()
    mk = None
    if mask is not None:
        mk = mask.to(device=q.device).expand(n_q, n_k).to(torch.uint8).contiguous()
    dropout_p = float(dropout_p)
    if not 0.0 <= dropout_p <= 1.0:
        raise ValueError(f"dropout probability has to be between 0 and 1, but got {dropout_p}")
    seed_t = None
    if dropout_p > 0.0 and seed is None:
        seed_t = draw_seed(q.device)
    elif isinstance(seed, torch.Tensor):
        seed_t, seed = seed, None
    return DenseAttentionBiasFunction.apply(q, k, v, bias, mk, float(scale), bool(node_scores),
                                            dropout_p, int(seed or 0), seed_t, head_chunk)


def draw_seed(device) -> torch.Tensor:
    """A 64-bit dropout seed drawn on ``device`` from torch's device generator,
    as an int64 tensor of one element that the kernels read when they run.
    torch.manual_seed / torch.cuda.manual_seed make it reproducible, no host
    sync is needed, and inside a captured HIP graph each replay draws a new
    seed (torch advances the generator's offset per replay), so dropout masks
    differ between replays as they do between eager steps."""
    return torch.randint(0, 2**62, (1,), dtype=torch.int64, device=device)


def dense_attention(q, k, v, scale=None, node_scores=True, dropout_p=0.0, seed=None):
    """Functional form of full_attention: q [.., N_q, H, d], k/v [.., N_k, H, d]
    -> (x [N_q, H, d], node_scores [N_k] or empty).  dropout_p > 0 applies
    dropout to the attention probabilities.  seed: an int (a fixed mask), an
    int64 device tensor of one element (read by the kernels when they run), or
    None to draw one on the device with draw_seed."""
    H, d = q.shape[-2], q.shape[-1]
    q = _prep(q.reshape(-1, H, d), "q")
    k = _prep(k.reshape(-1, H, d), "k")
    v = _prep(v.reshape(-1, H, d), "v")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    _dtype_code(q)
    if k.shape != v.shape or k.shape[1:] != q.shape[1:]:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if scale is None:
        scale = math.sqrt(d)
    dropout_p = float(dropout_p)
    if not 0.0 <= dropout_p <= 1.0:
        raise ValueError(f"dropout probability has to be between 0 and 1, but got {dropout_p}")
    if not float(scale) > 0.0:
        raise ValueError(f"scale must be > 0, got {scale}")
    seed_t = None
    if dropout_p > 0.0 and seed is None:
        seed_t = draw_seed(q.device)
    elif isinstance(seed, torch.Tensor):
        seed_t, seed = seed, None
    return DenseAttentionFunction.apply(q, k, v, float(scale), bool(node_scores), dropout_p,
                                        int(seed or 0), seed_t)


# ---------------------------------------------------------------- the module
class CoreAttention(nn.Module):
    """Same constructor/attributes/forward as the reference's CoreAttention.

    ``flash_layout`` (an addition) picks the flash branch's output layout:
    "graphormer" (default) as graphormer_dist_node_level.py:111-122 returns it
    (the [b, H, N, d] result transposed back to [b, N, H*d]); "gt_twin" as
    gt_dist_node_level_single_window.py:212-225 does, viewing the [b, H, N, d]
    result as [b, N, H*d] without the transpose (heads and nodes interleave).
    install() picks "gt_twin" for the GT twin's modules."""

    FLASH_LAYOUTS = ("graphormer", "gt_twin")

    def __init__(self, hidden_size, attention_dropout_rate, num_heads, cache: AdjacencyCache = None,
                 flash_layout: str = "graphormer"):
        super().__init__()
        if flash_layout not in self.FLASH_LAYOUTS:
            raise ValueError(f"flash_layout must be one of {self.FLASH_LAYOUTS}, got {flash_layout!r}")
        self.flash_layout = flash_layout
        self.hidden_size_per_attention_head = hidden_size // num_heads
        self.scale = math.sqrt(self.hidden_size_per_attention_head)
        self.num_heads = num_heads
        self.att_dropout = nn.Dropout(attention_dropout_rate)
        self.attention_dropout_rate = attention_dropout_rate
        self.adjacency_cache = cache or default_cache

    def full_attention(self, k, q, v, attn_bias, mask=None, pruning_mask=None):
        """graphormer_dist_node_level.py:42-65.  Returns (x [b, N, H, d], node_scores [N_k]).
        In training mode the probabilities go through att_dropout (p of the
        module's nn.Dropout), as the reference's self.att_dropout(x) does.
        With attn_bias, pruning_mask or mask the materialized path runs
        (dense_attention_bias); without them the fused kernels."""
        if q.size(0) != 1:
            raise NotImplementedError("batch size must be 1 (as in NeutronGT's window step)")
        p = self.att_dropout.p if self.training else 0.0
        if attn_bias is not None or mask is not None or pruning_mask is not None:
            x, ns = dense_attention_bias(q, k, v, self.scale, attn_bias=attn_bias,
                                         pruning_mask=pruning_mask, mask=mask, dropout_p=p)
        else:
            x, ns = dense_attention(q, k, v, scale=self.scale, dropout_p=p)
        return x.unsqueeze(0), ns

    def naive_attention(self, q, k, v, dropout_p=0.0):
        """graphormer_dist_node_level.py:100-105 on [b, N, H, d] inputs:
        softmax(q k^T / sqrt(d)) with dropout always applied (F.dropout with
        training=True), no node scores.  Returns (x [b, N, H, d], None)."""
        if q.size(0) != 1:
            raise NotImplementedError("batch size must be 1 (as in NeutronGT's window step)")
        d = q.shape[-1]
        x, _ = dense_attention(q, k, v, scale=1.0 / math.sqrt(d), node_scores=False,
                               dropout_p=dropout_p)
        return x.unsqueeze(0), None

    def sparse_attention_bias(self, q, k, v, edge_index, attn_bias, kv_ext=None,
                              interleave_grads=False):
        """graphormer_dist_node_level.py:67-98.  Returns (x [N_q, H, d], node_scores).
        ``kv_ext`` (k_r, v_r): extra key rows after k/v, without gradient.
        ``attn_bias`` [1, H, N, N] (optional): added to each edge's clamped
        score at [0, h, src, dst], as the reference's :81-84 does."""
        return sparse_attention(q, k, v, edge_index, num_heads=self.num_heads, scale=self.scale,
                                cache=self.adjacency_cache, kv_ext=kv_ext, attn_bias=attn_bias,
                                interleave_grads=interleave_grads)

    def forward(self, q, k, v, attn_bias=None, edge_index=None, attn_type=None, mask=None,
                pruning_mask=None, kv_ext=None, interleave_grads=False):
        """The reference's dispatch; ``kv_ext`` (an addition: (k_r, v_r), each
        [R, H, d], no gradient) appends key rows without a concatenation;
        ``interleave_grads`` (an addition, sparse path): dQ, dK, dV as views of
        one [N, 3, H, d] buffer, for a caller that projects q, k, v from one
        input (the other paths ignore it)."""
        batch_size, s_len = q.size(0), q.size(1)
        if kv_ext is not None and attn_type != "sparse":
            k = torch.cat([k, kv_ext[0].detach().to(k.dtype).reshape(1, -1, *k.shape[2:])], dim=1)
            v = torch.cat([v, kv_ext[1].detach().to(v.dtype).reshape(1, -1, *v.shape[2:])], dim=1)
        if attn_type == "sparse":
            x, score = self.sparse_attention_bias(q, k, v, edge_index, attn_bias, kv_ext=kv_ext,
                                                  interleave_grads=interleave_grads)
        elif attn_type == "flash":
            # The reference casts q/k/v to fp16 and the result back to fp32
            # (graphormer_dist_node_level.py:111-122).  Here the inputs are
            # rounded to fp16 as well (held in fp32, where fp16 values are
            # exact), the attention runs on the fp32 kernels, and the output is
            # rounded to fp16 before it is returned as fp32.  The gradients
            # pass through the same two casts, so they too are fp16-rounded.
            q16, k16, v16 = (t.half().float() for t in (q, k, v))
            x, score = self.naive_attention(q16, k16, v16, dropout_p=self.attention_dropout_rate)
            x = x.half().float()
            if self.flash_layout == "gt_twin":  # [b, H, N, d] memory, viewed as [b, N, H*d] below
                x = x.transpose(1, 2).contiguous()
        else:
            x, score = self.full_attention(k, q, v, attn_bias, mask=mask, pruning_mask=pruning_mask)
        x = x.view(batch_size, s_len, -1)
        return x, score


def install(model: nn.Module, cache: AdjacencyCache = None) -> int:
    """Replaces every ``local_attn`` CoreAttention-like submodule of ``model``
    (NeutronGT's MultiHeadAttention / DistributedAttentionNodeLevel) with this
    module, keeping hidden size, heads and dropout, and for modules of the GT
    twin (gt_dist_node_level_single_window) its flash-branch output layout.
    Returns the count."""
    n = 0
    for mod in list(model.modules()):
        old = getattr(mod, "local_attn", None)
        if isinstance(old, nn.Module) and hasattr(old, "hidden_size_per_attention_head") \
                and not isinstance(old, CoreAttention):
            twin = type(old).__module__.rsplit(".", 1)[-1] == "gt_dist_node_level_single_window"
            new = CoreAttention(old.hidden_size_per_attention_head * old.num_heads,
                                old.attention_dropout_rate, old.num_heads, cache=cache,
                                flash_layout="gt_twin" if twin else "graphormer")
            new.train(old.training)
            mod.local_attn = new
            n += 1
    return n
