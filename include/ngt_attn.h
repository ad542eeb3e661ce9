/*
 * ngt_attn.h -- C ABI of libngt_attn.so, the MI355X (gfx950) kernels behind
 * NeutronGT's window attention core.
 *
 * Every entry point takes device pointers, sizes and a hipStream_t (passed as
 * void*), launches asynchronously on that stream, never synchronises and never
 * allocates: scratch memory comes from the caller through a workspace pointer
 * whose size is given by the matching *_workspace_bytes() query.
 * Return value: NGT_OK (0) or an NGT_ERR_* code; ngt_last_error() returns the
 * message of the last failure on the calling thread.
 *
 * Tensor layouts (row-major, contiguous, 16-byte aligned base pointers):
 *   q   [n_q, H, d]    queries            (reference: q.view(-1, H, d))
 *   k,v [n_k, H, d]    keys / values
 *   out [n_q, H, d]    attention output   (reference returns x.view(1, N, H*d))
 * Element type is selected by `dtype` (NGT_F32 or NGT_BF16); all arithmetic is
 * fp32.
 */
#ifndef NGT_ATTN_H
#define NGT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NGT_ABI_VERSION 11

#define NGT_F32 0
#define NGT_BF16 1

#define NGT_OK 0
#define NGT_ERR_ARG 1         /* bad argument (shape, null pointer, range) */
#define NGT_ERR_UNSUPPORTED 2 /* shape the library has no kernel for */
#define NGT_ERR_HIP 3         /* HIP runtime error */
#define NGT_ERR_WORKSPACE 4   /* workspace smaller than the query said */

/* Indices into ngt_window_csr.info (device int32[NGT_INFO_LEN]). */
#define NGT_INFO_ITEMS_Q 0   /* work items, query-major */
#define NGT_INFO_PARTS_Q 1   /* partial slots, query-major */
#define NGT_INFO_SPLITS_Q 2  /* rows split over several items, query-major */
#define NGT_INFO_ITEMS_K 3
#define NGT_INFO_PARTS_K 4
#define NGT_INFO_SPLITS_K 5
#define NGT_INFO_DST_END 6   /* max(dst) + 1, or 0 without edges */
#define NGT_INFO_SRC_END 7   /* max(src) + 1, or 0 without edges */
#define NGT_INFO_BAD_EDGES 8 /* edges whose src/dst fell outside [0,n_k)/[0,n_q) */
#define NGT_INFO_MAX_DEG_Q 9
#define NGT_INFO_MAX_DEG_K 10
#define NGT_INFO_PACKED_Q 11  /* rows in the packed small-row list, query-major */
#define NGT_INFO_PACKED_K 12
#define NGT_INFO_SMALL_Q 13   /* packing threshold the build used, query-major */
#define NGT_INFO_SMALL_K 14
#define NGT_INFO_LEN 16

/*
 * Window adjacency in both orientations plus the degree-binned work lists the
 * kernels are scheduled from.  All pointers are device memory owned by the
 * caller; sizes are fixed by ngt_csr_sizes().
 *
 * Query-major ("CSR"): row i lists the edges e = (j -> i) with dst == i, sorted
 *   by (dst, src, edge id) -- duplicates kept, stable.  col = src, perm = edge id.
 * Key-major ("transposed CSR"): row j lists the edges with src == j, sorted by
 *   (src, dst, edge id).  t_col = dst, t_perm = edge id.
 * q2t[p] = key-major position of the query-major edge at position p.
 * Degree-binned schedule, per orientation:
 *   rows with more than chunk edges: cut into chunk-edge work items (listed
 *     first); each writes fp32 partials into its partial slot;
 *   rows with small < degree <= chunk: one work item per row, longest first;
 *   rows with degree <= small: the packed list (row ids, longest first); the
 *     kernels give each packed row one edge slot, several rows per wave.
 * Work items are int32x4 {row, edge_begin, edge_end, part}: part = -1 means the
 *   item covers the whole row; part >= 0 is the partial slot of one chunk.
 * Splits are int32x4 {row, part_begin, n_parts, 0}.
 */
/* small_q / small_k value asking ngt_csr_build to choose the packing
 * threshold from the rows' degrees: the first of 8, 16, 24, 32 (each capped
 * at chunk - 1) that packs at least 78 % of the rows, else the last; the
 * threshold used is reported in info[NGT_INFO_SMALL_Q / _K].  Measured as the
 * best or within 1 % of it on seven windows with 8 heads (GT arxiv windows
 * with 0-16 related keys per query, GPH_Slim windows of mean degree 8-28). */
#define NGT_SMALL_FROM_DEGREES (-1)

typedef struct ngt_window_csr {
  int32_t n_q;
  int32_t n_k;
  int64_t n_edges;
  int32_t chunk_q;   /* max edges per work item */
  int32_t chunk_k;
  int32_t small_q;   /* rows with <= small edges go to the packed list (0 <= small < chunk),
                        or NGT_SMALL_FROM_DEGREES */
  int32_t small_k;
  int32_t* rowptr;   /* [n_q + 1] */
  int32_t* col;      /* [E] */
  int32_t* perm;     /* [E] */
  int32_t* t_rowptr; /* [n_k + 1] */
  int32_t* t_col;    /* [E] */
  int32_t* t_perm;   /* [E] */
  int32_t* q2t;      /* [E] */
  int32_t* items_q;  /* [max_items_q * 4] */
  int32_t* splits_q; /* [max_splits_q * 4] */
  int32_t* packed_q; /* [n_q] */
  int32_t* items_k;  /* [max_items_k * 4] */
  int32_t* splits_k; /* [max_splits_k * 4] */
  int32_t* packed_k; /* [n_k] */
  int32_t* info;     /* [NGT_INFO_LEN] */
  int32_t max_items_q;
  int32_t max_splits_q;
  int32_t max_items_k;
  int32_t max_splits_k;
  /* Host copies of info[] that the launch functions size their grids and
   * partial buffers from; the caller fills them after ngt_csr_build (one
   * device-to-host copy of info). */
  int32_t n_items_q;
  int32_t n_parts_q;
  int32_t n_splits_q;
  int32_t n_packed_q;
  int32_t n_items_k;
  int32_t n_parts_k;
  int32_t n_splits_k;
  int32_t n_packed_k;
  /* Optional (NULL: not built): rows in descending degree order, ties by
   * descending row id -- every query row, and the key rows j < min(n_q, n_k)
   * (the window's own nodes).  The tiled kernels of dense windows schedule
   * blocks of rows of similar degree from them; without them every window
   * runs the work-list kernels. */
  int32_t* order_q;  /* [n_q] */
  int32_t* order_k;  /* [min(n_q, n_k)] */
} ngt_window_csr;

int ngt_abi_version(void);
const char* ngt_last_error(void);

/* Sizes of the ngt_window_csr arrays for a window (host-only arithmetic). */
int ngt_csr_sizes(int64_t n_edges, int32_t n_q, int32_t n_k, int32_t chunk_q, int32_t chunk_k,
                  int32_t* max_items_q, int32_t* max_splits_q, int32_t* max_items_k,
                  int32_t* max_splits_k);

/* Scratch bytes ngt_csr_build needs (queries the device's sort configuration). */
int ngt_csr_workspace_bytes(int64_t n_edges, int32_t n_q, int32_t n_k, size_t* bytes);

/*
 * Builds both orientations of the window adjacency from a COO edge_index.
 * Replaces the COO consumption in
 *   NeutronGT/models/graphormer_dist_node_level.py:75-97 (gathers by
 *   edge_index[0]/[1] and torch_scatter by edge_index[1]), with the edge list
 *   produced by NeutronGT/core/node_level_pipeline/window_state.py:122-140.
 * edge_index: int64 [2, n_edges] (row 0 = src/key, row 1 = dst/query).
 * Out-of-range edges are counted in info[NGT_INFO_BAD_EDGES] and dropped; the
 * caller must check that counter and reject the window (the reference raises a
 * device-side index error).
 */
int ngt_csr_build(const int64_t* edge_index, ngt_window_csr* csr, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * Sparse (topology-masked) attention forward.
 * Replaces CoreAttention.sparse_attention_bias, forward half:
 *   NeutronGT/models/graphormer_dist_node_level.py:67-98
 *   NeutronGT/models/gt_dist_node_level_single_window.py:112-179
 * For edge e = (j -> i) and head h:
 *   a = sum_c k[j,h,c] q[i,h,c] / scale;  p = exp(clamp(a, lo, hi))
 *   out[i,h,:] = sum_e p v[j,h,:] / (sum_e p + eps)
 * rinv[i,h] = 1 / (sum_e p + eps) (fp32, saved for the backward).
 * node_score[i] = mean_h sum_e p for i < node_score_len (may be NULL).
 * Requires n_heads <= 64; head_dim <= 64.
 */
int ngt_sparse_workspace_bytes(const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                               size_t* fwd_bytes, size_t* bwd_bytes);
int ngt_sparse_fwd(int dtype, const void* q, const void* k, const void* v,
                   const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim, float scale,
                   float clamp_lo, float clamp_hi, float eps, void* out, float* rinv,
                   float* node_score, int32_t node_score_len, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * ngt_sparse_fwd without a workspace argument, allocating nothing.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  Its scratch is a static device array of 32 MiB that
 * each device using the library holds until the process ends; a window whose
 * forward workspace (ngt_sparse_workspace_bytes' fwd_bytes) exceeds it is
 * rejected with NGT_ERR_UNSUPPORTED.  Same results as ngt_sparse_fwd, bit for
 * bit.  The scratch used is the current device's copy: `stream` must belong
 * to the current device (NGT_ERR_ARG otherwise; the null stream is the
 * current device's).  Every call on a device shares that device's array:
 * calls that overlap on one device (several streams or threads) race, so a
 * caller issues them on one stream at a time per device.
 */
int ngt_sparse_fwd_noalloc(int dtype, const void* q, const void* k, const void* v,
                           const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                           float scale, float clamp_lo, float clamp_hi, float eps, void* out,
                           float* rinv, float* node_score, int32_t node_score_len, void* stream);

/*
 * Sparse attention backward (what autograd derives from the same lines).
 * With G = grad_out, r = rinv, D_i = sum_c G[i,h,c] out[i,h,c]:
 *   dp_e = r_i (G_i . v_j - D_i);  da_e = dp_e p_e [lo <= a_e <= hi]
 *   grad_q[i] = sum_e da_e k_j / scale      (query-major pass)
 *   grad_k[j] = sum_e da_e q_i / scale      (key-major pass, no atomics)
 *   grad_v[j] = sum_e p_e r_i G_i           (key-major pass, no atomics)
 * da_e reaches the query-major pass through the workspace, or, on windows
 * with at least 32 edges per key row (csr->n_edges >= 32 csr->n_k) and no
 * per-edge bias, is recomputed there from the edge's K and V rows; both give
 * the same bits.  The workspace size does not depend on that choice.
 */
int ngt_sparse_bwd(int dtype, const void* q, const void* k, const void* v, const void* out,
                   const void* grad_out, const float* rinv, const ngt_window_csr* csr,
                   int32_t n_heads, int32_t head_dim, float scale, float clamp_lo, float clamp_hi,
                   void* grad_q, void* grad_k, void* grad_v, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * ngt_sparse_fwd / ngt_sparse_bwd with the key rows in two buffers: rows
 * j < n_k_main come from k/v, rows j >= n_k_main (up to csr->n_k) from
 * k_ext/v_ext row j - n_k_main.  Lets a caller append the detached K/V cache
 * of related keys (the reference concatenates it,
 * NeutronGT/models/graphormer_dist_node_level.py:162-168) without copying.
 * grad_k/grad_v are [n_k_main, H, d]: rows of k_ext/v_ext get no gradient.
 */
int ngt_sparse_fwd_ext(int dtype, const void* q, const void* k, const void* v, const void* k_ext,
                       const void* v_ext, int32_t n_k_main, const ngt_window_csr* csr,
                       int32_t n_heads, int32_t head_dim, float scale, float clamp_lo,
                       float clamp_hi, float eps, void* out, float* rinv, float* node_score,
                       int32_t node_score_len, void* workspace, size_t workspace_bytes,
                       void* stream);
int ngt_sparse_bwd_ext(int dtype, const void* q, const void* k, const void* v, const void* k_ext,
                       const void* v_ext, int32_t n_k_main, const void* out,
                       const void* grad_out, const float* rinv, const ngt_window_csr* csr,
                       int32_t n_heads, int32_t head_dim, float scale, float clamp_lo,
                       float clamp_hi, void* grad_q, void* grad_k, void* grad_v, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * ngt_sparse_bwd_ext writing grad_q, grad_k and grad_v with a row stride of
 * grad_row_stride elements (0: n_heads * head_dim, contiguous rows; else at
 * least that and a multiple of 16 bytes; the gradients 16-byte aligned).
 * Lets the caller of the Q/K/V projections (NeutronGT/models/
 * graphormer_dist_node_level.py:130-147: three nn.Linear of one input) take
 * the three gradients as one [N, 3 * H * d] matrix -- grad_q at column 0,
 * grad_k at H * d, grad_v at 2 * H * d, stride 3 * H * d -- and run the
 * projections' backward as one GEMM per operand.  Same values as
 * ngt_sparse_bwd_ext, bit for bit.
 */
int ngt_sparse_bwd_strided(int dtype, const void* q, const void* k, const void* v,
                           const void* k_ext, const void* v_ext, int32_t n_k_main,
                           const void* out, const void* grad_out, const float* rinv,
                           const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                           float scale, float clamp_lo, float clamp_hi, void* grad_q,
                           void* grad_k, void* grad_v, int64_t grad_row_stride, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * The optional per-pair bias of the sparse path.  Replaces the attn_bias term
 * of CoreAttention.sparse_attention_bias:
 *   NeutronGT/models/graphormer_dist_node_level.py:81-84
 *   (twin NeutronGT/models/gt_dist_node_level_single_window.py:151-157)
 * where a dense [1, H, N, N] bias, indexed [h, src, dst], is added to each
 * edge's clamped score:  p_e = exp(clamp(a_e, lo, hi) + bias[h, j, i]).
 *
 * ngt_edge_bias_gather copies bias[h][src][dst] (fp32, element strides
 * stride_h / stride_src / stride_dst; src < csr->n_k, dst < csr->n_q) into
 * per-edge arrays [E, H] in both CSR orders: edge_bias_q for the query-major
 * positions, edge_bias_t for the key-major ones.
 * ngt_sparse_fwd_bias / ngt_sparse_bwd_bias are ngt_sparse_fwd_ext /
 * ngt_sparse_bwd_ext with that term (edge_bias_q in the forward, edge_bias_t
 * in the backward).  The backward also writes, when grad_edge_bias_t is not
 * null, the score gradient of every edge in key-major order [E, H]:
 * dp_e p_e, the bias's gradient (the clamp mask does not apply to it).
 * ngt_edge_bias_grad adds those per pair, in key-major edge order (duplicate
 * edges are adjacent there), and stores the sums into grad_bias[h][src][dst];
 * entries of pairs without an edge are not written (zero them first).
 */
int ngt_edge_bias_gather(const ngt_window_csr* csr, int32_t n_heads, const float* bias,
                         int64_t stride_h, int64_t stride_src, int64_t stride_dst,
                         float* edge_bias_q, float* edge_bias_t, void* stream);
int ngt_sparse_fwd_bias(int dtype, const void* q, const void* k, const void* v,
                        const void* k_ext, const void* v_ext, int32_t n_k_main,
                        const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim, float scale,
                        float clamp_lo, float clamp_hi, float eps, const float* edge_bias_q,
                        void* out, float* rinv, float* node_score, int32_t node_score_len,
                        void* workspace, size_t workspace_bytes, void* stream);
int ngt_sparse_bwd_bias(int dtype, const void* q, const void* k, const void* v,
                        const void* k_ext, const void* v_ext, int32_t n_k_main, const void* out,
                        const void* grad_out, const float* rinv, const ngt_window_csr* csr,
                        int32_t n_heads, int32_t head_dim, float scale, float clamp_lo,
                        float clamp_hi, const float* edge_bias_t, float* grad_edge_bias_t,
                        void* grad_q, void* grad_k, void* grad_v, void* workspace,
                        size_t workspace_bytes, void* stream);
int ngt_edge_bias_grad(const ngt_window_csr* csr, int32_t n_heads, const float* grad_edge_bias_t,
                       float* grad_bias, int64_t stride_h, int64_t stride_src,
                       int64_t stride_dst, void* stream);

/*
 * Dense attention with the reference's optional terms, in its materialized
 * form.  Replaces the attn_bias / pruning_mask / mask lines of
 * CoreAttention.full_attention:
 *   NeutronGT/models/graphormer_dist_node_level.py:51-58
 *   (twin NeutronGT/models/gt_dist_node_level_single_window.py:80-97)
 * with the products S = Q K^T, O = (P o M) V, G V^T, (P o M)^T G, dS K and
 * dS^T Q left to library GEMMs; all arrays fp32 and contiguous.  The softmax
 * calls cover the n_heads consecutive heads head0 .. head0 + n_heads - 1 of
 * the window, so a caller can run the window a few heads at a time: their
 * arrays are [n_heads, n_q, n_k] and hold just those heads (head0 places the
 * dropout mask).
 * ngt_dense_bias_softmax_fwd: z = mask[i][j] ? -1e9 : s * scale + bias
 *   (bias nullable: the sum of attn_bias and pruning_mask; mask nullable,
 *   uint8 [n_q, n_k], nonzero = filled); p = softmax_j(z); pd = p o M with
 *   the dropout multiplier of ngt_dense_fwd (same seed, same mask; pd only
 *   with dropout_p > 0); lse [n_heads, n_q] = max + log(sum) (nullable).
 *   n_heads * n_q must not exceed 2^24 (NGT_ERR_ARG), here and in the
 *   backward.
 * ngt_dense_bias_softmax_bwd: with dpd = dL/d(p o M): dP = M o dpd,
 *   D_i = sum_j p dP, ds = p o (dP - D), 0 where masked.  ds is also the
 *   gradient of bias (and so of attn_bias and pruning_mask).
 * ngt_dense_abs_head_sum: m [n_q, n_k] = (accumulate ? m : 0) + the sum over
 *   the call's n_heads heads of s [n_heads, n_q, n_k], in head order, of
 *   |s * scale|; calls over consecutive head ranges give the bits of one
 *   call over all heads.
 * ngt_dense_abs_colsum: node_score[j] = sum_i m[i][j] / n_heads (the
 *   reference's abs(score).mean(dim=1).sum(dim=0), with m from
 *   ngt_dense_abs_head_sum over all n_heads heads), in a fixed order, with a
 *   caller workspace of ngt_dense_abs_colsum_workspace_bytes(n_k).
 */
int ngt_dense_bias_softmax_fwd(int32_t n_heads, int32_t head0, int32_t n_q, int32_t n_k,
                               const float* s, float scale, const float* bias,
                               const uint8_t* mask, float dropout_p, uint64_t seed,
                               const uint64_t* seed_dev, float* p, float* pd, float* lse,
                               void* stream);
int ngt_dense_bias_softmax_bwd(int32_t n_heads, int32_t head0, int32_t n_q, int32_t n_k,
                               const float* p, const float* dpd, const uint8_t* mask,
                               float dropout_p, uint64_t seed, const uint64_t* seed_dev,
                               float* ds, void* stream);
int ngt_dense_abs_head_sum(int32_t n_heads, int32_t n_q, int32_t n_k, const float* s, float scale,
                           int32_t accumulate, float* m, void* stream);
int ngt_dense_abs_colsum_workspace_bytes(int32_t n_k, size_t* bytes);
int ngt_dense_abs_colsum(int32_t n_heads, int32_t n_q, int32_t n_k, const float* m,
                         float* node_score, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Dense full-window attention (all pairs, no mask/bias).
 * Replaces CoreAttention.full_attention:
 *   NeutronGT/models/graphormer_dist_node_level.py:42-65
 *   NeutronGT/models/gt_dist_node_level_single_window.py:56-109
 * and the "flash" branch's naive_attention (graphormer_dist_node_level.py:
 * 100-105, 113-124; scale = 1/sqrt(d), dropout always on):
 *   S = (q * scale) k^T per head (full_attention multiplies by sqrt(d));
 *   P = softmax(S);  out = dropout(P) v;  lse[h,i] = logsumexp_j S[h,i,j]
 *   (fp32, for backward); node_score[j] = sum_i mean_h |S[h,i,j]| (may be NULL).
 * dropout_p in [0, 1] is the reference's att_dropout on P (training mode):
 * element (h, i, j) is kept with probability 1 - round(p * 65536) / 65536 and
 * scaled by 1 / (1 - p); the keep bit is a hash of (seed, h, i, j), so
 * ngt_dense_bwd with the same seed and p reproduces the forward's mask.
 * p > 0 needs n_q * ceil(n_k / 2) <= 2^32.
 * out_f32 (bf16 only, may be NULL): the forward also writes out in fp32 there,
 * and the backward then takes D_i = G_i . out_i from it instead of the
 * bf16-rounded out (out may then be NULL in the backward).  For rows whose
 * softmax is peaked, dS = P (dP - D) nearly cancels and the rounded out
 * alone moves dQ by percents.
 * workspace: fwd_bytes / bwd_bytes from ngt_dense_workspace_bytes for the
 * same dtype, sizes and node_scores (non-zero when node_score will be passed).
 * The forward uses it for node-score partials (H * n_k floats on the bf16
 * matrix-core path, d <= 32; per-block partials on the vector-ALU kernels)
 * and for per-split softmax states when it splits the keys of a large window
 * over several blocks (the vector-ALU kernels, fp32 and bf16 at head_dim 64;
 * the matrix-core path when no node scores are asked for); a size of 0 means
 * none is needed.  The backward uses it for D per query and head and, on the
 * matrix-core path, for the partial dQ of its key splits.
 * seed_dev (may be NULL): a device uint64 the kernels read the seed from when
 * they start, instead of `seed`; a captured HIP graph that rewrites it before
 * each replay draws a new mask per replay.  Forward and backward must see the
 * same value.
 * scale must be > 0 (NGT_ERR_ARG otherwise).
 */
int ngt_dense_workspace_bytes(int dtype, int32_t n_q, int32_t n_k, int32_t n_heads,
                              int32_t head_dim, int32_t node_scores, size_t* fwd_bytes,
                              size_t* bwd_bytes);
int ngt_dense_fwd(int dtype, const void* q, const void* k, const void* v, int32_t n_q,
                  int32_t n_k, int32_t n_heads, int32_t head_dim, float scale, float dropout_p,
                  uint64_t seed, const uint64_t* seed_dev, void* out, float* out_f32, float* lse,
                  float* node_score, void* workspace, size_t workspace_bytes, void* stream);
int ngt_dense_bwd(int dtype, const void* q, const void* k, const void* v, const void* out,
                  const float* out_f32, const void* grad_out, const float* lse, int32_t n_q,
                  int32_t n_k, int32_t n_heads, int32_t head_dim, float scale, float dropout_p,
                  uint64_t seed, const uint64_t* seed_dev, void* grad_q, void* grad_k,
                  void* grad_v, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Related-node selection for one window.
 * Replaces weightMetis_keepParent._merge_related_nodes,
 *   NeutronGT/core/metisPartition.py:397-425.
 * xadj/adjncy/eweights: int32 symmetric weighted CSR of the global graph
 *   (as built by NeutronGT/core/ppr_preprocess.py:30-71).
 * partition: int64 [n_part] global node ids (distinct).
 * For every neighbour nb outside the partition, w[nb] = sum of the weights of
 * the edges (u, nb) with u in the partition; ranking is by w descending, ties
 * by first appearance in (partition order, adjacency order); the top
 * len(w) * topk_percent // 100 are kept.  out (int64, capacity n_nodes) gets
 * sorted(partition U selected); out_len (device int32[3]) gets
 * {output length, number of external neighbours, number of invalid entries
 * (node ids out of range, negative weights, weight sums >= 2^33)}; the caller
 * must reject the result when the third is non-zero.
 */
int ngt_related_workspace_bytes(int32_t n_nodes, int32_t n_part, size_t* bytes);
int ngt_merge_related_nodes(const int32_t* xadj, const int32_t* adjncy, const int32_t* eweights,
                            int32_t n_nodes, const int64_t* partition, int32_t n_part,
                            int32_t topk_percent, int64_t* out, int32_t* out_len,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * METIS adjacency and edge weights from a PPR edge list, on the GPU.
 * Replaces build_adj_fromat, NeutronGT/core/ppr_preprocess.py:30-71.
 * edge_index: int64 [2, n_entries] (row 1 at edge_index + n_entries);
 * ppr_val: fp32 [n_entries].  Entry e is the undirected key (min, max) of its
 * endpoints; the values of one key are added in fp32 in entry order starting
 * from 0 (a fixed order: the reference's scatter_add_ run sequentially), and
 * w = int32(clamp_min(sum * 1000, 1)) with truncation.  Out: the symmetric
 * CSR xadj int32 [n_nodes + 1], adjncy / eweights int32 [2U] (capacity
 * 2 * n_entries suffices) over the U unique keys: rows in ascending node id,
 * inside row u the keys (u, v > u) in ascending v, then the keys (v < u, u)
 * in ascending v.  info (device int64[3]) = {U, entries with an id outside
 * [0, n_nodes), weights >= 2^31}; the caller must reject the result when
 * either count is non-zero.  Workspace: ngt_adj_weights_workspace_bytes.
 */
int ngt_adj_weights_workspace_bytes(int64_t n_entries, int64_t n_nodes, size_t* bytes);
int ngt_adj_weights(const int64_t* edge_index, const float* ppr_val, int64_t n_entries,
                    int64_t n_nodes, int32_t* xadj, int32_t* adjncy, int32_t* eweights,
                    int64_t* info, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Row gather dst[r, :] = src[idx[r], :] for r < n_rows (row_bytes a multiple
 * of 4).  Assembles a window's feature block from the feature table and the
 * duplicate-node cache, as in
 *   NeutronGT/core/node_level_pipeline/train_eval.py:234-242.
 * Indices outside [0, n_src) are counted in *bad (device int32) and their row
 * is zero-filled.
 */
int ngt_gather_rows(const void* src, int64_t n_src, const int64_t* idx, int64_t n_rows,
                    int64_t row_bytes, void* dst, int32_t* bad, void* stream);

/*
 * Duplicate-node layout of a rank's windows.
 * Replaces _compute_local_duplicate_nodes and build_dup_cache_metadata,
 *   NeutronGT/core/node_level_pipeline/window_state.py:52-73 and :181-205.
 * nodes: int64 [n_nodes], the rank's n_windows windows back to back; window
 * w is nodes[win_ptr[w] .. win_ptr[w+1]) (win_ptr: device int64
 * [n_windows + 1], non-decreasing, win_ptr[0] = 0, win_ptr[n_windows] =
 * n_nodes).  A node id is a duplicate when it occurs at least min_count
 * times in nodes (min_count 2: the rerange; 1: every id, the cache metadata
 * of given duplicate lists; 1 <= min_count <= 65536).  Out:
 *   reranged [n_nodes]: each window's duplicates in their original order,
 *     then its other nodes in their original order (torch.cat of
 *     part[isin(part, dups)] and part[~isin(part, dups)]);
 *   cache_ids [capacity n_nodes]: the sorted unique duplicate ids
 *     (torch.unique(..., sorted=True));
 *   dup_index [capacity n_nodes]: for every window in order, the cache
 *     position of each of its duplicates (torch.searchsorted(cache_ids, .));
 *     window w's entries are dup_index[dup_ptr[w] .. dup_ptr[w+1]), and its
 *     duplicate count is dup_ptr[w+1] - dup_ptr[w];
 *   dup_ptr [n_windows + 1] (int64);
 *   info (device int64[3]) = {cache entries, total duplicates, elements
 *     outside the windows win_ptr describes}; the caller must reject the
 *     result when the third is non-zero.
 * Workspace: ngt_window_dup_workspace_bytes(n_nodes).
 */
int ngt_window_dup_workspace_bytes(int64_t n_nodes, size_t* bytes);
int ngt_window_dup_layout(const int64_t* nodes, int64_t n_nodes, const int64_t* win_ptr,
                          int32_t n_windows, int32_t min_count, int64_t* reranged,
                          int64_t* dup_ptr, int64_t* cache_ids, int64_t* dup_index,
                          int64_t* info, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sequential segmented sum: out[s] = vals[seg[s]] + ... + vals[seg[s+1]-1],
 * accumulated from 0.0f in index order, for s < n_seg (seg: int64 [n_seg+1]).
 * This is the rounding of the fp32 scores.index_add_ in node_in
 * (NeutronGT/core/metisPartition.py:197-201) once the contributions are
 * grouped by candidate in their original order.  Segments outside
 * [0, n_vals] are counted in *bad (device int32) and give 0.
 */
int ngt_segment_sum_f32(const float* vals, int64_t n_vals, const int64_t* seg, int64_t n_seg,
                        float* out, int32_t* bad, void* stream);

/*
 * Personalised PageRank by APPNP propagation with per-row top-k: one step of
 * personal_pagerank_appnp (NeutronGT/core/ppr_backends/appnp_backend.py:
 * 179-224, whose SpGEMM is cusparse_spgemm.cu:65-267) for n_rows seed rows.
 *
 * Graph: CSR rowptr [n_nodes+1], col (int64), inv_deg[c] = 1 / max(deg(c), 1)
 * (fp32, the transition value of every edge c -> n).  State: fixed width K
 * (1 <= K <= 64): row r holds st_cnt[r] entries st_col/st_val[r*K + j] in rank
 * order (value descending, column ascending); seeds[r] is the row's seed.
 *
 * ngt_ppr_count writes row_off [n_rows+1] (int64): the exclusive scan of
 *   sum_j deg(st_col[r, j]) + 1 per row; row_off[n_rows] is the product count
 *   ngt_ppr_step needs (read it, then size the step's workspace).  Its
 *   workspace is 8*(n_rows+1) rounded up to 256 bytes plus a scan buffer; ask
 *   with ngt_ppr_count_workspace_bytes.
 * ngt_ppr_step computes next = topK(keep * (state P) + alpha * e_seed) into
 *   out_col/out_val/out_cnt (same layout as the state; must not alias it).
 *   keep is 1 - alpha rounded to fp32 from double (the reference scales an
 *   fp32 tensor by a Python float).  Products of one (row, column) are added
 *   in the order (state rank, CSR position), so the result is deterministic.
 * Bad ids (state columns, neighbours, seeds outside [0, n_nodes), negative
 * degrees) are counted in *status (device int32) and skipped; so is a total
 * below row_off[n_rows] (then nothing is expanded).
 * ngt_ppr_step_direct computes the same step, bit for bit, without the
 *   product list: each (row, column) sum is evaluated where the column first
 *   occurs, from searches in the row's other state lists, and each chunk of
 *   512 entries of one list keeps its best K before a per-row merge.  total
 *   is row_off[n_rows] from ngt_ppr_count (or any upper bound of the product
 *   count): the workspace, O(n_rows * (K + 1) + total / 512) * K * 8 bytes,
 *   is sized from it; no sort.  Needs every CSR row's columns in ascending
 *   order (transition_csr's order).  max_mult >= 1, the
 *   most times one column repeats within a CSR row (1 for a graph without
 *   duplicate edges), lets it skip columns, and whole lists, whose values
 *   are shown to fall below the row's K-th best (0: no skipping; the result
 *   is the same).
 *   status points to two int32: [0] bad ids as above, [1] CSR rows met out of
 *   order, a column repeated more than max_mult times, or a total too small
 *   for the state's lists (the output is then invalid).
 */
int ngt_ppr_count_workspace_bytes(int32_t n_rows, size_t* bytes);
int ngt_ppr_count(const int64_t* rowptr, int64_t n_nodes, const int32_t* st_col,
                  const int32_t* st_cnt, int32_t n_rows, int32_t K, int64_t* row_off,
                  int32_t* status, void* workspace, size_t workspace_bytes, void* stream);
int ngt_ppr_step_workspace_bytes(int64_t total, int32_t n_rows, size_t* bytes);
int ngt_ppr_step(const int64_t* rowptr, const int64_t* col, const float* inv_deg,
                 int64_t n_nodes, const int32_t* st_col, const float* st_val,
                 const int32_t* st_cnt, const int64_t* seeds, int32_t n_rows, int32_t K,
                 float alpha, float keep, const int64_t* row_off, int64_t total,
                 int32_t* out_col, float* out_val, int32_t* out_cnt, int32_t* status,
                 void* workspace, size_t workspace_bytes, void* stream);
int ngt_ppr_step_direct_workspace_bytes(int64_t total, int32_t n_rows, int32_t K, size_t* bytes);
int ngt_ppr_step_direct(const int64_t* rowptr, const int64_t* col, const float* inv_deg,
                        int64_t n_nodes, const int32_t* st_col, const float* st_val,
                        const int32_t* st_cnt, const int64_t* seeds, int32_t n_rows, int32_t K,
                        float alpha, float keep, int32_t max_mult, int64_t total,
                        int32_t* out_col, float* out_val, int32_t* out_cnt, int32_t* status,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Induced window subgraph with relabelling, on the GPU.
 *
 * ngt_subgraph_coo replaces torch_geometric.utils.subgraph(subset, edge_index,
 *   relabel_nodes=True, num_nodes) as called at
 *   NeutronGT/core/node_level_pipeline/window_state.py:82,127 and
 *   NeutronGT/core/metisPartition.py:280,290: edge e of edge_index (int64
 *   [2, n_edges], row 0 at edge_index, row 1 at edge_index + n_edges) is kept
 *   iff both endpoints are in subset; kept edges keep their order; node ids
 *   become positions in subset.
 * ngt_subgraph_csr replaces _subgraph_from_csr,
 *   NeutronGT/core/node_level_pipeline/window_state.py:92-119: for each node of
 *   node_set in order, its neighbours col[rowptr[g] .. rowptr[g+1]) (n_col
 *   entries in col) that are in node_set, in CSR order; out row 0 = the row
 *   node's position, row 1 = the neighbour's position.
 *
 * out: int64 [2, cap] (row 1 at out + cap), may be NULL to only count.
 * result: device int64[2] = {number of kept edges, error bits}; error bits:
 *   1 set node out of range, 2 duplicate set node, 4 edge endpoint out of
 *   range, 8 CSR row outside col.  Entries past cap are not written; call once
 *   with out = NULL, read result, then again with cap = result[0].
 * Workspace from ngt_subgraph_workspace_bytes(n_nodes, n_edges, n_set, ...)
 * with n_edges = edges of edge_index (COO form) or entries of col (CSR form);
 * the map it holds is rebuilt by every call.  The CSR form spreads each row
 * over waves of 2,048 entries, so hub rows do not serialise.
 */
int ngt_subgraph_workspace_bytes(int64_t n_nodes, int64_t n_edges, int32_t n_set, size_t* bytes);
int ngt_subgraph_coo(const int64_t* edge_index, int64_t n_edges, int64_t n_nodes,
                     const int64_t* subset, int32_t n_subset, int64_t* out, int64_t cap,
                     int64_t* result, void* workspace, size_t workspace_bytes, void* stream);
int ngt_subgraph_csr(const int64_t* rowptr, const int64_t* col, int64_t n_col, int64_t n_nodes,
                     const int64_t* node_set, int32_t n_set, int64_t* out, int64_t cap,
                     int64_t* result, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-kernel timing (no counterpart in the reference: instrumentation for the
 * benchmark's roofline figure).  While enabled, every kernel launch of this
 * library is bracketed by a hipEvent pair on its stream.  ngt_timing_summary
 * waits for the recorded events and writes one "name count total_ms" line per
 * kernel into buf (NUL-terminated), then forgets the records.
 */
int ngt_timing_enable(int on);
int ngt_timing_summary(char* buf, size_t len);

/*
 * LayerNorm over the last dimension (n_cols, a multiple of 4, at most 2048):
 *   y = (x - mean) / sqrt(var + eps) * gamma + beta per row, fp32 math,
 *   x in in_dtype, y in out_dtype (NGT_F32 or NGT_BF16), mean/rstd [n_rows]
 *   fp32 saved for the backward; gamma/beta fp32.  The backward writes dx in
 *   in_dtype from dy in grad_dtype, and dgamma/dbeta (fp32, either may be
 *   NULL) as column sums added in a fixed order.  Row bases 16-byte aligned
 *   for fp32, 8-byte for bf16 (each lane moves 4 elements per access).
 * Replaces the encoder's nn.LayerNorm under bf16 autocast
 * (NeutronGT/models/graphormer_dist_node_level.py:176-206, final_ln at
 * :242-381; NeutronGT/models/gt_dist_node_level_single_window.py:305-353).
 */
int ngt_layernorm_fwd(int in_dtype, const void* x, int64_t n_rows, int32_t n_cols,
                      const float* gamma, const float* beta, float eps, int out_dtype, void* y,
                      float* mean, float* rstd, void* stream);
int ngt_layernorm_bwd_workspace_bytes(int64_t n_rows, int32_t n_cols, size_t* bytes);
int ngt_layernorm_bwd(int in_dtype, const void* x, int grad_dtype, const void* dy, int64_t n_rows,
                      int32_t n_cols, const float* gamma, const float* mean, const float* rstd,
                      void* dx, float* dgamma, float* dbeta, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Residual add, dropout and LayerNorm in one pass (the pre-LN sub-layer
 * boundary of the Graphormer layer, NeutronGT/models/graphormer_dist_node_level.py:196-206):
 *   sum = x + dropout_p(y)  (x, y, sum in dtype; sum may be NULL),
 *   out = LayerNorm(sum)    (out_dtype; mean/rstd fp32 [n_rows]).
 * sum is rounded to dtype before the LayerNorm reads it.  Element (r, c) is
 * kept as the dense-attention mask keeps (head 0, query r, key c) for the same
 * seed, scaled by 1/(1-p); 0 <= p < 1.  The backward takes the saved sum, the
 * gradients of out and (may be NULL) of sum, and writes dx = g_sum + LN
 * backward, dy = dx * mask (both in dtype), dgamma/dbeta fp32 (fixed order).
 * Workspace: ngt_layernorm_bwd_workspace_bytes.  seed_dev (may be NULL) as
 * for ngt_dense_fwd: the seed is read from device memory at launch.  Row
 * alignment as for ngt_layernorm_fwd.
 */
int ngt_add_layernorm_fwd(int dtype, const void* x, const void* y, int64_t n_rows, int32_t n_cols,
                          float dropout_p, uint64_t seed, const uint64_t* seed_dev,
                          const float* gamma, const float* beta, float eps, void* sum,
                          int out_dtype, void* out, float* mean, float* rstd, void* stream);
int ngt_add_layernorm_bwd(int dtype, const void* sum, int grad_dtype, const void* g_out,
                          const void* g_sum, int64_t n_rows, int32_t n_cols, float dropout_p,
                          uint64_t seed, const uint64_t* seed_dev, const float* gamma,
                          const float* mean, const float* rstd, void* dx, void* dy,
                          float* dgamma, float* dbeta, void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * Column sums of a bf16 matrix in fp32: out[j] = sum_k dy[k][j], dy
 * [n_rows, n_cols] row-major (any n_cols >= 1; 16-byte loads when n_cols is
 * a multiple of 8 and dy 16-byte aligned); summed in a fixed order, the same
 * for either load width.  The bias gradient of the encoder's linear layers
 * under bf16 autocast (the autograd of nn.Linear's bias in
 * MultiHeadAttention, the FFN and the readout,
 * NeutronGT/models/graphormer_dist_node_level.py:130-206, :242-381).
 */
int ngt_colsum_workspace_bytes(int64_t n_rows, int32_t n_cols, size_t* bytes);
int ngt_colsum_bf16(const void* dy, int64_t n_rows, int32_t n_cols, float* out, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * out[i] = sum over c = 0 .. n_chunks-1, in that order, of in[c * n + i]
 * (fp32; in is [n_chunks, n] row-major, out [n]; n_chunks >= 1).  The sum of
 * the row-chunk partials of the encoder's split-K weight gradient dW = dY^T X
 * (the autograd of nn.Linear's weight, NeutronGT/models/
 * graphormer_dist_node_level.py:130-206): a batched GEMM leaves one partial
 * dW per chunk of rows.  16-byte loads when n is a multiple of 4 and both
 * pointers are 16-byte aligned; the same order either way.
 */
int ngt_chunk_sum_f32(const float* in, int32_t n_chunks, int64_t n, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NGT_ATTN_H */
