// Dense full-window attention with the reference's optional terms: a dense
// additive bias (attn_bias + pruning_mask) and a boolean mask filled with
// -1e9 before the softmax (NeutronGT/models/graphormer_dist_node_level.py:
// 42-65; twin gt_dist_node_level_single_window.py:56-109).  A dense
// [H, n_q, n_k] term makes the step O(n_q n_k H) in memory whatever the
// kernel, so this path keeps the reference's materialized form: the caller
// runs the four products S = Q K^T, O = P V, dP = G V^T, dV = P^T G,
// dQ = dS K, dK = dS^T Q as library GEMMs, and the kernels here do the rest
// row by row in fp32: logits, mask, softmax, dropout, the softmax backward
// and the node scores sum_i mean_h |S|.
#include "ngt_common.h"

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr float kMasked = -1e9f;  // masked_fill value of the reference
// Rows (head, query) of the softmax kernels: one block each, and a dispatch
// holds fewer than 2^32 work-items.
constexpr int64_t kMaxRows = int64_t(1) << 24;
constexpr int kColChunks = 64;    // row chunks of the column sums

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, kWave);
  return x;
}

// Block-wide reductions in a fixed order (waves in index order).
__device__ __forceinline__ float block_max(float x, float* red) {
  x = wave_max(x);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  __syncthreads();
  if (lane == 0) red[w] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = fmaxf(r, red[i]);
  return r;
}
__device__ __forceinline__ float block_sum(float x, float* red) {
  x = wave_sum(x);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  __syncthreads();
  if (lane == 0) red[w] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r += red[i];
  return r;
}

__device__ __forceinline__ float logit(const float* __restrict__ s, const float* __restrict__ b,
                                       const uint8_t* __restrict__ mk, int64_t j, float scale) {
  if (mk && mk[j]) return kMasked;
  const float x = s[j] * scale;
  return b ? x + b[j] : x;
}

// One block per (head, query row): z = mask ? -1e9 : S scale + bias;
// P = softmax(z) written to p; P o M (the dropout multiplier) to pd when
// dropout is on; lse = max + log(sum) (when lse is given).  grid = H * n_q
// over the heads head0 .. head0 + H - 1 of the window (the arrays hold just
// those heads; head0 places the dropout mask).
template <bool DROP>
__global__ __launch_bounds__(kBlock) void k_bias_softmax_fwd(
    const float* __restrict__ s, float scale, const float* __restrict__ bias,
    const uint8_t* __restrict__ mask, int32_t head0, int32_t n_q, int32_t n_k, DropoutMask dm,
    float* __restrict__ p, float* __restrict__ pd, float* __restrict__ lse) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;  // h * n_q + i
  const int h = head0 + static_cast<int>(row / n_q);
  const int i = static_cast<int>(row % n_q);
  const int64_t off = row * n_k;
  const float* sr = s + off;
  const float* br = bias ? bias + off : nullptr;
  const uint8_t* mr = mask ? mask + int64_t(i) * n_k : nullptr;
  float mx = -INFINITY;
  for (int64_t j = threadIdx.x; j < n_k; j += kBlock) mx = fmaxf(mx, logit(sr, br, mr, j, scale));
  mx = block_max(mx, red);
  float sum = 0.f;
  for (int64_t j = threadIdx.x; j < n_k; j += kBlock) sum += __expf(logit(sr, br, mr, j, scale) - mx);
  sum = block_sum(sum, red);
  const float inv = 1.0f / sum;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  for (int64_t j = threadIdx.x; j < n_k; j += kBlock) {
    const float pj = __expf(logit(sr, br, mr, j, scale) - mx) * inv;
    p[off + j] = pj;
    if constexpr (DROP)
      pd[off + j] = pj * drop_scale(dm, drop_word(dm, uint32_t(i), uint32_t(j)), uint32_t(j));
  }
  if (lse && threadIdx.x == 0) lse[row] = mx + __logf(sum);
}

// One block per (head, query row): with dpd = dL/d(P o M) (= G V^T),
// dP = M o dpd, D = sum_j P_j dP_j, dS = P o (dP - D), zero where masked
// (masked_fill passes no gradient).  grid = H * n_q over heads head0 ...
template <bool DROP>
__global__ __launch_bounds__(kBlock) void k_bias_softmax_bwd(
    const float* __restrict__ p, const float* __restrict__ dpd, const uint8_t* __restrict__ mask,
    int32_t head0, int32_t n_q, int32_t n_k, DropoutMask dm, float* __restrict__ ds) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  const int h = head0 + static_cast<int>(row / n_q);
  const int i = static_cast<int>(row % n_q);
  const int64_t off = row * n_k;
  const uint8_t* mr = mask ? mask + int64_t(i) * n_k : nullptr;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  auto dp_at = [&](int64_t j) {
    float x = dpd[off + j];
    if constexpr (DROP) x *= drop_scale(dm, drop_word(dm, uint32_t(i), uint32_t(j)), uint32_t(j));
    return x;
  };
  float d = 0.f;
  for (int64_t j = threadIdx.x; j < n_k; j += kBlock) d = fmaf(p[off + j], dp_at(j), d);
  d = block_sum(d, red);
  for (int64_t j = threadIdx.x; j < n_k; j += kBlock)
    ds[off + j] = (mr && mr[j]) ? 0.f : p[off + j] * (dp_at(j) - d);
}

// m[i][j] = (accumulate ? m[i][j] : 0) + sum over the launch's heads, in head
// order, of |S[h][i][j] scale|: the head sum of the node scores, built over
// one or several launches of consecutive heads with the same roundings as a
// single pass over all heads.
__global__ __launch_bounds__(kBlock) void k_abs_head_sum(const float* __restrict__ s, float scale,
                                                        int32_t H, int64_t plane, int32_t acc,
                                                        float* __restrict__ m) {
  const int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (t >= plane) return;
  float x = acc ? m[t] : 0.f;
  for (int h = 0; h < H; ++h) x += fabsf(s[int64_t(h) * plane + t] * scale);
  m[t] = x;
}

// Column sums of m / H over rows in two fixed-order passes:
// part[c][j] = sum over the rows of chunk c of m[i][j] * (1/H) (the head
// mean), then ns[j] = sum_c part[c][j].  The reference takes the head mean
// first, then the row sum (abs(score).mean(dim=1)...sum(dim=0)).
__global__ __launch_bounds__(kBlock) void k_abs_colsum_part(const float* __restrict__ m,
                                                           float invh, int32_t n_q, int32_t n_k,
                                                           int32_t rows_per_chunk,
                                                           float* __restrict__ part) {
  const int64_t j = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (j >= n_k) return;
  const int c = blockIdx.y;
  const int i0 = c * rows_per_chunk, i1 = min(n_q, i0 + rows_per_chunk);
  float acc = 0.f;
  for (int i = i0; i < i1; ++i) acc += m[int64_t(i) * n_k + j] * invh;
  part[int64_t(c) * n_k + j] = acc;
}

__global__ __launch_bounds__(kBlock) void k_abs_colsum_total(const float* __restrict__ part,
                                                            int32_t chunks, int32_t n_k,
                                                            float* __restrict__ ns) {
  const int64_t j = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (j >= n_k) return;
  float a = 0.f;
  for (int c = 0; c < chunks; ++c) a += part[int64_t(c) * n_k + j];
  ns[j] = a;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_dense_bias_softmax_fwd(int32_t n_heads, int32_t head0, int32_t n_q,
                                          int32_t n_k, const float* s, float scale,
                                          const float* bias,
                                          const uint8_t* mask, float dropout_p, uint64_t seed,
                                          const uint64_t* seed_dev, float* p, float* pd,
                                          float* lse, void* stream) {
  if (n_heads < 1 || head0 < 0 || n_q < 0 || n_k < 0)
    return set_error(NGT_ERR_ARG, "ngt_dense_bias_softmax_fwd: bad sizes");
  if (int64_t(n_heads) * n_q > kMaxRows)  // one block of kBlock work-items per row
    return set_error(NGT_ERR_ARG, "ngt_dense_bias_softmax_fwd: n_heads * n_q > %lld",
                     static_cast<long long>(kMaxRows));
  DropoutMask dm{};
  bool drop = false;
  NGT_CHECK_OK(make_dropout("ngt_dense_bias_softmax_fwd", dropout_p, seed, seed_dev, n_q, n_k, &dm,
                            &drop));
  if (n_q == 0 || n_k == 0) return NGT_OK;
  if (!s || !p || (drop && !pd))
    return set_error(NGT_ERR_ARG, "ngt_dense_bias_softmax_fwd: null pointer");
  const dim3 grid(unsigned(int64_t(n_heads) * n_q));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (drop)
    hipLaunchKernelGGL(k_bias_softmax_fwd<true>, grid, dim3(kBlock), 0, st, s, scale, bias, mask,
                       head0, n_q, n_k, dm, p, pd, lse);
  else
    hipLaunchKernelGGL(k_bias_softmax_fwd<false>, grid, dim3(kBlock), 0, st, s, scale, bias, mask,
                       head0, n_q, n_k, dm, p, pd, lse);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_dense_bias_softmax_bwd(int32_t n_heads, int32_t head0, int32_t n_q,
                                          int32_t n_k, const float* p, const float* dpd,
                                          const uint8_t* mask,
                                          float dropout_p, uint64_t seed,
                                          const uint64_t* seed_dev, float* ds, void* stream) {
  if (n_heads < 1 || head0 < 0 || n_q < 0 || n_k < 0)
    return set_error(NGT_ERR_ARG, "ngt_dense_bias_softmax_bwd: bad sizes");
  if (int64_t(n_heads) * n_q > kMaxRows)  // one block of kBlock work-items per row
    return set_error(NGT_ERR_ARG, "ngt_dense_bias_softmax_bwd: n_heads * n_q > %lld",
                     static_cast<long long>(kMaxRows));
  DropoutMask dm{};
  bool drop = false;
  NGT_CHECK_OK(make_dropout("ngt_dense_bias_softmax_bwd", dropout_p, seed, seed_dev, n_q, n_k, &dm,
                            &drop));
  if (n_q == 0 || n_k == 0) return NGT_OK;
  if (!p || !dpd || !ds) return set_error(NGT_ERR_ARG, "ngt_dense_bias_softmax_bwd: null pointer");
  const dim3 grid(unsigned(int64_t(n_heads) * n_q));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (drop)
    hipLaunchKernelGGL(k_bias_softmax_bwd<true>, grid, dim3(kBlock), 0, st, p, dpd, mask, head0,
                       n_q, n_k, dm, ds);
  else
    hipLaunchKernelGGL(k_bias_softmax_bwd<false>, grid, dim3(kBlock), 0, st, p, dpd, mask, head0,
                       n_q, n_k, dm, ds);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_dense_abs_colsum_workspace_bytes(int32_t n_k, size_t* bytes) {
  if (n_k < 0 || !bytes) return set_error(NGT_ERR_ARG, "ngt_dense_abs_colsum_workspace_bytes");
  *bytes = size_t(kColChunks) * size_t(n_k) * sizeof(float);
  return NGT_OK;
}

extern "C" int ngt_dense_abs_head_sum(int32_t n_heads, int32_t n_q, int32_t n_k, const float* s,
                                      float scale, int32_t accumulate, float* m, void* stream) {
  if (n_heads < 1 || n_q < 0 || n_k < 0)
    return set_error(NGT_ERR_ARG, "ngt_dense_abs_head_sum: bad sizes");
  const int64_t plane = int64_t(n_q) * n_k;
  if (plane == 0) return NGT_OK;
  if (!s || !m) return set_error(NGT_ERR_ARG, "ngt_dense_abs_head_sum: null pointer");
  const int64_t blocks = (plane + kBlock - 1) / kBlock;
  if (blocks > 0x7fffffff)
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_dense_abs_head_sum: n_q * n_k too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_abs_head_sum, dim3(unsigned(blocks)), dim3(kBlock), 0, st, s, scale,
                     n_heads, plane, accumulate ? 1 : 0, m);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_dense_abs_colsum(int32_t n_heads, int32_t n_q, int32_t n_k, const float* m,
                                    float* ns, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  if (n_heads < 1 || n_q < 0 || n_k < 0)
    return set_error(NGT_ERR_ARG, "ngt_dense_abs_colsum: bad sizes");
  if (n_k == 0) return NGT_OK;
  const size_t need = size_t(kColChunks) * size_t(n_k) * sizeof(float);
  if (!ns || (n_q > 0 && !m)) return set_error(NGT_ERR_ARG, "ngt_dense_abs_colsum: null pointer");
  if (!workspace || workspace_bytes < need)
    return set_error(NGT_ERR_WORKSPACE, "ngt_dense_abs_colsum: workspace %zu < %zu",
                     workspace_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rows = (n_q + kColChunks - 1) / kColChunks;
  const unsigned bx = unsigned((int64_t(n_k) + kBlock - 1) / kBlock);
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(k_abs_colsum_part, dim3(bx, kColChunks), dim3(kBlock), 0, st, m,
                     1.0f / float(n_heads), n_q, n_k, rows > 0 ? rows : 1, part);
  NGT_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(k_abs_colsum_total, dim3(bx), dim3(kBlock), 0, st, part, kColChunks, n_k, ns);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}
