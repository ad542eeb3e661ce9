// Bias gradient of a bf16 linear layer: db[j] = sum over rows k of dy[k][j]
// in fp32, summed in a fixed order (deterministic).
//
// Part of the backward of the encoder's nn.Linear layers (MultiHeadAttention
// projections and FFN, NeutronGT/models/graphormer_dist_node_level.py:130-206)
// under bf16 autocast, where dy is [32,768 x 768]; the weight gradient itself
// is a library GEMM (neutrongt_amd/linear.py).  A column reduction of a tall
// matrix: blocks own 256 columns (a thread 8 adjacent columns, one 16-byte
// load per row when the width allows) of a chunk of rows, and a second pass adds the chunks'
// partials in chunk order.  HBM-bound: K * n * 2 bytes read once.
#include "ngt_common.h"

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr int kColsPerBlock = 256;      // 32 threads x 8 columns
constexpr int kRowLanes = kBlock / 32;  // threads per column group
constexpr int kRowsPerChunk = 256;
constexpr int kUnroll = 4;  // 32,768 x 768: 16.9 -> 12.2 us per pass (hipEvent, stand-alone)

// part[chunk][j] = sum over the chunk's rows of dy[k][j].
// grid = (ceil(n / 256), n_chunks).  VEC: n a multiple of 8 and dy 16-byte
// aligned, one 16-byte load per row and thread; otherwise (e.g. a 47-class
// readout) the thread's 8 columns are read one bf16 at a time, those past n
// skipped.  Both add each column's rows in the same order.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_colsum(const bf16_t* __restrict__ dy, int64_t K,
                                                   int32_t n, float* __restrict__ part) {
  __shared__ float red[kRowLanes][kColsPerBlock];
  const int cg = threadIdx.x & 31;  // 8-column group of this thread
  const int rl = threadIdx.x >> 5;  // row lane
  const int col = blockIdx.x * kColsPerBlock + cg * 8;
  const int64_t r0 = int64_t(blockIdx.y) * kRowsPerChunk;
  const int64_t r1 = r0 + kRowsPerChunk < K ? r0 + kRowsPerChunk : K;
  float s[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) s[c] = 0.f;
  if (col < n) {
    // kUnroll rows' loads in flight before they are added (in row order)
    for (int64_t r = r0 + rl; r < r1; r += kRowLanes * kUnroll) {
      if constexpr (VEC) {
        uint4 w[kUnroll];
#pragma unroll
        for (int t = 0; t < kUnroll; ++t) {
          const int64_t rr = r + int64_t(t) * kRowLanes;
          w[t] = rr < r1 ? *reinterpret_cast<const uint4*>(dy + rr * n + col)
                         : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int t = 0; t < kUnroll; ++t) {
          const uint32_t u[4] = {w[t].x, w[t].y, w[t].z, w[t].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            s[2 * c] += bf16_to_f32(static_cast<uint16_t>(u[c] & 0xffffu));
            s[2 * c + 1] += bf16_to_f32(static_cast<uint16_t>(u[c] >> 16));
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < kUnroll; ++t) {
          const int64_t rr = r + int64_t(t) * kRowLanes;
          if (rr < r1) {
#pragma unroll
            for (int c = 0; c < 8; ++c)
              if (col + c < n) s[c] += bf16_to_f32(dy[rr * n + col + c].x);
          }
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) red[rl][cg * 8 + c] = s[c];
  __syncthreads();
  const int j = blockIdx.x * kColsPerBlock + threadIdx.x;
  if (j < n) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < kRowLanes; ++q) t += red[q][threadIdx.x];
    part[int64_t(blockIdx.y) * n + j] = t;
  }
}

// db[j] = sum of part[chunk][j] over chunks: 16 lanes per column each add the
// chunks c = lane mod 16 in order, then the 16 lane sums are added in lane
// order (fixed order; one serial lane per column ran at 31 us for 128 chunks,
// 8 lanes at 8.7 us, 16 lanes 6.4 us, hipEvent, stand-alone).
constexpr int kRedLanes = 16;
constexpr int kRedCols = kBlock / kRedLanes;
__global__ __launch_bounds__(kBlock) void k_colsum_reduce(const float* __restrict__ part,
                                                          int32_t n_chunks, int32_t n,
                                                          float* __restrict__ db) {
  __shared__ float red[kRedLanes][kRedCols];
  const int cl = threadIdx.x % kRedCols;
  const int ln = threadIdx.x / kRedCols;
  const int j = blockIdx.x * kRedCols + cl;
  float t = 0.f;
  if (j < n)
    for (int c = ln; c < n_chunks; c += kRedLanes) t += part[int64_t(c) * n + j];
  red[ln][cl] = t;
  __syncthreads();
  if (ln == 0 && j < n) {
    float u = 0.f;
#pragma unroll
    for (int q = 0; q < kRedLanes; ++q) u += red[q][cl];
    db[j] = u;
  }
}

inline int64_t chunks_for(int64_t K) { return (K + kRowsPerChunk - 1) / kRowsPerChunk; }

int check(const char* fn, int64_t K, int n) {
  if (K < 0 || n < 1)
    return set_error(NGT_ERR_ARG, "%s: bad sizes n_rows=%lld n_cols=%d", fn,
                     static_cast<long long>(K), n);
  if (chunks_for(K) > 65535)
    return set_error(NGT_ERR_UNSUPPORTED, "%s: n_rows=%lld exceeds %lld", fn,
                     static_cast<long long>(K), 65535LL * kRowsPerChunk);
  return NGT_OK;
}

// out[i] = sum over c = 0 .. n_chunks-1, in that order, of in[c * n + i]: the
// row-chunk partials of the split-K weight gradient added up.  4 elements a
// thread (one 16-byte load per chunk when n is a multiple of 4 and the
// pointers 16-byte aligned), the loads of 4 chunks in flight at once.
// HBM-bound: n_chunks * n * 4 bytes read, n * 4 written.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_chunk_sum(const float* __restrict__ in,
                                                       int32_t n_chunks, int64_t n,
                                                       float* __restrict__ out) {
  const int64_t stride = int64_t(gridDim.x) * kBlock * 4;
  for (int64_t i = (blockIdx.x * int64_t(kBlock) + threadIdx.x) * 4; i < n; i += stride) {
    if (VEC) {
      float4 acc = *reinterpret_cast<const float4*>(in + i);
      int32_t c = 1;
      for (; c + 4 <= n_chunks; c += 4) {
        float4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = *reinterpret_cast<const float4*>(in + (c + k) * n + i);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc.x += v[k].x;
          acc.y += v[k].y;
          acc.z += v[k].z;
          acc.w += v[k].w;
        }
      }
      for (; c < n_chunks; ++c) {
        const float4 v = *reinterpret_cast<const float4*>(in + c * n + i);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      *reinterpret_cast<float4*>(out + i) = acc;
    } else {
      for (int64_t e = i; e < i + 4 && e < n; ++e) {
        float acc = in[e];
        for (int32_t c = 1; c < n_chunks; ++c) acc += in[c * n + e];
        out[e] = acc;
      }
    }
  }
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_chunk_sum_f32(const float* in, int32_t n_chunks, int64_t n, float* out,
                                 void* stream) {
  if (n_chunks < 1 || n < 0 || (n > 0 && (!in || !out)))
    return set_error(NGT_ERR_ARG, "ngt_chunk_sum_f32: bad arguments");
  if (n == 0) return NGT_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = n % 4 == 0 && !(reinterpret_cast<uintptr_t>(in) & 15) &&
                   !(reinterpret_cast<uintptr_t>(out) & 15);
  int64_t blocks = (n + kBlock * 4 - 1) / (kBlock * 4);
  if (blocks > 65536) blocks = 65536;
  KernelTimer timer_("chunk_sum", st);
  if (vec)
    hipLaunchKernelGGL(k_chunk_sum<true>, dim3(unsigned(blocks)), dim3(kBlock), 0, st, in, n_chunks,
                       n, out);
  else
    hipLaunchKernelGGL(k_chunk_sum<false>, dim3(unsigned(blocks)), dim3(kBlock), 0, st, in,
                       n_chunks, n, out);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_colsum_workspace_bytes(int64_t n_rows, int32_t n_cols, size_t* bytes) {
  NGT_CHECK_OK(check("ngt_colsum_workspace_bytes", n_rows, n_cols));
  if (!bytes) return set_error(NGT_ERR_ARG, "ngt_colsum_workspace_bytes: null bytes");
  *bytes = size_t(chunks_for(n_rows)) * n_cols * 4;
  return NGT_OK;
}

extern "C" int ngt_colsum_bf16(const void* dy, int64_t n_rows, int32_t n_cols, float* out,
                               void* workspace, size_t workspace_bytes, void* stream) {
  NGT_CHECK_OK(check("ngt_colsum_bf16", n_rows, n_cols));
  if (!out) return set_error(NGT_ERR_ARG, "ngt_colsum_bf16: null out");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nc = chunks_for(n_rows);
  if (nc > 0) {
    if (!dy) return set_error(NGT_ERR_ARG, "ngt_colsum_bf16: null dy");
    if (reinterpret_cast<uintptr_t>(dy) & 1)
      return set_error(NGT_ERR_ARG, "ngt_colsum_bf16: dy must be 2-byte aligned");
    const bool vec = n_cols % 8 == 0 && !(reinterpret_cast<uintptr_t>(dy) & 15);
    const size_t need = size_t(nc) * n_cols * 4;
    if (!workspace || workspace_bytes < need)
      return set_error(NGT_ERR_WORKSPACE, "ngt_colsum_bf16: workspace %zu < %zu", workspace_bytes,
                       need);
    KernelTimer timer_("colsum", st);
    const dim3 grid((n_cols + kColsPerBlock - 1) / kColsPerBlock, static_cast<unsigned>(nc));
    if (vec)
      hipLaunchKernelGGL(k_colsum<true>, grid, dim3(kBlock), 0, st, static_cast<const bf16_t*>(dy),
                         n_rows, n_cols, static_cast<float*>(workspace));
    else
      hipLaunchKernelGGL(k_colsum<false>, grid, dim3(kBlock), 0, st,
                         static_cast<const bf16_t*>(dy), n_rows, n_cols,
                         static_cast<float*>(workspace));
    NGT_HIP_CHECK(hipGetLastError());
  }
  // no rows: the reduce adds no chunks and writes zeros
  hipLaunchKernelGGL(k_colsum_reduce, dim3((n_cols + kRedCols - 1) / kRedCols), dim3(kBlock), 0, st,
                     static_cast<const float*>(workspace), static_cast<int32_t>(nc), n_cols, out);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}
