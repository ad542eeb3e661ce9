// Dense full-window attention (all pairs), forward and backward.
//
// Reference: CoreAttention.full_attention
//   NeutronGT/models/graphormer_dist_node_level.py:42-65
//   S = (q * sqrt(d)) k^T      (the reference multiplies by sqrt(d))
//   P = softmax(S, -1);  out = P v;  node_score[j] = sum_i mean_h |S[h,i,j]|
// The backward is what autograd derives: dV = P^T G, dP = G V^T,
// dS = P (dP - rowsum(dP P)) = P (dP - D) with D_i = G_i . out_i,
// dQ = sqrt(d) dS K, dK = sqrt(d) dS^T Q.
// With dropout (training mode, reference att_dropout on P): out = (P o M) v
// with M = keep / (1 - p); dV = (P o M)^T G, dP = (G V^T) o M, and D_i = G_i .
// out_i still equals rowsum(dP o P).  The mask is regenerated from
// (seed, head, query, key) in every kernel (DropoutMask).
//
// Layout of one wave: 16 rows (lane % 16) x 4 column groups (lane / 16) of 8
// columns each, i.e. a 16 x 32 tile of S per step.  The forward keeps an
// online softmax per row (running max m, running sum l); every lane owns the
// partial sums of its own 8 columns and the four column groups of a row are
// combined once at the end.  Key/query tiles are read straight from global
// memory: a head's K/V (or Q/G) slice is a few hundred KB and stays in L2.
#include "ngt_common.h"

#include <math.h>
#include <stdlib.h>

#include <utility>

namespace ngt {

// Matrix-core kernels (ngt_dense_mfma.hip).
bool mfma_dense_supported(int d);
int mfma_dense_fwd(int d, const void* q, const void* k, const void* v, int n_q, int n_k, int H,
                   float scale, const DropoutMask* dm, void* out, float* out32, float* lse,
                   float* part, hipStream_t st);
int mfma_dense_bwd(int d, const void* q, const void* k, const void* v, const void* g,
                   const float* lse, const float* dsum, int n_q, int n_k, int H, float scale,
                   const DropoutMask* dm, void* gq, void* gk, void* gv, hipStream_t st);

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kRows = 16;        // rows per wave
constexpr int kColsPerLane = 8;  // columns per lane per tile
constexpr int kTile = 4 * kColsPerLane;
constexpr int kRowsPerBlock = kWaves * kRows;
constexpr int kScoreChunk = 8192;  // keys per LDS node-score accumulator pass

template <int DH>
__device__ __forceinline__ float dotv(const float (&a)[DH], const float (&b)[DH]) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int c = 0; c < DH; c += 2) {
    s0 = fmaf(a[c], b[c], s0);
    if (c + 1 < DH) s1 = fmaf(a[c + 1], b[c + 1], s1);
  }
  return s0 + s1;
}

// Sum over the 16 lanes of a DPP row (lanes 16g .. 16g+15); every lane of the
// row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x122, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x121, 0xf, 0xf, false));
  return x;
}

// ------------------------------------------------------------------ forward
// grid = (ceil(n_q / 64), H).  ns_part (optional) is [gridDim.x * H, n_k]:
// per block and head, sum over the block's 64 query rows of |S[h, i, j]|.
template <typename T, int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_dense_fwd(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, int32_t n_q,
    int32_t n_k, int32_t H, float scale, DropoutMask dm, T* __restrict__ out,
    float* __restrict__ out32, float* __restrict__ lse, float* __restrict__ ns_part) {
  __shared__ float ns_lds[kScoreChunk];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int h = blockIdx.y;
  const int64_t qi = int64_t(blockIdx.x) * kRowsPerBlock + wave * kRows + r;
  const bool q_ok = qi < n_q;
  if constexpr (DROP) dm = drop_for_head(dm, h);

  float qs[DH];
  if (q_ok) {
    load_row<T, DH>(q + (qi * H + h) * DH, qs);
#pragma unroll
    for (int c = 0; c < DH; ++c) qs[c] *= scale;
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) qs[c] = 0.f;
  }
  float acc[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  float m = -INFINITY, l = 0.f;
  const bool scores = ns_part != nullptr;

  for (int kc = 0; kc < n_k; kc += kScoreChunk) {
    const int kc_end = min(n_k, kc + kScoreChunk);
    if (scores) {
      __syncthreads();
      for (int t = threadIdx.x; t < kScoreChunk; t += kBlock) ns_lds[t] = 0.f;
      __syncthreads();
    }
    for (int kb = kc; kb < kc_end; kb += kTile) {
      float s[kColsPerLane];
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < kColsPerLane; ++i) {
        const int64_t kj = kb + g * kColsPerLane + i;
        if (kj < kc_end) {
          float kr[DH];
          load_row<T, DH>(k + (kj * H + h) * DH, kr);
          s[i] = dotv<DH>(qs, kr);
          tmax = fmaxf(tmax, s[i]);
        } else {
          s[i] = -INFINITY;
        }
      }
      if (scores) {
#pragma unroll
        for (int i = 0; i < kColsPerLane; ++i) {
          const float a = row16_sum(q_ok && s[i] != -INFINITY ? fabsf(s[i]) : 0.f);
          const int kj = kb + g * kColsPerLane + i;
          if (r == 0 && kj < kc_end) atomicAdd(&ns_lds[kj - kc], a);
        }
      }
      tmax = fmaxf(tmax, shfl_xor(tmax, 16));
      tmax = fmaxf(tmax, shfl_xor(tmax, 32));
      const float m_new = fmaxf(m, tmax);
      const float alpha = __expf(m - m_new);
      l *= alpha;
#pragma unroll
      for (int c = 0; c < DH; ++c) acc[c] *= alpha;
      uint32_t dw[kColsPerLane / 2];  // one dropout word per key pair
      if constexpr (DROP) {
#pragma unroll
        for (int i = 0; i < kColsPerLane / 2; ++i)
          dw[i] = drop_word(dm, uint32_t(qi), uint32_t(kb + g * kColsPerLane + 2 * i));
      }
#pragma unroll
      for (int i = 0; i < kColsPerLane; ++i) {
        const int64_t kj = kb + g * kColsPerLane + i;
        if (kj < kc_end) {
          const float p = __expf(s[i] - m_new);
          l += p;  // the softmax normaliser uses every key
          float pv = p;
          if constexpr (DROP) pv *= drop_scale(dm, dw[i / 2], uint32_t(kj));
          float vr[DH];
          load_row<T, DH>(v + (kj * H + h) * DH, vr);
#pragma unroll
          for (int c = 0; c < DH; ++c) acc[c] = fmaf(pv, vr[c], acc[c]);
        }
      }
      m = m_new;
    }
    if (scores) {
      __syncthreads();
      float* dst = ns_part + (int64_t(blockIdx.x) * H + h) * n_k + kc;
      for (int t = threadIdx.x; t < kc_end - kc; t += kBlock) dst[t] = ns_lds[t];
    }
  }
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    acc[c] += shfl_xor(acc[c], 16);
    acc[c] += shfl_xor(acc[c], 32);
  }
  if (q_ok && g == 0) {
    float o[DH];
    const float inv = n_k > 0 ? 1.0f / l : 0.f;
#pragma unroll
    for (int c = 0; c < DH; ++c) o[c] = acc[c] * inv;
    store_row<T, DH>(out + (qi * H + h) * DH, o);
    if (out32) store_f32<DH>(out32 + (qi * H + h) * DH, o);
    lse[int64_t(h) * n_q + qi] = n_k > 0 ? m + __logf(l) : -INFINITY;
  }
}

// node_score[j] = sum over rows of ns_part[:, j] / H.
__global__ void k_dense_scores(const float* __restrict__ part, int32_t rows, int32_t n_k, int32_t H,
                               float* __restrict__ ns) {
  for (int64_t j = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; j < n_k;
       j += int64_t(gridDim.x) * blockDim.x) {
    float s = 0.f;
    for (int r = 0; r < rows; ++r) s += part[int64_t(r) * n_k + j];
    ns[j] = s / float(H);
  }
}

// ----------------------------------------------------------------- backward
// Dq[h, i] = sum_c G[i,h,c] out[i,h,c].  For bf16 the forward's fp32 copy of
// out (TO = float) is used when there is one: D enters dS = P (dP - D) where
// the two terms nearly cancel for peaked rows, and the bf16-rounded out alone
// moves dQ by a few percent there.
template <typename TO, typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_dense_rowstat(const TO* __restrict__ out,
                                                          const T* __restrict__ g, int32_t n_q,
                                                          int32_t H, float* __restrict__ dq) {
  const int64_t n = int64_t(n_q) * H;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < n;
       t += int64_t(gridDim.x) * blockDim.x) {
    float o[DH], gg[DH];
    load_row<TO, DH>(out + t * DH, o);
    load_row<T, DH>(g + t * DH, gg);
    const int64_t i = t / H, h = t % H;
    dq[h * n_q + i] = dotv<DH>(o, gg);
  }
}

// Key-major pass: lane owns key row (lane % 16) of the wave and 8 queries of
// each 32-query tile.  grid = (ceil(n_k / 64), H).
template <typename T, int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_dense_bwd_kv(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ g, const float* __restrict__ lse, const float* __restrict__ dsum,
    int32_t n_q, int32_t n_k, int32_t H, float scale, DropoutMask dm, T* __restrict__ grad_k,
    T* __restrict__ grad_v) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int grp = lane >> 4;
  const int h = blockIdx.y;
  const int64_t kj = int64_t(blockIdx.x) * kRowsPerBlock + wave * kRows + r;
  const bool k_ok = kj < n_k;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  float kr[DH], vr[DH], dk[DH], dv[DH];
  if (k_ok) {
    load_row<T, DH>(k + (kj * H + h) * DH, kr);
    load_row<T, DH>(v + (kj * H + h) * DH, vr);
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) kr[c] = vr[c] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) dk[c] = dv[c] = 0.f;
  const float* lse_h = lse + int64_t(h) * n_q;
  const float* ds_h = dsum + int64_t(h) * n_q;
  for (int qb = grp * kColsPerLane; qb < n_q; qb += kTile) {
#pragma unroll 2
    for (int i = 0; i < kColsPerLane; ++i) {
      const int64_t qi = qb + i;
      if (qi < n_q) {
        float qs[DH], gi[DH];
        load_row<T, DH>(q + (qi * H + h) * DH, qs);
        load_row<T, DH>(g + (qi * H + h) * DH, gi);
#pragma unroll
        for (int c = 0; c < DH; ++c) qs[c] *= scale;
        const float p = __expf(dotv<DH>(qs, kr) - lse_h[qi]);
        float m = 1.f;
        if constexpr (DROP)
          m = drop_scale(dm, drop_word(dm, uint32_t(qi), uint32_t(kj)), uint32_t(kj));
        const float ds = p * (m * dotv<DH>(gi, vr) - ds_h[qi]);
        const float pm = p * m;
#pragma unroll
        for (int c = 0; c < DH; ++c) {
          dv[c] = fmaf(pm, gi[c], dv[c]);
          dk[c] = fmaf(ds, qs[c], dk[c]);
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dk[c] += shfl_xor(dk[c], 16);
    dk[c] += shfl_xor(dk[c], 32);
    dv[c] += shfl_xor(dv[c], 16);
    dv[c] += shfl_xor(dv[c], 32);
  }
  if (k_ok && grp == 0) {
    store_row<T, DH>(grad_k + (kj * H + h) * DH, dk);
    store_row<T, DH>(grad_v + (kj * H + h) * DH, dv);
  }
}

// Query-major pass: lane owns query row (lane % 16) and 8 keys per tile.
template <typename T, int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_dense_bwd_q(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ g, const float* __restrict__ lse, const float* __restrict__ dsum,
    int32_t n_q, int32_t n_k, int32_t H, float scale, DropoutMask dm, T* __restrict__ grad_q) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int grp = lane >> 4;
  const int h = blockIdx.y;
  const int64_t qi = int64_t(blockIdx.x) * kRowsPerBlock + wave * kRows + r;
  const bool q_ok = qi < n_q;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  float qs[DH], gi[DH], dq[DH];
  float L = 0.f, Dq = 0.f;
  if (q_ok) {
    load_row<T, DH>(q + (qi * H + h) * DH, qs);
    load_row<T, DH>(g + (qi * H + h) * DH, gi);
#pragma unroll
    for (int c = 0; c < DH; ++c) qs[c] *= scale;
    L = lse[int64_t(h) * n_q + qi];
    Dq = dsum[int64_t(h) * n_q + qi];
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) qs[c] = gi[c] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) dq[c] = 0.f;
  for (int kb = grp * kColsPerLane; kb < n_k; kb += kTile) {
#pragma unroll 2
    for (int i = 0; i < kColsPerLane; ++i) {
      const int64_t kj = kb + i;
      if (kj < n_k) {
        float kr[DH], vr[DH];
        load_row<T, DH>(k + (kj * H + h) * DH, kr);
        load_row<T, DH>(v + (kj * H + h) * DH, vr);
        const float p = __expf(dotv<DH>(qs, kr) - L);
        float m = 1.f;
        if constexpr (DROP)
          m = drop_scale(dm, drop_word(dm, uint32_t(qi), uint32_t(kj)), uint32_t(kj));
        const float ds = p * (m * dotv<DH>(gi, vr) - Dq);
#pragma unroll
        for (int c = 0; c < DH; ++c) dq[c] = fmaf(ds, kr[c], dq[c]);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dq[c] += shfl_xor(dq[c], 16);
    dq[c] += shfl_xor(dq[c], 32);
    dq[c] *= scale;
  }
  if (q_ok && grp == 0) store_row<T, DH>(grad_q + (qi * H + h) * DH, dq);
}

// ------------------------------------------------------------------ host side
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline int64_t qblocks(int32_t n) { return (int64_t(n) + kRowsPerBlock - 1) / kRowsPerBlock; }

size_t fwd_ws(int32_t n_q, int32_t n_k, int32_t H) {
  return align256(size_t(qblocks(n_q)) * H * size_t(n_k) * 4);
}
size_t bwd_ws(int32_t n_q, int32_t H) { return align256(size_t(n_q) * H * 4); }

template <typename T, int DH>
int launch_fwd(const void* q, const void* k, const void* v, int n_q, int n_k, int H, float scale,
               const DropoutMask* dm, void* out, float* out32, float* lse, float* ns, char* ws,
               hipStream_t st) {
  if (n_q == 0) return NGT_OK;
  float* part = ns ? reinterpret_cast<float*>(ws) : nullptr;
  dim3 grid(static_cast<unsigned>(qblocks(n_q)), static_cast<unsigned>(H));
  {
    KernelTimer timer_("dense_fwd", st);
    const DropoutMask m = dm ? *dm : DropoutMask{};
    if (dm)
      hipLaunchKernelGGL((k_dense_fwd<T, DH, true>), grid, dim3(kBlock), 0, st,
                         static_cast<const T*>(q), static_cast<const T*>(k),
                         static_cast<const T*>(v), n_q, n_k, H, scale, m, static_cast<T*>(out),
                         out32, lse, part);
    else
      hipLaunchKernelGGL((k_dense_fwd<T, DH, false>), grid, dim3(kBlock), 0, st,
                         static_cast<const T*>(q), static_cast<const T*>(k),
                         static_cast<const T*>(v), n_q, n_k, H, scale, m, static_cast<T*>(out),
                         out32, lse, part);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (ns && n_k > 0) {
    const int rows = static_cast<int>(qblocks(n_q) * H);
    hipLaunchKernelGGL(k_dense_scores, dim3((n_k + kBlock - 1) / kBlock), dim3(kBlock), 0, st,
                       part, rows, n_k, H, ns);
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

template <typename T, int DH>
int launch_bwd(const void* q, const void* k, const void* v, const void* out, const float* out32,
               const void* g, const float* lse, int n_q, int n_k, int H, float scale,
               const DropoutMask* dm, void* gq, void* gk, void* gv, char* ws, hipStream_t st) {
  const DropoutMask m = dm ? *dm : DropoutMask{};
  float* dsum = reinterpret_cast<float*>(ws);
  if (n_q > 0) {
    int64_t blocks = (int64_t(n_q) * H + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    {
      KernelTimer timer_("dense_rowstat", st);
      if (out32)
        hipLaunchKernelGGL((k_dense_rowstat<float, T, DH>), dim3(int(blocks)), dim3(kBlock), 0, st,
                           out32, static_cast<const T*>(g), n_q, H, dsum);
      else
        hipLaunchKernelGGL((k_dense_rowstat<T, T, DH>), dim3(int(blocks)), dim3(kBlock), 0, st,
                           static_cast<const T*>(out), static_cast<const T*>(g), n_q, H, dsum);
      NGT_HIP_CHECK(hipGetLastError());
    }
  }
  if (n_k > 0) {
    dim3 grid(static_cast<unsigned>(qblocks(n_k)), static_cast<unsigned>(H));
    {
      KernelTimer timer_("dense_bwd_kv", st);
      if (dm)
        hipLaunchKernelGGL((k_dense_bwd_kv<T, DH, true>), grid, dim3(kBlock), 0, st,
                           static_cast<const T*>(q), static_cast<const T*>(k),
                           static_cast<const T*>(v), static_cast<const T*>(g), lse, dsum, n_q,
                           n_k, H, scale, m, static_cast<T*>(gk), static_cast<T*>(gv));
      else
        hipLaunchKernelGGL((k_dense_bwd_kv<T, DH, false>), grid, dim3(kBlock), 0, st,
                           static_cast<const T*>(q), static_cast<const T*>(k),
                           static_cast<const T*>(v), static_cast<const T*>(g), lse, dsum, n_q,
                           n_k, H, scale, m, static_cast<T*>(gk), static_cast<T*>(gv));
      NGT_HIP_CHECK(hipGetLastError());
    }
  }
  if (n_q > 0) {
    dim3 grid(static_cast<unsigned>(qblocks(n_q)), static_cast<unsigned>(H));
    {
      KernelTimer timer_("dense_bwd_q", st);
      if (dm)
        hipLaunchKernelGGL((k_dense_bwd_q<T, DH, true>), grid, dim3(kBlock), 0, st,
                           static_cast<const T*>(q), static_cast<const T*>(k),
                           static_cast<const T*>(v), static_cast<const T*>(g), lse, dsum, n_q,
                           n_k, H, scale, m, static_cast<T*>(gq));
      else
        hipLaunchKernelGGL((k_dense_bwd_q<T, DH, false>), grid, dim3(kBlock), 0, st,
                           static_cast<const T*>(q), static_cast<const T*>(k),
                           static_cast<const T*>(v), static_cast<const T*>(g), lse, dsum, n_q,
                           n_k, H, scale, m, static_cast<T*>(gq));
      NGT_HIP_CHECK(hipGetLastError());
    }
  }
  return NGT_OK;
}

template <typename T, int DH>
struct FwdOp {
  template <typename... A>
  static int run(A&&... a) {
    return launch_fwd<T, DH>(std::forward<A>(a)...);
  }
};
template <typename T, int DH>
struct BwdOp {
  template <typename... A>
  static int run(A&&... a) {
    return launch_bwd<T, DH>(std::forward<A>(a)...);
  }
};

template <template <typename, int> class F, typename... Args>
int dispatch(int dtype, int d, Args&&... args) {
#define NGT_CASE(DH)                                                         \
  case DH:                                                                   \
    return dtype == NGT_F32 ? F<float, DH>::run(std::forward<Args>(args)...) \
                            : F<bf16_t, DH>::run(std::forward<Args>(args)...);
  switch (d) {
    NGT_CASE(8)
    NGT_CASE(16)
    NGT_CASE(24)
    NGT_CASE(32)
    NGT_CASE(64)
    default:
      return set_error(NGT_ERR_UNSUPPORTED, "dense: head_dim=%d has no kernel", d);
  }
#undef NGT_CASE
}

int check_args(const char* fn, int dtype, int n_q, int n_k, int H, int d) {
  if (dtype != NGT_F32 && dtype != NGT_BF16)
    return set_error(NGT_ERR_ARG, "%s: unknown dtype %d", fn, dtype);
  if (n_q < 0 || n_k < 0 || H < 1 || H > 65535)
    return set_error(NGT_ERR_ARG, "%s: bad sizes n_q=%d n_k=%d H=%d", fn, n_q, n_k, H);
  if (d != 8 && d != 16 && d != 24 && d != 32 && d != 64)
    return set_error(NGT_ERR_UNSUPPORTED, "%s: head_dim=%d (supported 8,16,24,32,64)", fn, d);
  return NGT_OK;
}

// Dropout parameters from p and the seed; *on = false for p = 0.
int make_dropout(const char* fn, float p, uint64_t seed, int n_q, int n_k, DropoutMask* dm,
                 bool* on) {
  *on = false;
  if (!(p >= 0.f && p <= 1.f))
    return set_error(NGT_ERR_ARG, "%s: dropout_p=%g outside [0, 1]", fn, double(p));
  if (p == 0.f) return NGT_OK;
  const uint64_t words = uint64_t(n_q) * ((uint64_t(n_k) + 1) / 2);
  if (words > (uint64_t(1) << 32))
    return set_error(NGT_ERR_UNSUPPORTED,
                     "%s: dropout needs n_q * ceil(n_k / 2) <= 2^32 (n_q=%d n_k=%d)", fn, n_q, n_k);
  dm->seed = seed;
  dm->head_key = 0;
  dm->n_kp = static_cast<uint32_t>((uint64_t(n_k) + 1) / 2);
  if (p >= 1.f) {  // everything dropped: keep-all mask with scale 0
    dm->thr = 0;
    dm->scale = 0.f;
  } else {
    dm->thr = static_cast<uint32_t>(lrint(double(p) * 65536.0));
    dm->scale = static_cast<float>(1.0 / (1.0 - double(p)));
  }
  *on = true;
  return NGT_OK;
}

// The bf16 path runs on the matrix cores (ngt_dense_mfma.hip) for d <= 32;
// NGT_DENSE_VALU=1 selects the vector-ALU kernels instead (for comparison).
bool use_mfma(int dtype, int d) {
  static const bool valu = getenv("NGT_DENSE_VALU") != nullptr;
  return dtype == NGT_BF16 && mfma_dense_supported(d) && !valu;
}

int rowstat_bf16(int d, const void* out, const float* out32, const void* g, int n_q, int H,
                 float* dsum, hipStream_t st) {
  int64_t blocks = (int64_t(n_q) * H + kBlock - 1) / kBlock;
  if (blocks > 65536) blocks = 65536;
  KernelTimer timer_("dense_rowstat", st);
#define NGT_RS(DH)                                                                             \
  case DH:                                                                                     \
    if (out32)                                                                                 \
      hipLaunchKernelGGL((k_dense_rowstat<float, bf16_t, DH>), dim3(int(blocks)), dim3(kBlock), \
                         0, st, out32, static_cast<const bf16_t*>(g), n_q, H, dsum);           \
    else                                                                                       \
      hipLaunchKernelGGL((k_dense_rowstat<bf16_t, bf16_t, DH>), dim3(int(blocks)),              \
                         dim3(kBlock), 0, st, static_cast<const bf16_t*>(out),                  \
                         static_cast<const bf16_t*>(g), n_q, H, dsum);                          \
    break;
  switch (d) {
    NGT_RS(8)
    NGT_RS(16)
    NGT_RS(24)
    NGT_RS(32)
    default:
      return set_error(NGT_ERR_UNSUPPORTED, "rowstat: head_dim %d", d);
  }
#undef NGT_RS
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_dense_workspace_bytes(int32_t n_q, int32_t n_k, int32_t n_heads,
                                         int32_t head_dim, size_t* fwd_bytes, size_t* bwd_bytes) {
  const int rc = check_args("ngt_dense_workspace_bytes", NGT_F32, n_q, n_k, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (fwd_bytes) *fwd_bytes = fwd_ws(n_q, n_k, n_heads);
  if (bwd_bytes) *bwd_bytes = bwd_ws(n_q, n_heads);
  return NGT_OK;
}

extern "C" int ngt_dense_fwd(int dtype, const void* q, const void* k, const void* v, int32_t n_q,
                             int32_t n_k, int32_t n_heads, int32_t head_dim, float scale,
                             float dropout_p, uint64_t seed, void* out, float* out_f32,
                             float* lse, float* node_score, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc = check_args("ngt_dense_fwd", dtype, n_q, n_k, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  DropoutMask dmv{};
  bool drop = false;
  NGT_CHECK_OK(make_dropout("ngt_dense_fwd", dropout_p, seed, n_q, n_k, &dmv, &drop));
  const DropoutMask* dm = drop ? &dmv : nullptr;
  if (n_q > 0 && (!q || !out || !lse)) return set_error(NGT_ERR_ARG, "ngt_dense_fwd: null q/out/lse");
  if (n_k > 0 && (!k || !v)) return set_error(NGT_ERR_ARG, "ngt_dense_fwd: null k/v");
  if (node_score && n_q > 0) {
    const size_t need = fwd_ws(n_q, n_k, n_heads);
    if (!workspace || workspace_bytes < need)
      return set_error(NGT_ERR_WORKSPACE, "ngt_dense_fwd: workspace %zu < %zu", workspace_bytes,
                       need);
  }
  if (node_score && n_q == 0 && n_k > 0)
    NGT_HIP_CHECK(hipMemsetAsync(node_score, 0, size_t(n_k) * 4, static_cast<hipStream_t>(stream)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_mfma(dtype, head_dim)) {
    if (n_q == 0) return NGT_OK;
    float* part = node_score ? static_cast<float*>(workspace) : nullptr;
    rc = mfma_dense_fwd(head_dim, q, k, v, n_q, n_k, n_heads, scale, dm, out, out_f32, lse, part,
                        st);
    if (rc != NGT_OK || !node_score || n_k == 0) return rc;
    hipLaunchKernelGGL(k_dense_scores, dim3((n_k + kBlock - 1) / kBlock), dim3(kBlock), 0, st,
                       part, n_heads, n_k, n_heads, node_score);
    NGT_HIP_CHECK(hipGetLastError());
    return NGT_OK;
  }
  return dispatch<FwdOp>(dtype, head_dim, q, k, v, int(n_q), int(n_k), int(n_heads), scale, dm,
                         out, out_f32, lse, node_score, static_cast<char*>(workspace), st);
}

extern "C" int ngt_dense_bwd(int dtype, const void* q, const void* k, const void* v,
                             const void* out, const float* out_f32, const void* grad_out,
                             const float* lse, int32_t n_q,
                             int32_t n_k, int32_t n_heads, int32_t head_dim, float scale,
                             float dropout_p, uint64_t seed, void* grad_q, void* grad_k,
                             void* grad_v, void* workspace, size_t workspace_bytes,
                             void* stream) {
  int rc = check_args("ngt_dense_bwd", dtype, n_q, n_k, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  DropoutMask dmv{};
  bool drop = false;
  NGT_CHECK_OK(make_dropout("ngt_dense_bwd", dropout_p, seed, n_q, n_k, &dmv, &drop));
  const DropoutMask* dm = drop ? &dmv : nullptr;
  if (n_q > 0 && (!q || (!out && !out_f32) || !grad_out || !lse || !grad_q))
    return set_error(NGT_ERR_ARG, "ngt_dense_bwd: null query-side pointer");
  if (n_k > 0 && (!k || !v || !grad_k || !grad_v))
    return set_error(NGT_ERR_ARG, "ngt_dense_bwd: null key-side pointer");
  const size_t need = bwd_ws(n_q, n_heads);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(NGT_ERR_WORKSPACE, "ngt_dense_bwd: workspace %zu < %zu", workspace_bytes,
                     need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_mfma(dtype, head_dim)) {
    float* dsum = static_cast<float*>(workspace);
    if (n_q > 0) {
      rc = rowstat_bf16(head_dim, out, out_f32, grad_out, n_q, n_heads, dsum, st);
      if (rc != NGT_OK) return rc;
    }
    return mfma_dense_bwd(head_dim, q, k, v, grad_out, lse, dsum, n_q, n_k, n_heads, scale, dm,
                          grad_q, grad_k, grad_v, st);
  }
  return dispatch<BwdOp>(dtype, head_dim, q, k, v, out, out_f32, grad_out, lse, int(n_q), int(n_k),
                         int(n_heads), scale, dm, grad_q, grad_k, grad_v,
                         static_cast<char*>(workspace), st);
}
