// LayerNorm over the last dimension, forward and backward, fp32 math on fp32
// or bf16 rows, with the output in either type.
//
// The encoder's LayerNorms (graphormer_dist_node_level.py:176-206 pre-LN
// self_attention_norm / ffn_norm and final_ln; the GT twin's post-LN
// layer_norm1/2, gt_dist_node_level_single_window.py:305-353).  Under bf16
// autocast torch runs each one as a cast of the bf16 residual stream to fp32,
// the fp32 LayerNorm, and a cast of its output back to bf16 for the next
// linear layer; its backward takes three more kernels.  Here a wave owns a row:
// y = (x - mean) * rstd * gamma + beta with mean and the variance of the
// deviations from two passes over the row held in registers, written straight
// in the consumer's type.  The backward is
//   dx = rstd * (g - mean_c(g) - xhat * mean_c(g * xhat)),  g = dy * gamma,
// per row, and dgamma = sum_rows dy * xhat, dbeta = sum_rows dy as per-block
// column partials added in block order by a second pass (deterministic).
#include "ngt_common.h"

#include <math.h>

#include <type_traits>

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxQ = 8;  // 4-element groups per lane: n_cols <= 64 * 4 * 8 = 2048
constexpr int kRowsPerBwdBlock = 32;

template <typename T>
__device__ __forceinline__ void load4f(const T* p, float (&v)[4]);
template <>
__device__ __forceinline__ void load4f<float>(const float* p, float (&v)[4]) {
  const float4 w = *reinterpret_cast<const float4*>(p);
  v[0] = w.x;
  v[1] = w.y;
  v[2] = w.z;
  v[3] = w.w;
}
template <>
__device__ __forceinline__ void load4f<bf16_t>(const bf16_t* p, float (&v)[4]) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  v[0] = bf16_to_f32(static_cast<uint16_t>(w.x & 0xffffu));
  v[1] = bf16_to_f32(static_cast<uint16_t>(w.x >> 16));
  v[2] = bf16_to_f32(static_cast<uint16_t>(w.y & 0xffffu));
  v[3] = bf16_to_f32(static_cast<uint16_t>(w.y >> 16));
}

template <typename T>
__device__ __forceinline__ void store4f(T* p, const float (&v)[4]);
template <>
__device__ __forceinline__ void store4f<float>(float* p, const float (&v)[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4f<bf16_t>(bf16_t* p, const float (&v)[4]) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

// grid = ceil(n_rows / 4); wave w of block b owns row 4b + w.
// Q = 4-element groups per lane (ceil(n_cols / 256)), a template constant so
// that a row's values stay in exactly the registers it needs.
template <typename TI, typename TO, int Q>
__global__ __launch_bounds__(kBlock) void k_ln_fwd(const TI* __restrict__ x, int64_t n_rows,
                                                   int32_t n_cols, const float* __restrict__ gamma,
                                                   const float* __restrict__ beta, float eps,
                                                   TO* __restrict__ y, float* __restrict__ mean,
                                                   float* __restrict__ rstd) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // whole wave; no block barrier follows
  const int nq = n_cols / 4;
  const TI* xr = x + row * n_cols;
  float v[Q][4];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
      load4f<TI>(xr + 4 * qd, v[j]);
      s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
    }
  }
  const float mu = wave_sum(s) / float(n_cols);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float dlt = v[j][c] - mu;
        ss = fmaf(dlt, dlt, ss);
      }
    }
  }
  const float var = wave_sum(ss) / float(n_cols);
  const float rs = 1.0f / sqrtf(var + eps);
  TO* yr = y + row * n_cols;
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int col = 4 * qd + c;
        o[c] = fmaf((v[j][c] - mu) * rs, gamma[col], beta[col]);
      }
      store4f<TO>(yr + 4 * qd, o);
    }
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
}

// Rows 32b .. 32b+31: dx per row (one wave at a time per row), and the
// block's column partials of dgamma / dbeta, part[b][0..n_cols) and
// part[b][n_cols..2 n_cols).
template <typename TI, typename TG, int Q>
__global__ __launch_bounds__(kBlock) void k_ln_bwd(const TI* __restrict__ x,
                                                   const TG* __restrict__ dy, int64_t n_rows,
                                                   int32_t n_cols, const float* __restrict__ gamma,
                                                   const float* __restrict__ mean,
                                                   const float* __restrict__ rstd,
                                                   TI* __restrict__ dx, float* __restrict__ part) {
  extern __shared__ float red[];  // [kWaves][2 * n_cols]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int nq = n_cols / 4;
  float dg[Q][4], db[Q][4];
#pragma unroll
  for (int j = 0; j < Q; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) dg[j][c] = db[j][c] = 0.f;
  const int64_t r0 = int64_t(blockIdx.x) * kRowsPerBwdBlock;
  for (int rr = wave; rr < kRowsPerBwdBlock; rr += kWaves) {
    const int64_t row = r0 + rr;
    if (row >= n_rows) break;
    const float mu = mean[row], rs = rstd[row];
    float xh[Q][4], g[Q][4];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      const int qd = lane + j * kWave;
      if (qd < nq) {
        float xv[4], dv[4];
        load4f<TI>(x + row * n_cols + 4 * qd, xv);
        load4f<TG>(dy + row * n_cols + 4 * qd, dv);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          xh[j][c] = (xv[c] - mu) * rs;
          g[j][c] = dv[c] * gamma[4 * qd + c];
          s1 += g[j][c];
          s2 = fmaf(g[j][c], xh[j][c], s2);
          dg[j][c] = fmaf(dv[c], xh[j][c], dg[j][c]);
          db[j][c] += dv[c];
        }
      }
    }
    const float c1 = wave_sum(s1) / float(n_cols);
    const float c2 = wave_sum(s2) / float(n_cols);
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      const int qd = lane + j * kWave;
      if (qd < nq) {
        float o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = rs * (g[j][c] - c1 - xh[j][c] * c2);
        store4f<TI>(dx + row * n_cols + 4 * qd, o);
      }
    }
  }
  // block column partials: waves added in wave order through LDS
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        red[wave * 2 * n_cols + 4 * qd + c] = dg[j][c];
        red[wave * 2 * n_cols + n_cols + 4 * qd + c] = db[j][c];
      }
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < 2 * n_cols; t += kBlock) {
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) a += red[w * 2 * n_cols + t];
    part[int64_t(blockIdx.x) * 2 * n_cols + t] = a;
  }
}

// dgamma / dbeta = sums of the block partials: 32 lanes per column each add
// blocks b = lane mod 32 in order, then the 32 lane sums in lane order (8
// lanes left each with 128 serial loads for 32,768 rows: 38 us).
constexpr int kRedLanes = 32;
constexpr int kRedCols = kBlock / kRedLanes;
__global__ __launch_bounds__(kBlock) void k_ln_bwd_reduce(const float* __restrict__ part,
                                                          int32_t n_blocks, int32_t n_cols,
                                                          float* __restrict__ dgamma,
                                                          float* __restrict__ dbeta) {
  __shared__ float red[kRedLanes][kRedCols];
  const int cl = threadIdx.x % kRedCols;
  const int ln = threadIdx.x / kRedCols;
  const int t = blockIdx.x * kRedCols + cl;
  float a = 0.f;
  if (t < 2 * n_cols)
    for (int b = ln; b < n_blocks; b += kRedLanes) a += part[int64_t(b) * 2 * n_cols + t];
  red[ln][cl] = a;
  __syncthreads();
  if (ln != 0 || t >= 2 * n_cols) return;
  float u = 0.f;
#pragma unroll
  for (int q = 0; q < kRedLanes; ++q) u += red[q][cl];
  if (t < n_cols) {
    if (dgamma) dgamma[t] = u;
  } else if (dbeta) {
    dbeta[t - n_cols] = u;
  }
}

int check(const char* fn, int dt, int64_t n_rows, int n_cols) {
  if (dt != NGT_F32 && dt != NGT_BF16) return set_error(NGT_ERR_ARG, "%s: unknown dtype %d", fn, dt);
  if (n_rows < 0 || n_cols < 4 || n_cols % 4 || n_cols > 64 * 4 * kMaxQ)
    return set_error(NGT_ERR_UNSUPPORTED,
                     "%s: n_cols=%d (a multiple of 4 in 4..%d), n_rows=%lld", fn, n_cols,
                     64 * 4 * kMaxQ, static_cast<long long>(n_rows));
  return NGT_OK;
}

// Address bits that must be clear in a row base: each lane moves 4 elements
// per access (16 bytes for fp32, 8 for bf16); n_cols % 4 == 0 keeps every row
// at that alignment once the base is.
inline uintptr_t row_align(int dt) { return dt == NGT_F32 ? 15 : 7; }
inline bool misaligned(const void* p, int dt) {
  return (reinterpret_cast<uintptr_t>(p) & row_align(dt)) != 0;
}

// Smallest supported Q with 64 * 4 * Q >= n_cols.
inline int quads_for(int n_cols) {
  const int q = (n_cols + 255) / 256;
  return q <= 1 ? 1 : q <= 2 ? 2 : q <= 3 ? 3 : q <= 4 ? 4 : q <= 6 ? 6 : 8;
}

inline int64_t bwd_blocks(int64_t n_rows) {
  return (n_rows + kRowsPerBwdBlock - 1) / kRowsPerBwdBlock;
}


// ----------------------------------------------- residual add + dropout + LN
// The pre-LN sub-layer boundary of the Graphormer layer
// (graphormer_dist_node_level.py:196-206):  s = x + dropout_p(y), out = LN(s),
// both kept (s is the residual stream).  s is rounded to T before the
// LayerNorm reads it, as the unfused sequence does.  The dropout bit of
// element (row, col) is the DropoutMask hash with head 0, query row, key col.
template <typename T>
__device__ __forceinline__ float round_to(float v);
template <>
__device__ __forceinline__ float round_to<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float round_to<bf16_t>(float v) {
  return bf16_to_f32(f32_to_bf16(v));
}

template <bool DROP>
__device__ __forceinline__ void drop4(const DropoutMask& dm, int64_t row, int col, float (&m)[4]) {
  if (!DROP) {
    m[0] = m[1] = m[2] = m[3] = 1.f;
    return;
  }
  const uint32_t w0 = drop_word(dm, uint32_t(row), uint32_t(col));
  const uint32_t w1 = drop_word(dm, uint32_t(row), uint32_t(col + 2));
  m[0] = drop_scale(dm, w0, col);
  m[1] = drop_scale(dm, w0, col + 1);
  m[2] = drop_scale(dm, w1, col + 2);
  m[3] = drop_scale(dm, w1, col + 3);
}

template <typename T, typename TO, int Q, bool DROP>
__global__ __launch_bounds__(kBlock) void k_add_ln_fwd(
    const T* __restrict__ x, const T* __restrict__ y, int64_t n_rows, int32_t n_cols,
    DropoutMask dm, const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
    T* __restrict__ sum, TO* __restrict__ out, float* __restrict__ mean,
    float* __restrict__ rstd) {
  if constexpr (DROP) dm = drop_for_head(dm, 0);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // whole wave; no block barrier follows
  const int nq = n_cols / 4;
  float v[Q][4];
  float sacc = 0.f;
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
      float xv[4], yv[4], m[4];
      load4f<T>(x + row * n_cols + 4 * qd, xv);
      load4f<T>(y + row * n_cols + 4 * qd, yv);
      drop4<DROP>(dm, row, 4 * qd, m);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[j][c] = round_to<T>(xv[c] + yv[c] * m[c]);
        sacc += v[j][c];
      }
      if (sum) store4f<T>(sum + row * n_cols + 4 * qd, v[j]);
    }
  }
  const float mu = wave_sum(sacc) / float(n_cols);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float dlt = v[j][c] - mu;
        ss = fmaf(dlt, dlt, ss);
      }
    }
  }
  const float rs = 1.0f / sqrtf(wave_sum(ss) / float(n_cols) + eps);
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int col = 4 * qd + c;
        o[c] = fmaf((v[j][c] - mu) * rs, gamma[col], beta[col]);
      }
      store4f<TO>(out + row * n_cols + 4 * qd, o);
    }
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
}

// ds = g_sum + LN backward of g_out (at s); dx = ds, dy = ds * mask; block
// partials of dgamma / dbeta as in k_ln_bwd.
template <typename T, typename TG, int Q, bool DROP>
__global__ __launch_bounds__(kBlock) void k_add_ln_bwd(
    const T* __restrict__ sum, const TG* __restrict__ g_out, const T* __restrict__ g_sum,
    int64_t n_rows, int32_t n_cols, DropoutMask dm, const float* __restrict__ gamma,
    const float* __restrict__ mean, const float* __restrict__ rstd, T* __restrict__ dx,
    T* __restrict__ dy, float* __restrict__ part) {
  if constexpr (DROP) dm = drop_for_head(dm, 0);
  extern __shared__ float red[];  // [kWaves][2 * n_cols]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int nq = n_cols / 4;
  float dg[Q][4], db[Q][4];
#pragma unroll
  for (int j = 0; j < Q; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) dg[j][c] = db[j][c] = 0.f;
  const int64_t r0 = int64_t(blockIdx.x) * kRowsPerBwdBlock;
  for (int rr = wave; rr < kRowsPerBwdBlock; rr += kWaves) {
    const int64_t row = r0 + rr;
    if (row >= n_rows) break;
    const float mu = mean[row], rs = rstd[row];
    float xh[Q][4], g[Q][4];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      const int qd = lane + j * kWave;
      if (qd < nq) {
        float sv[4], dv[4];
        load4f<T>(sum + row * n_cols + 4 * qd, sv);
        load4f<TG>(g_out + row * n_cols + 4 * qd, dv);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          xh[j][c] = (sv[c] - mu) * rs;
          g[j][c] = dv[c] * gamma[4 * qd + c];
          s1 += g[j][c];
          s2 = fmaf(g[j][c], xh[j][c], s2);
          dg[j][c] = fmaf(dv[c], xh[j][c], dg[j][c]);
          db[j][c] += dv[c];
        }
      }
    }
    const float c1 = wave_sum(s1) / float(n_cols);
    const float c2 = wave_sum(s2) / float(n_cols);
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      const int qd = lane + j * kWave;
      if (qd < nq) {
        float gs[4] = {0.f, 0.f, 0.f, 0.f}, m[4], o[4], oy[4];
        if (g_sum) load4f<T>(g_sum + row * n_cols + 4 * qd, gs);
        drop4<DROP>(dm, row, 4 * qd, m);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          o[c] = gs[c] + rs * (g[j][c] - c1 - xh[j][c] * c2);
          oy[c] = o[c] * m[c];
        }
        store4f<T>(dx + row * n_cols + 4 * qd, o);
        store4f<T>(dy + row * n_cols + 4 * qd, oy);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const int qd = lane + j * kWave;
    if (qd < nq) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        red[wave * 2 * n_cols + 4 * qd + c] = dg[j][c];
        red[wave * 2 * n_cols + n_cols + 4 * qd + c] = db[j][c];
      }
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < 2 * n_cols; t += kBlock) {
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) a += red[w * 2 * n_cols + t];
    part[int64_t(blockIdx.x) * 2 * n_cols + t] = a;
  }
}

// Dropout parameters of the fused op (p in [0, 1)); *on = false for p = 0.
int add_ln_dropout(const char* fn, float p, uint64_t seed, const uint64_t* seed_dev,
                   int64_t n_rows, int n_cols, DropoutMask* dm, bool* on) {
  *on = false;
  if (!(p >= 0.f && p < 1.f))
    return set_error(NGT_ERR_ARG, "%s: dropout_p=%g outside [0, 1)", fn, double(p));
  if (p == 0.f) return NGT_OK;
  const uint64_t n_kp = (uint64_t(n_cols) + 1) / 2;
  if (uint64_t(n_rows) * n_kp > (uint64_t(1) << 32))
    return set_error(NGT_ERR_UNSUPPORTED, "%s: dropout needs n_rows * n_cols / 2 <= 2^32", fn);
  dm->seed = seed;
  dm->seed_dev = seed_dev;
  dm->head_key = drop_head_key(seed, 0);
  dm->n_kp = static_cast<uint32_t>(n_kp);
  dm->thr = static_cast<uint32_t>(lrint(double(p) * 65536.0));
  dm->scale = static_cast<float>(1.0 / (1.0 - double(p)));
  *on = true;
  return NGT_OK;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_layernorm_fwd(int in_dtype, const void* x, int64_t n_rows, int32_t n_cols,
                                 const float* gamma, const float* beta, float eps, int out_dtype,
                                 void* y, float* mean, float* rstd, void* stream) {
  NGT_CHECK_OK(check("ngt_layernorm_fwd", in_dtype, n_rows, n_cols));
  NGT_CHECK_OK(check("ngt_layernorm_fwd", out_dtype, n_rows, n_cols));
  if (n_rows == 0) return NGT_OK;
  if (!x || !gamma || !beta || !y || !mean || !rstd)
    return set_error(NGT_ERR_ARG, "ngt_layernorm_fwd: null pointer");
  if (misaligned(x, in_dtype) || misaligned(y, out_dtype))
    return set_error(NGT_ERR_ARG,
                     "ngt_layernorm_fwd: rows must be 16-byte (fp32) / 8-byte (bf16) aligned");
  if (!(eps >= 0.f)) return set_error(NGT_ERR_ARG, "ngt_layernorm_fwd: eps must be >= 0");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t blocks = (n_rows + kWaves - 1) / kWaves;
  if (blocks > 0x7fffffff) return set_error(NGT_ERR_UNSUPPORTED, "ngt_layernorm_fwd: too many rows");
  KernelTimer timer_("layernorm_fwd", st);
  const int nq = quads_for(n_cols);
#define NGT_LN_FQ(TI, TO, Q)                                                                 \
  case Q:                                                                                    \
    hipLaunchKernelGGL((k_ln_fwd<TI, TO, Q>), dim3(unsigned(blocks)), dim3(kBlock), 0, st,   \
                       static_cast<const TI*>(x), n_rows, n_cols, gamma, beta, eps,          \
                       static_cast<TO*>(y), mean, rstd);                                     \
    break;
#define NGT_LN_F(TI, TO)                                                                     \
  switch (nq) {                                                                              \
    NGT_LN_FQ(TI, TO, 1) NGT_LN_FQ(TI, TO, 2) NGT_LN_FQ(TI, TO, 3) NGT_LN_FQ(TI, TO, 4)      \
    NGT_LN_FQ(TI, TO, 6) NGT_LN_FQ(TI, TO, 8)                                                \
  }
  if (in_dtype == NGT_F32 && out_dtype == NGT_F32) {
    NGT_LN_F(float, float)
  } else if (in_dtype == NGT_F32) {
    NGT_LN_F(float, bf16_t)
  } else if (out_dtype == NGT_F32) {
    NGT_LN_F(bf16_t, float)
  } else {
    NGT_LN_F(bf16_t, bf16_t)
  }
#undef NGT_LN_F
#undef NGT_LN_FQ
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_layernorm_bwd_workspace_bytes(int64_t n_rows, int32_t n_cols, size_t* bytes) {
  NGT_CHECK_OK(check("ngt_layernorm_bwd_workspace_bytes", NGT_F32, n_rows, n_cols));
  if (!bytes) return set_error(NGT_ERR_ARG, "ngt_layernorm_bwd_workspace_bytes: null bytes");
  *bytes = size_t(bwd_blocks(n_rows)) * 2 * n_cols * 4;
  return NGT_OK;
}

extern "C" int ngt_layernorm_bwd(int in_dtype, const void* x, int grad_dtype, const void* dy,
                                 int64_t n_rows, int32_t n_cols, const float* gamma,
                                 const float* mean, const float* rstd, void* dx, float* dgamma,
                                 float* dbeta, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  NGT_CHECK_OK(check("ngt_layernorm_bwd", in_dtype, n_rows, n_cols));
  NGT_CHECK_OK(check("ngt_layernorm_bwd", grad_dtype, n_rows, n_cols));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nb = bwd_blocks(n_rows);
  if (nb > 0) {
    if (!x || !dy || !gamma || !mean || !rstd || !dx)
      return set_error(NGT_ERR_ARG, "ngt_layernorm_bwd: null pointer");
    if (misaligned(x, in_dtype) || misaligned(dy, grad_dtype) || misaligned(dx, in_dtype))
      return set_error(NGT_ERR_ARG,
                       "ngt_layernorm_bwd: rows must be 16-byte (fp32) / 8-byte (bf16) aligned");
    const size_t need = size_t(nb) * 2 * n_cols * 4;
    if (!workspace || workspace_bytes < need)
      return set_error(NGT_ERR_WORKSPACE, "ngt_layernorm_bwd: workspace %zu < %zu",
                       workspace_bytes, need);
    if (nb > 0x7fffffff) return set_error(NGT_ERR_UNSUPPORTED, "ngt_layernorm_bwd: too many rows");
    KernelTimer timer_("layernorm_bwd", st);
    const size_t lds = size_t(kWaves) * 2 * n_cols * 4;
    float* part = static_cast<float*>(workspace);
    const int nq = quads_for(n_cols);
#define NGT_LN_BQ(TI, TG, Q)                                                                   \
  case Q:                                                                                      \
    hipLaunchKernelGGL((k_ln_bwd<TI, TG, Q>), dim3(unsigned(nb)), dim3(kBlock), lds, st,       \
                       static_cast<const TI*>(x), static_cast<const TG*>(dy), n_rows, n_cols,  \
                       gamma, mean, rstd, static_cast<TI*>(dx), part);                         \
    break;
#define NGT_LN_B(TI, TG)                                                                       \
  switch (nq) {                                                                                \
    NGT_LN_BQ(TI, TG, 1) NGT_LN_BQ(TI, TG, 2) NGT_LN_BQ(TI, TG, 3) NGT_LN_BQ(TI, TG, 4)        \
    NGT_LN_BQ(TI, TG, 6) NGT_LN_BQ(TI, TG, 8)                                                  \
  }
    if (in_dtype == NGT_F32 && grad_dtype == NGT_F32) {
      NGT_LN_B(float, float)
    } else if (in_dtype == NGT_F32) {
      NGT_LN_B(float, bf16_t)
    } else if (grad_dtype == NGT_F32) {
      NGT_LN_B(bf16_t, float)
    } else {
      NGT_LN_B(bf16_t, bf16_t)
    }
#undef NGT_LN_B
#undef NGT_LN_BQ
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (dgamma || dbeta) {
    // no rows: the reduce adds no partials and writes zeros
    hipLaunchKernelGGL(k_ln_bwd_reduce, dim3((2 * n_cols + kRedCols - 1) / kRedCols), dim3(kBlock), 0,
                       st, static_cast<const float*>(workspace), static_cast<int32_t>(nb), n_cols,
                       dgamma, dbeta);
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

extern "C" int ngt_add_layernorm_fwd(int dtype, const void* x, const void* y, int64_t n_rows,
                                     int32_t n_cols, float dropout_p, uint64_t seed,
                                     const uint64_t* seed_dev, const float* gamma,
                                     const float* beta, float eps, void* sum, int out_dtype,
                                     void* out, float* mean, float* rstd, void* stream) {
  NGT_CHECK_OK(check("ngt_add_layernorm_fwd", dtype, n_rows, n_cols));
  NGT_CHECK_OK(check("ngt_add_layernorm_fwd", out_dtype, n_rows, n_cols));
  DropoutMask dm{};
  bool drop = false;
  NGT_CHECK_OK(add_ln_dropout("ngt_add_layernorm_fwd", dropout_p, seed, seed_dev, n_rows, n_cols,
                              &dm, &drop));
  if (n_rows == 0) return NGT_OK;
  if (!x || !y || !gamma || !beta || !out || !mean || !rstd)
    return set_error(NGT_ERR_ARG, "ngt_add_layernorm_fwd: null pointer");
  if (misaligned(x, dtype) || misaligned(y, dtype) || misaligned(sum, dtype) ||
      misaligned(out, out_dtype))
    return set_error(NGT_ERR_ARG,
                     "ngt_add_layernorm_fwd: rows must be 16-byte (fp32) / 8-byte (bf16) aligned");
  if (!(eps >= 0.f)) return set_error(NGT_ERR_ARG, "ngt_add_layernorm_fwd: eps must be >= 0");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t blocks = (n_rows + kWaves - 1) / kWaves;
  if (blocks > 0x7fffffff)
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_add_layernorm_fwd: too many rows");
  const int nq = quads_for(n_cols);
  KernelTimer timer_("add_layernorm_fwd", st);
  auto launch = [&](auto t, auto to, auto dr) {
    using T = decltype(t);
    using TO = decltype(to);
    constexpr bool D = decltype(dr)::value;
    const dim3 g(static_cast<unsigned>(blocks)), b(kBlock);
    const T* xx = static_cast<const T*>(x);
    const T* yy = static_cast<const T*>(y);
    T* ss = static_cast<T*>(sum);
    TO* oo = static_cast<TO*>(out);
    switch (nq) {
      case 1: hipLaunchKernelGGL((k_add_ln_fwd<T, TO, 1, D>), g, b, 0, st, xx, yy, n_rows, n_cols, dm, gamma, beta, eps, ss, oo, mean, rstd); break;
      case 2: hipLaunchKernelGGL((k_add_ln_fwd<T, TO, 2, D>), g, b, 0, st, xx, yy, n_rows, n_cols, dm, gamma, beta, eps, ss, oo, mean, rstd); break;
      case 3: hipLaunchKernelGGL((k_add_ln_fwd<T, TO, 3, D>), g, b, 0, st, xx, yy, n_rows, n_cols, dm, gamma, beta, eps, ss, oo, mean, rstd); break;
      case 4: hipLaunchKernelGGL((k_add_ln_fwd<T, TO, 4, D>), g, b, 0, st, xx, yy, n_rows, n_cols, dm, gamma, beta, eps, ss, oo, mean, rstd); break;
      case 6: hipLaunchKernelGGL((k_add_ln_fwd<T, TO, 6, D>), g, b, 0, st, xx, yy, n_rows, n_cols, dm, gamma, beta, eps, ss, oo, mean, rstd); break;
      default: hipLaunchKernelGGL((k_add_ln_fwd<T, TO, 8, D>), g, b, 0, st, xx, yy, n_rows, n_cols, dm, gamma, beta, eps, ss, oo, mean, rstd); break;
    }
  };
  auto with_drop = [&](auto t, auto to) {
    if (drop)
      launch(t, to, std::true_type{});
    else
      launch(t, to, std::false_type{});
  };
  if (dtype == NGT_F32)
    out_dtype == NGT_F32 ? with_drop(float{}, float{}) : with_drop(float{}, bf16_t{});
  else
    out_dtype == NGT_F32 ? with_drop(bf16_t{}, float{}) : with_drop(bf16_t{}, bf16_t{});
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_add_layernorm_bwd(int dtype, const void* sum, int grad_dtype,
                                     const void* g_out, const void* g_sum, int64_t n_rows,
                                     int32_t n_cols, float dropout_p, uint64_t seed,
                                     const uint64_t* seed_dev, const float* gamma,
                                     const float* mean, const float* rstd, void* dx, void* dy,
                                     float* dgamma, float* dbeta, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  NGT_CHECK_OK(check("ngt_add_layernorm_bwd", dtype, n_rows, n_cols));
  NGT_CHECK_OK(check("ngt_add_layernorm_bwd", grad_dtype, n_rows, n_cols));
  DropoutMask dm{};
  bool drop = false;
  NGT_CHECK_OK(add_ln_dropout("ngt_add_layernorm_bwd", dropout_p, seed, seed_dev, n_rows, n_cols,
                              &dm, &drop));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nb = bwd_blocks(n_rows);
  if (nb > 0) {
    if (!sum || !g_out || !gamma || !mean || !rstd || !dx || !dy)
      return set_error(NGT_ERR_ARG, "ngt_add_layernorm_bwd: null pointer");
    if (misaligned(sum, dtype) || misaligned(g_out, grad_dtype) || misaligned(g_sum, dtype) ||
        misaligned(dx, dtype) || misaligned(dy, dtype))
      return set_error(NGT_ERR_ARG,
                       "ngt_add_layernorm_bwd: rows must be 16-byte (fp32) / 8-byte (bf16) aligned");
    const size_t need = size_t(nb) * 2 * n_cols * 4;
    if (!workspace || workspace_bytes < need)
      return set_error(NGT_ERR_WORKSPACE, "ngt_add_layernorm_bwd: workspace %zu < %zu",
                       workspace_bytes, need);
    if (nb > 0x7fffffff)
      return set_error(NGT_ERR_UNSUPPORTED, "ngt_add_layernorm_bwd: too many rows");
    KernelTimer timer_("add_layernorm_bwd", st);
    const size_t lds = size_t(kWaves) * 2 * n_cols * 4;
    float* part = static_cast<float*>(workspace);
    const int nq = quads_for(n_cols);
    auto launch = [&](auto t, auto tg, auto dr) {
      using T = decltype(t);
      using TG = decltype(tg);
      constexpr bool D = decltype(dr)::value;
      const dim3 g(static_cast<unsigned>(nb)), b(kBlock);
      const T* ss = static_cast<const T*>(sum);
      const TG* go = static_cast<const TG*>(g_out);
      const T* gs = static_cast<const T*>(g_sum);
      T* ox = static_cast<T*>(dx);
      T* oy = static_cast<T*>(dy);
      switch (nq) {
        case 1: hipLaunchKernelGGL((k_add_ln_bwd<T, TG, 1, D>), g, b, lds, st, ss, go, gs, n_rows, n_cols, dm, gamma, mean, rstd, ox, oy, part); break;
        case 2: hipLaunchKernelGGL((k_add_ln_bwd<T, TG, 2, D>), g, b, lds, st, ss, go, gs, n_rows, n_cols, dm, gamma, mean, rstd, ox, oy, part); break;
        case 3: hipLaunchKernelGGL((k_add_ln_bwd<T, TG, 3, D>), g, b, lds, st, ss, go, gs, n_rows, n_cols, dm, gamma, mean, rstd, ox, oy, part); break;
        case 4: hipLaunchKernelGGL((k_add_ln_bwd<T, TG, 4, D>), g, b, lds, st, ss, go, gs, n_rows, n_cols, dm, gamma, mean, rstd, ox, oy, part); break;
        case 6: hipLaunchKernelGGL((k_add_ln_bwd<T, TG, 6, D>), g, b, lds, st, ss, go, gs, n_rows, n_cols, dm, gamma, mean, rstd, ox, oy, part); break;
        default: hipLaunchKernelGGL((k_add_ln_bwd<T, TG, 8, D>), g, b, lds, st, ss, go, gs, n_rows, n_cols, dm, gamma, mean, rstd, ox, oy, part); break;
      }
    };
    auto with_drop = [&](auto t, auto tg) {
      if (drop)
        launch(t, tg, std::true_type{});
      else
        launch(t, tg, std::false_type{});
    };
    if (dtype == NGT_F32)
      grad_dtype == NGT_F32 ? with_drop(float{}, float{}) : with_drop(float{}, bf16_t{});
    else
      grad_dtype == NGT_F32 ? with_drop(bf16_t{}, float{}) : with_drop(bf16_t{}, bf16_t{});
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (dgamma || dbeta) {
    hipLaunchKernelGGL(k_ln_bwd_reduce, dim3((2 * n_cols + kRedCols - 1) / kRedCols), dim3(kBlock),
                       0, st, static_cast<const float*>(workspace), static_cast<int32_t>(nb),
                       n_cols, dgamma, dbeta);
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}
