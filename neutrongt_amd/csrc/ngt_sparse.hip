// Topology-masked window attention, forward and backward, driven by the
// query-major and key-major CSR built in ngt_csr.hip.
//
// Reference semantics (NeutronGT/models/graphormer_dist_node_level.py:67-98):
//   a_e   = sum_c k[j,h,c] q[i,h,c] / sqrt(d)      e = (j -> i)
//   p_e   = exp(clamp(a_e, -5, 5))                 (no max subtraction)
//   out_i = sum_e p_e v_j / (sum_e p_e + 1e-6)
//   score_i = sum_e mean_h p_e
// Because no running maximum is subtracted, partial sums over disjoint edge
// subsets combine by plain addition; long rows are therefore split into
// fixed-size chunks whose partials a finalize kernel adds in chunk order.
//
// Wave layout: lane = slot * L + h with L = next_pow2(H) lanes per edge and
// S = 64 / L edge slots per wave.  Each lane owns one head of one edge and the
// d-element head slice of every gathered row, so one slot reads a full
// contiguous K/V row (H*d elements) per edge: coalesced row-segment gathers.
#include "ngt_common.h"

#include <utility>

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

template <int DH>
__device__ __forceinline__ float dot(const float (&a)[DH], const float (&b)[DH]) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int c = 0; c < DH; c += 2) {
    s0 = fmaf(a[c], b[c], s0);
    if (c + 1 < DH) s1 = fmaf(a[c + 1], b[c + 1], s1);
  }
  return s0 + s1;
}

__device__ __forceinline__ float clampf(float a, float lo, float hi) {
  return fminf(fmaxf(a, lo), hi);
}

// ------------------------------------------------------------------ forward
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_fwd(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ col, const int4* __restrict__ items, int32_t n_items, int32_t H,
    int32_t L, float inv_scale, float lo, float hi, float eps, T* __restrict__ out,
    float* __restrict__ rinv, float* __restrict__ node_score, int32_t ns_len,
    float* __restrict__ part_acc, float* __restrict__ part_z) {
  const int lane = threadIdx.x & (kWave - 1);
  const int item = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (item >= n_items) return;
  const int4 it = items[item];
  const int h = lane & (L - 1);
  const int slot = lane / L;
  const int S = kWave / L;
  const bool active = h < H;
  const int64_t row = it.x;

  float qr[DH], acc[DH];
  float z = 0.f;
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  if (active) {
    load_row<T, DH>(q + (row * H + h) * DH, qr);
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) qr[c] = 0.f;
  }

  int e = it.y + slot;
  const int end = it.z;
  for (; e + S < end; e += 2 * S) {
    const int64_t j0 = col[e];
    const int64_t j1 = col[e + S];
    if (active) {
      float k0[DH], v0[DH], k1[DH], v1[DH];
      load_row<T, DH>(k + (j0 * H + h) * DH, k0);
      load_row<T, DH>(k + (j1 * H + h) * DH, k1);
      load_row<T, DH>(v + (j0 * H + h) * DH, v0);
      load_row<T, DH>(v + (j1 * H + h) * DH, v1);
      const float p0 = __expf(clampf(dot<DH>(qr, k0) * inv_scale, lo, hi));
      const float p1 = __expf(clampf(dot<DH>(qr, k1) * inv_scale, lo, hi));
      z += p0;
      z += p1;
#pragma unroll
      for (int c = 0; c < DH; ++c) acc[c] = fmaf(p1, v1[c], fmaf(p0, v0[c], acc[c]));
    }
  }
  if (e < end) {
    const int64_t j0 = col[e];
    if (active) {
      float k0[DH], v0[DH];
      load_row<T, DH>(k + (j0 * H + h) * DH, k0);
      load_row<T, DH>(v + (j0 * H + h) * DH, v0);
      const float p0 = __expf(clampf(dot<DH>(qr, k0) * inv_scale, lo, hi));
      z += p0;
#pragma unroll
      for (int c = 0; c < DH; ++c) acc[c] = fmaf(p0, v0[c], acc[c]);
    }
  }

  reduce_slots<DH>(acc, z, L);
  if (it.w < 0) {
    const float zs = reduce_heads(z, L);  // inactive lanes hold z = 0
    if (slot == 0 && active) {
      const float den = z + eps;
      float o[DH];
#pragma unroll
      for (int c = 0; c < DH; ++c) o[c] = acc[c] / den;
      store_row<T, DH>(out + (row * H + h) * DH, o);
      rinv[row * H + h] = 1.0f / den;
    }
    if (lane == 0 && node_score != nullptr && row < ns_len) node_score[row] = zs / float(H);
  } else if (slot == 0 && active) {
    const int64_t p = int64_t(it.w) * H + h;
    store_f32<DH>(part_acc + p * DH, acc);
    part_z[p] = z;
  }
}

template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_fwd_finalize(
    const int4* __restrict__ splits, int32_t n_splits, int32_t H, int32_t L, float eps,
    const float* __restrict__ part_acc, const float* __restrict__ part_z, T* __restrict__ out,
    float* __restrict__ rinv, float* __restrict__ node_score, int32_t ns_len) {
  const int lane = threadIdx.x & (kWave - 1);
  const int w = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (w >= n_splits) return;
  const int4 sp = splits[w];
  const int h = lane & (L - 1);
  const int slot = lane / L;
  const int S = kWave / L;
  const bool active = h < H;
  const int64_t row = sp.x;
  float acc[DH];
  float z = 0.f;
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  if (active) {
    for (int p = slot; p < sp.z; p += S) {
      const int64_t at = int64_t(sp.y + p) * H + h;
      float t[DH];
      load_f32<DH>(part_acc + at * DH, t);
#pragma unroll
      for (int c = 0; c < DH; ++c) acc[c] += t[c];
      z += part_z[at];
    }
  }
  reduce_slots<DH>(acc, z, L);
  const float zs = reduce_heads(z, L);
  if (slot == 0 && active) {
    const float den = z + eps;
    float o[DH];
#pragma unroll
    for (int c = 0; c < DH; ++c) o[c] = acc[c] / den;
    store_row<T, DH>(out + (row * H + h) * DH, o);
    rinv[row * H + h] = 1.0f / den;
  }
  if (lane == 0 && node_score != nullptr && row < ns_len) node_score[row] = zs / float(H);
}

// ----------------------------------------------------------------- backward
// rd[i,h] = {r, r * D} with r = 1/(Z+eps), D = sum_c G[i,h,c] out[i,h,c].
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_rowstat(const T* __restrict__ out,
                                                    const T* __restrict__ g,
                                                    const float* __restrict__ rinv,
                                                    int64_t n_rows_heads,
                                                    float2* __restrict__ rd) {
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < n_rows_heads;
       t += int64_t(gridDim.x) * blockDim.x) {
    float o[DH], gg[DH];
    load_row<T, DH>(out + t * DH, o);
    load_row<T, DH>(g + t * DH, gg);
    const float r = rinv[t];
    rd[t] = make_float2(r, r * dot<DH>(o, gg));
  }
}

// Key-major pass: grad_k, grad_v of key row j and da_e for every edge of j
// (stored at the key-major edge position for the query-major pass).
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_bwd_kv(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ g, const float2* __restrict__ rd, const int32_t* __restrict__ t_col,
    const int4* __restrict__ items, int32_t n_items, int32_t H, int32_t L, float inv_scale,
    float lo, float hi, T* __restrict__ grad_k, T* __restrict__ grad_v, float* __restrict__ ds,
    float* __restrict__ part_kv) {
  const int lane = threadIdx.x & (kWave - 1);
  const int item = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (item >= n_items) return;
  const int4 it = items[item];
  const int h = lane & (L - 1);
  const int slot = lane / L;
  const int S = kWave / L;
  const bool active = h < H;
  const int64_t row = it.x;

  float kr[DH], vr[DH], dk[DH], dv[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dk[c] = 0.f;
    dv[c] = 0.f;
  }
  if (active) {
    load_row<T, DH>(k + (row * H + h) * DH, kr);
    load_row<T, DH>(v + (row * H + h) * DH, vr);
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) {
      kr[c] = 0.f;
      vr[c] = 0.f;
    }
  }
  for (int e = it.y + slot; e < it.z; e += S) {
    const int64_t i = t_col[e];
    if (active) {
      float qi[DH], gi[DH];
      load_row<T, DH>(q + (i * H + h) * DH, qi);
      load_row<T, DH>(g + (i * H + h) * DH, gi);
      const float2 r = rd[i * H + h];
      const float a = dot<DH>(qi, kr) * inv_scale;
      const float p = __expf(clampf(a, lo, hi));
      const float dp = r.x * dot<DH>(gi, vr) - r.y;
      const float da = (a >= lo && a <= hi) ? dp * p : 0.f;
      const float pr = p * r.x;
#pragma unroll
      for (int c = 0; c < DH; ++c) {
        dk[c] = fmaf(da, qi[c], dk[c]);
        dv[c] = fmaf(pr, gi[c], dv[c]);
      }
      ds[int64_t(e) * H + h] = da;
    }
  }
  reduce_slots2<DH>(dk, dv, L);
  if (slot == 0 && active) {
#pragma unroll
    for (int c = 0; c < DH; ++c) dk[c] *= inv_scale;
    if (it.w < 0) {
      store_row<T, DH>(grad_k + (row * H + h) * DH, dk);
      store_row<T, DH>(grad_v + (row * H + h) * DH, dv);
    } else {
      float* p = part_kv + (int64_t(it.w) * H + h) * (2 * DH);
      store_f32<DH>(p, dk);
      store_f32<DH>(p + DH, dv);
    }
  }
}

template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_bwd_kv_finalize(
    const int4* __restrict__ splits, int32_t n_splits, int32_t H, int32_t L,
    const float* __restrict__ part_kv, T* __restrict__ grad_k, T* __restrict__ grad_v) {
  const int lane = threadIdx.x & (kWave - 1);
  const int w = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (w >= n_splits) return;
  const int4 sp = splits[w];
  const int h = lane & (L - 1);
  const int slot = lane / L;
  const int S = kWave / L;
  const bool active = h < H;
  const int64_t row = sp.x;
  float dk[DH], dv[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dk[c] = 0.f;
    dv[c] = 0.f;
  }
  if (active) {
    for (int p = slot; p < sp.z; p += S) {
      const float* src = part_kv + (int64_t(sp.y + p) * H + h) * (2 * DH);
      float a[DH], b[DH];
      load_f32<DH>(src, a);
      load_f32<DH>(src + DH, b);
#pragma unroll
      for (int c = 0; c < DH; ++c) {
        dk[c] += a[c];
        dv[c] += b[c];
      }
    }
  }
  reduce_slots2<DH>(dk, dv, L);
  if (slot == 0 && active) {
    store_row<T, DH>(grad_k + (row * H + h) * DH, dk);
    store_row<T, DH>(grad_v + (row * H + h) * DH, dv);
  }
}

// Query-major pass: grad_q[i] = sum_e da_e k_j / scale.
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_bwd_q(
    const T* __restrict__ k, const int32_t* __restrict__ col, const int32_t* __restrict__ q2t,
    const float* __restrict__ ds, const int4* __restrict__ items, int32_t n_items, int32_t H,
    int32_t L, float inv_scale, T* __restrict__ grad_q, float* __restrict__ part_q) {
  const int lane = threadIdx.x & (kWave - 1);
  const int item = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (item >= n_items) return;
  const int4 it = items[item];
  const int h = lane & (L - 1);
  const int slot = lane / L;
  const int S = kWave / L;
  const bool active = h < H;
  const int64_t row = it.x;
  float dq[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) dq[c] = 0.f;
  int e = it.y + slot;
  for (; e + S < it.z; e += 2 * S) {
    const int64_t j0 = col[e], j1 = col[e + S];
    const int64_t t0 = q2t[e], t1 = q2t[e + S];
    if (active) {
      float k0[DH], k1[DH];
      load_row<T, DH>(k + (j0 * H + h) * DH, k0);
      load_row<T, DH>(k + (j1 * H + h) * DH, k1);
      const float d0 = ds[t0 * H + h];
      const float d1 = ds[t1 * H + h];
#pragma unroll
      for (int c = 0; c < DH; ++c) dq[c] = fmaf(d1, k1[c], fmaf(d0, k0[c], dq[c]));
    }
  }
  if (e < it.z) {
    const int64_t j0 = col[e];
    const int64_t t0 = q2t[e];
    if (active) {
      float k0[DH];
      load_row<T, DH>(k + (j0 * H + h) * DH, k0);
      const float d0 = ds[t0 * H + h];
#pragma unroll
      for (int c = 0; c < DH; ++c) dq[c] = fmaf(d0, k0[c], dq[c]);
    }
  }
  reduce_slots1<DH>(dq, L);
  if (slot == 0 && active) {
#pragma unroll
    for (int c = 0; c < DH; ++c) dq[c] *= inv_scale;
    if (it.w < 0)
      store_row<T, DH>(grad_q + (row * H + h) * DH, dq);
    else
      store_f32<DH>(part_q + (int64_t(it.w) * H + h) * DH, dq);
  }
}

template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_bwd_q_finalize(const int4* __restrict__ splits,
                                                           int32_t n_splits, int32_t H, int32_t L,
                                                           const float* __restrict__ part_q,
                                                           T* __restrict__ grad_q) {
  const int lane = threadIdx.x & (kWave - 1);
  const int w = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (w >= n_splits) return;
  const int4 sp = splits[w];
  const int h = lane & (L - 1);
  const int slot = lane / L;
  const int S = kWave / L;
  const bool active = h < H;
  const int64_t row = sp.x;
  float dq[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) dq[c] = 0.f;
  if (active) {
    for (int p = slot; p < sp.z; p += S) {
      float a[DH];
      load_f32<DH>(part_q + (int64_t(sp.y + p) * H + h) * DH, a);
#pragma unroll
      for (int c = 0; c < DH; ++c) dq[c] += a[c];
    }
  }
  reduce_slots1<DH>(dq, L);
  if (slot == 0 && active) store_row<T, DH>(grad_q + (row * H + h) * DH, dq);
}

// ------------------------------------------------------------------ host side
inline int blocks_for_waves(int64_t waves) {
  return static_cast<int>((waves + kWavesPerBlock - 1) / kWavesPerBlock);
}

inline int lanes_for_heads(int H) {
  int L = 1;
  while (L < H) L <<= 1;
  return L;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct FwdLayout {
  size_t part_acc, part_z, total;
};
struct BwdLayout {
  size_t rd, ds, part_kv, part_q, total;
};

FwdLayout fwd_layout(const ngt_window_csr* c, int H, int d) {
  FwdLayout L{};
  size_t off = 0;
  L.part_acc = off;
  off += align256(size_t(c->n_parts_q) * H * d * 4);
  L.part_z = off;
  off += align256(size_t(c->n_parts_q) * H * 4);
  L.total = off;
  return L;
}

BwdLayout bwd_layout(const ngt_window_csr* c, int H, int d) {
  BwdLayout L{};
  size_t off = 0;
  L.rd = off;
  off += align256(size_t(c->n_q) * H * 8);
  L.ds = off;
  off += align256(size_t(c->n_edges) * H * 4);
  L.part_kv = off;
  off += align256(size_t(c->n_parts_k) * H * 2 * d * 4);
  L.part_q = off;
  off += align256(size_t(c->n_parts_q) * H * d * 4);
  L.total = off;
  return L;
}

int check_common(const char* fn, int dtype, const ngt_window_csr* csr, int H, int d) {
  if (!csr) return set_error(NGT_ERR_ARG, "%s: null csr", fn);
  if (dtype != NGT_F32 && dtype != NGT_BF16)
    return set_error(NGT_ERR_ARG, "%s: unknown dtype %d", fn, dtype);
  if (H < 1 || H > 64)
    return set_error(NGT_ERR_UNSUPPORTED, "%s: n_heads=%d (supported 1..64)", fn, H);
  if (d != 8 && d != 16 && d != 24 && d != 32 && d != 64)
    return set_error(NGT_ERR_UNSUPPORTED, "%s: head_dim=%d (supported 8,16,24,32,64)", fn, d);
  if (csr->n_items_q < 0 || csr->n_items_k < 0 || csr->n_items_q > csr->max_items_q ||
      csr->n_items_k > csr->max_items_k || csr->n_splits_q > csr->max_splits_q ||
      csr->n_splits_k > csr->max_splits_k)
    return set_error(NGT_ERR_ARG, "%s: csr counters not filled from info[]", fn);
  return NGT_OK;
}

template <typename T, int DH>
int launch_fwd(const ngt_window_csr* c, const void* q, const void* k, const void* v, int H,
               float inv_scale, float lo, float hi, float eps, void* out, float* rinv, float* ns,
               int ns_len, char* ws, hipStream_t st) {
  const int L = lanes_for_heads(H);
  const FwdLayout lay = fwd_layout(c, H, DH);
  float* part_acc = reinterpret_cast<float*>(ws + lay.part_acc);
  float* part_z = reinterpret_cast<float*>(ws + lay.part_z);
  if (c->n_items_q > 0) {
    hipLaunchKernelGGL((k_fwd<T, DH>), dim3(blocks_for_waves(c->n_items_q)), dim3(kBlock), 0, st,
                       static_cast<const T*>(q), static_cast<const T*>(k),
                       static_cast<const T*>(v), c->col, reinterpret_cast<const int4*>(c->items_q),
                       c->n_items_q, H, L, inv_scale, lo, hi, eps, static_cast<T*>(out), rinv, ns,
                       ns_len, part_acc, part_z);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (c->n_splits_q > 0) {
    hipLaunchKernelGGL((k_fwd_finalize<T, DH>), dim3(blocks_for_waves(c->n_splits_q)),
                       dim3(kBlock), 0, st, reinterpret_cast<const int4*>(c->splits_q),
                       c->n_splits_q, H, L, eps, part_acc, part_z, static_cast<T*>(out), rinv, ns,
                       ns_len);
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

template <typename T, int DH>
int launch_bwd(const ngt_window_csr* c, const void* q, const void* k, const void* v,
               const void* out, const void* g, const float* rinv, int H, float inv_scale,
               float lo, float hi, void* gq, void* gk, void* gv, char* ws, hipStream_t st) {
  const int L = lanes_for_heads(H);
  const BwdLayout lay = bwd_layout(c, H, DH);
  float2* rd = reinterpret_cast<float2*>(ws + lay.rd);
  float* ds = reinterpret_cast<float*>(ws + lay.ds);
  float* part_kv = reinterpret_cast<float*>(ws + lay.part_kv);
  float* part_q = reinterpret_cast<float*>(ws + lay.part_q);
  const int64_t nrh = int64_t(c->n_q) * H;
  if (nrh > 0) {
    int64_t blocks = (nrh + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL((k_rowstat<T, DH>), dim3(int(blocks)), dim3(kBlock), 0, st,
                       static_cast<const T*>(out), static_cast<const T*>(g), rinv, nrh, rd);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (c->n_items_k > 0) {
    hipLaunchKernelGGL((k_bwd_kv<T, DH>), dim3(blocks_for_waves(c->n_items_k)), dim3(kBlock), 0,
                       st, static_cast<const T*>(q), static_cast<const T*>(k),
                       static_cast<const T*>(v), static_cast<const T*>(g), rd, c->t_col,
                       reinterpret_cast<const int4*>(c->items_k), c->n_items_k, H, L, inv_scale,
                       lo, hi, static_cast<T*>(gk), static_cast<T*>(gv), ds, part_kv);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (c->n_splits_k > 0) {
    hipLaunchKernelGGL((k_bwd_kv_finalize<T, DH>), dim3(blocks_for_waves(c->n_splits_k)),
                       dim3(kBlock), 0, st, reinterpret_cast<const int4*>(c->splits_k),
                       c->n_splits_k, H, L, part_kv, static_cast<T*>(gk), static_cast<T*>(gv));
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (c->n_items_q > 0) {
    hipLaunchKernelGGL((k_bwd_q<T, DH>), dim3(blocks_for_waves(c->n_items_q)), dim3(kBlock), 0,
                       st, static_cast<const T*>(k), c->col, c->q2t, ds,
                       reinterpret_cast<const int4*>(c->items_q), c->n_items_q, H, L, inv_scale,
                       static_cast<T*>(gq), part_q);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (c->n_splits_q > 0) {
    hipLaunchKernelGGL((k_bwd_q_finalize<T, DH>), dim3(blocks_for_waves(c->n_splits_q)),
                       dim3(kBlock), 0, st, reinterpret_cast<const int4*>(c->splits_q),
                       c->n_splits_q, H, L, part_q, static_cast<T*>(gq));
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

template <template <typename, int> class F, typename... Args>
int dispatch(int dtype, int d, Args&&... args) {
#define NGT_CASE(DH)                                                       \
  case DH:                                                                 \
    return dtype == NGT_F32 ? F<float, DH>::run(std::forward<Args>(args)...) \
                            : F<bf16_t, DH>::run(std::forward<Args>(args)...);
  switch (d) {
    NGT_CASE(8)
    NGT_CASE(16)
    NGT_CASE(24)
    NGT_CASE(32)
    NGT_CASE(64)
    default:
      return set_error(NGT_ERR_UNSUPPORTED, "head_dim=%d has no kernel", d);
  }
#undef NGT_CASE
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

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_sparse_workspace_bytes(const ngt_window_csr* csr, int32_t n_heads,
                                          int32_t head_dim, size_t* fwd_bytes,
                                          size_t* bwd_bytes) {
  const int rc = check_common("ngt_sparse_workspace_bytes", NGT_F32, csr, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (fwd_bytes) *fwd_bytes = fwd_layout(csr, n_heads, head_dim).total;
  if (bwd_bytes) *bwd_bytes = bwd_layout(csr, n_heads, head_dim).total;
  return NGT_OK;
}

extern "C" int ngt_sparse_fwd(int dtype, const void* q, const void* k, const void* v,
                              const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                              float scale, float clamp_lo, float clamp_hi, float eps, void* out,
                              float* rinv, float* node_score, int32_t node_score_len,
                              void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common("ngt_sparse_fwd", dtype, csr, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (!(scale > 0.f)) return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: scale must be > 0");
  if (csr->n_q > 0 && (!q || !out || !rinv))
    return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: null q/out/rinv");
  if (csr->n_edges > 0 && (!k || !v)) return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: null k/v");
  if (node_score_len < 0 || node_score_len > csr->n_q)
    return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: node_score_len out of range");
  const size_t need = fwd_layout(csr, n_heads, head_dim).total;
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(NGT_ERR_WORKSPACE, "ngt_sparse_fwd: workspace %zu < %zu", workspace_bytes,
                     need);
  return dispatch<FwdOp>(dtype, head_dim, csr, q, k, v, int(n_heads), 1.0f / scale, clamp_lo,
                         clamp_hi, eps, out, rinv, node_score, int(node_score_len),
                         static_cast<char*>(workspace), static_cast<hipStream_t>(stream));
}

extern "C" int ngt_sparse_bwd(int dtype, const void* q, const void* k, const void* v,
                              const void* out, const void* grad_out, const float* rinv,
                              const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                              float scale, float clamp_lo, float clamp_hi, void* grad_q,
                              void* grad_k, void* grad_v, void* workspace, size_t workspace_bytes,
                              void* stream) {
  int rc = check_common("ngt_sparse_bwd", dtype, csr, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (!(scale > 0.f)) return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: scale must be > 0");
  if (csr->n_q > 0 && (!q || !out || !grad_out || !rinv || !grad_q))
    return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: null query-side pointer");
  if (csr->n_k > 0 && (!k || !v || !grad_k || !grad_v))
    return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: null key-side pointer");
  const size_t need = bwd_layout(csr, n_heads, head_dim).total;
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(NGT_ERR_WORKSPACE, "ngt_sparse_bwd: workspace %zu < %zu", workspace_bytes,
                     need);
  return dispatch<BwdOp>(dtype, head_dim, csr, q, k, v, out, grad_out, rinv, int(n_heads),
                         1.0f / scale, clamp_lo, clamp_hi, grad_q, grad_k, grad_v,
                         static_cast<char*>(workspace), static_cast<hipStream_t>(stream));
}
