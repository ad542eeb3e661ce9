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
// Vector-ALU kernels (fp32, and bf16 at d = 64): one row per lane (query
// rows in the forward and dQ pass, key rows in the dK/dV pass), the other
// side streamed at wave-uniform addresses, so its rows arrive through scalar
// loads and feed the lane's FMAs from scalar registers.  The forward keeps an
// online softmax per row (running max m, running sum l); a block's 4 waves
// split the streamed rows and add their partial results in a fixed order at
// the end.
#include "ngt_common.h"

#include <math.h>
#include <stdlib.h>

#include <type_traits>
#include <utility>

namespace ngt {

// Matrix-core kernels (ngt_dense_mfma.hip).
bool mfma_dense_supported(int d);
MfSplit mfma_fwd_split(int n_q, int n_k, int H, bool node_scores);
MfSplit mfma_dq_split(int n_q, int n_k, int H);
int mfma_fused_blocks(int n_q, int n_k, int H, int d);
int mfma_dense_fwd(int d, const void* q, const void* k, const void* v, int n_q, int n_k, int H,
                   float scale, const DropoutMask* dm, void* out, float* out32, float* lse,
                   float* part, MfSplit sp, float* part_ml, float* part_acc, hipStream_t st);
int mfma_dense_bwd(int d, const void* q, const void* k, const void* v, const void* g,
                   const void* out, const float* out32, const float* lse, float* dsum, int n_q,
                   int n_k, int H, float scale, const DropoutMask* dm, void* gq, void* gk, void* gv,
                   MfSplit sq, float* part_dq, int fused_blocks, hipStream_t st);

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kRowsPerBlock = kWave;  // one row per lane; the block's waves split the other side
constexpr int kKeyTile = 32;          // forward: keys per online-softmax step of a wave
constexpr int kStreamTile = 16;       // backward: streamed rows per step of a wave
constexpr int kNsKeys = 16;           // keys per node-score transpose
constexpr int kNsStride = kNsKeys + 4;
constexpr int kSumChunk = 16;  // values per lane per round of the cross-wave sum
constexpr int kLdsFloats = kWaves * kWave * kNsStride;
static_assert((kWaves - 1) * kSumChunk * kWave <= kLdsFloats, "cross-wave sum buffer");
static_assert(kKeyTile % kNsKeys == 0 && kStreamTile % 2 == 0, "tiles cover whole key pairs");

// One dependent FMA chain: the kernels keep several rows' dot products in
// flight, so a second partial sum would only add an addition.  (Four partial
// sums from d = 32 on were measured: the d = 32 forward slowed 2.25 -> 2.53 ms
// and the d = 64 dK/dV pass spilled, 13.7 -> 18.0 ms.)
template <int DH>
__device__ __forceinline__ float dot1(const float (&a)[DH], const float (&b)[DH]) {
  float s = a[0] * b[0];
#pragma unroll
  for (int c = 1; c < DH; ++c) s = fmaf(a[c], b[c], s);
  return s;
}

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

// An opaque copy of a wave-uniform integer, pinned to a scalar register.
// Addresses of streamed rows built from it stay in scalar registers (and
// their loads scalar) even where the compiler has already copied the
// original into a vector register for a per-lane address.
__device__ __forceinline__ int uniform_int(int x) {
  asm volatile("" : "+s"(x));
  return x;
}

// Marks x as read and rewritten here.  Volatile asm statements keep their
// order, so a group of arithmetic followed by pins of its results completes
// before the next statement (and the loads whose addresses come from a later
// uniform_int); without it the scheduler is free to hoist every scalar load
// of a tile ahead of all arithmetic.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

// x summed lane by lane over the block's waves, in wave order, into wave 0's
// registers (the other waves' copies are left as they were).  buf holds
// (kWaves - 1) * kSumChunk * kWave floats and may be reused by the caller
// before the call: every round starts with a barrier.
template <int N>
__device__ __forceinline__ void waves_sum(float (&x)[N], float* buf, int w, int lane) {
#pragma unroll
  for (int c0 = 0; c0 < N; c0 += kSumChunk) {
    __syncthreads();
    if (w > 0) {
#pragma unroll
      for (int c = 0; c < kSumChunk && c0 + c < N; ++c)
        buf[((w - 1) * kSumChunk + c) * kWave + lane] = x[c0 + c];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int c = 0; c < kSumChunk && c0 + c < N; ++c) {
        float s = x[c0 + c];
#pragma unroll
        for (int u = 0; u < kWaves - 1; ++u) s += buf[(u * kSumChunk + c) * kWave + lane];
        x[c0 + c] = s;
      }
    }
  }
}

// ------------------------------------------------------------------ forward
// One block = 64 query rows (one per lane) of one head; its 4 waves take the
// 32-key tiles in turn (wave w: tiles w, w + 4, ...) and meet at the end.
// Block b serves rows 64 (b / H) .. of head b % H: consecutive blocks take
// consecutive heads, so the round-robin of blocks over the 8 XCDs gives each
// XCD's L2 the K/V slices of its own heads.  The keys' rows are read at
// wave-uniform addresses (scalar loads), so a lane's arithmetic takes them
// straight from scalar registers.  Per tile a lane keeps its row's online
// softmax (running max m, running sum l, rescale once per tile).
// ns_part (optional) is [n_blocks, n_k]: per block (64 rows of one head),
// sum over its rows of |S[h, i, j]|, one writer per key.
template <typename T, int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_dense_fwd(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, int32_t n_q,
    int32_t n_k, int32_t H, float scale, DropoutMask dm, int32_t n_split, int32_t split_keys,
    T* __restrict__ out, float* __restrict__ out32, float* __restrict__ lse,
    float* __restrict__ ns_part, float* __restrict__ part_ml, float* __restrict__ part_acc) {
  __shared__ float lds[kLdsFloats];
  __shared__ float m_lds[kWaves * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // block -> (rows, key split, head) in scalar registers: the division runs
  // on the vector ALU, and addresses built from a vector register would turn
  // the streamed rows' scalar loads into vector loads
  const int h = __builtin_amdgcn_readfirstlane(blockIdx.x % H);
  const int rs = __builtin_amdgcn_readfirstlane(blockIdx.x / H);
  const int sp = __builtin_amdgcn_readfirstlane(rs % n_split);
  const int rb = __builtin_amdgcn_readfirstlane(rs / n_split);
  const int k0 = sp * split_keys;                 // this block's keys: [k0, k1)
  const int k1 = min(n_k, k0 + split_keys);
  const int64_t qi = int64_t(rb) * kRowsPerBlock + lane;
  const bool q_ok = qi < n_q;
  if constexpr (DROP) dm = drop_for_head(dm, h);

  float qs[DH];
  if (q_ok) {
    load_row<T, DH>(q + (qi * H + h) * DH, qs);
#pragma unroll
    for (int c = 0; c < DH; ++c) qs[c] *= scale;
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) qs[c] = 0.f;  // S = 0 exactly: no node-score share
  }
  float acc[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int64_t HD = int64_t(H) * DH;  // row stride of q, k, v
  const T* k_h = k + int64_t(uniform_int(h)) * DH;  // streamed rows of this head
  const T* v_h = v + int64_t(uniform_int(h)) * DH;
  float* ns_w = lds + w * kWave * kNsStride;
  float* ns_dst = ns_part ? ns_part + (int64_t(rb) * H + h) * n_k : nullptr;

  // keys per scalar-load group: up to 64 scalar registers of K (or V) rows in
  // flight; unbounded, the scheduler hoists a whole tile's loads and spills
  constexpr int kLoadGroup = DH >= 64 ? 1 : 64 / DH;
  static_assert(kKeyTile % kLoadGroup == 0, "load groups tile the key tile");
  const int n_tiles = (k1 - k0 + kKeyTile - 1) / kKeyTile;
  for (int t = w; t < n_tiles; t += kWaves) {
    // One body for every tile: key indices past k1 load row k1 - 1 (in
    // bounds) and get S = -inf, hence p = 0; their node-score columns are
    // never stored.
    const int kb = k0 + t * kKeyTile;
    const int k_last = k1 - 1;
    float s[kKeyTile];
#pragma unroll
    for (int g0 = 0; g0 < kKeyTile; g0 += kLoadGroup) {
      const int kg = uniform_int(kb + g0);
      float kr[kLoadGroup][DH];
#pragma unroll
      for (int i = 0; i < kLoadGroup; ++i)
        load_row<T, DH>(k_h + int64_t(min(kg + i, k_last)) * HD, kr[i]);
#pragma unroll
      for (int i = 0; i < kLoadGroup; ++i) {
        s[g0 + i] = dot1<DH>(qs, kr[i]);
        pin(s[g0 + i]);
      }
    }
    if (kb + kKeyTile > k1) {
#pragma unroll
      for (int i = 0; i < kKeyTile; ++i)
        if (kb + i > k_last) s[i] = -INFINITY;
    }
    float tmax = s[0];
#pragma unroll
    for (int i = 1; i < kKeyTile; ++i) tmax = fmaxf(tmax, s[i]);
    const float m_new = fmaxf(m, tmax);
    const float alpha = __expf(m - m_new);
    l *= alpha;
#pragma unroll
    for (int c = 0; c < DH; ++c) acc[c] *= alpha;
    uint32_t dw[kKeyTile / 2];  // one dropout word per key pair
    if constexpr (DROP) {
#pragma unroll
      for (int i = 0; i < kKeyTile / 2; ++i) dw[i] = drop_word(dm, uint32_t(qi), uint32_t(kb + 2 * i));
    }
    // (the V rows' addresses come from new opaque copies of the tile base:
    // left to itself the compiler keeps the K loop's 32 row offsets live)
#pragma unroll
    for (int g0 = 0; g0 < kKeyTile; g0 += kLoadGroup) {
      const int kg = uniform_int(kb + g0);
      float vr[kLoadGroup][DH];
#pragma unroll
      for (int i = 0; i < kLoadGroup; ++i)
        load_row<T, DH>(v_h + int64_t(min(kg + i, k_last)) * HD, vr[i]);
#pragma unroll
      for (int i = 0; i < kLoadGroup; ++i) {
        const float p = __expf(s[g0 + i] - m_new);
        l += p;  // the softmax normaliser uses every key
        float pv = p;
        if constexpr (DROP) pv *= drop_scale(dm, dw[(g0 + i) / 2], uint32_t(kb + g0 + i));
#pragma unroll
        for (int c = 0; c < DH; ++c) acc[c] = fmaf(pv, vr[i][c], acc[c]);
      }
      pin(l);
#pragma unroll
      for (int c = 0; c < DH; ++c) pin(acc[c]);
    }
    m = m_new;
    if (ns_dst) {
      // |S| of 16 keys x 64 rows through this wave's LDS patch: lane = row
      // writes its 16 values, then lane = (key, quarter of the rows) adds 16
      // rows and the four quarters meet by shuffles (fixed order).
#pragma unroll
      for (int h0 = 0; h0 < kKeyTile; h0 += kNsKeys) {
#pragma unroll
        for (int c = 0; c < kNsKeys; c += 4) {
          const float4 a = {fabsf(s[h0 + c]), fabsf(s[h0 + c + 1]), fabsf(s[h0 + c + 2]),
                            fabsf(s[h0 + c + 3])};
          *reinterpret_cast<float4*>(ns_w + lane * kNsStride + c) = a;
        }
        __builtin_amdgcn_wave_barrier();
        const int key = lane & (kNsKeys - 1);
        const int rq = lane >> 4;
        float x = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) x += ns_w[(rq * 16 + r) * kNsStride + key];
        x += shfl_xor(x, 16);
        x += shfl_xor(x, 32);
        const int kj = kb + h0 + key;
        if (lane < kNsKeys && kj < k1) ns_dst[kj] = x;
        __builtin_amdgcn_wave_barrier();
      }
    }
  }

  // the waves' partial softmax states: common maximum, then sums in wave order
  m_lds[w * kWave + lane] = m;
  __syncthreads();
  float M = m_lds[lane];
#pragma unroll
  for (int u = 1; u < kWaves; ++u) M = fmaxf(M, m_lds[u * kWave + lane]);
  const float alpha = m == -INFINITY ? 0.f : __expf(m - M);
  float x[DH + 1];
#pragma unroll
  for (int c = 0; c < DH; ++c) x[c] = acc[c] * alpha;
  x[DH] = l * alpha;
  waves_sum<DH + 1>(x, lds, w, lane);
  if (n_split > 1) {
    // the split's softmax state (max M, sum l, unnormalised acc) for the combine
    if (w == 0 && q_ok) {
      const int64_t r = (int64_t(sp) * H + h) * n_q + qi;
      part_ml[2 * r] = M;
      part_ml[2 * r + 1] = x[DH];
      float a[DH];
#pragma unroll
      for (int c = 0; c < DH; ++c) a[c] = x[c];
      store_f32<DH>(part_acc + ((int64_t(sp) * n_q + qi) * H + h) * DH, a);
    }
    return;
  }
  if (w == 0 && q_ok) {
    float o[DH];
    const float inv = n_k > 0 ? 1.0f / x[DH] : 0.f;
#pragma unroll
    for (int c = 0; c < DH; ++c) o[c] = x[c] * inv;
    store_row<T, DH>(out + (qi * H + h) * DH, o);
    if (out32) store_f32<DH>(out32 + (qi * H + h) * DH, o);
    lse[int64_t(h) * n_q + qi] = n_k > 0 ? M + __logf(x[DH]) : -INFINITY;
  }
}

// The key splits' softmax states of one (query, head) per thread, in split
// order: M = max M_s, l = sum l_s e^(M_s - M), out = sum acc_s e^(M_s - M) / l.
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_dense_combine(
    const float* __restrict__ part_ml, const float* __restrict__ part_acc, int32_t n_split,
    int32_t n_q, int32_t H, T* __restrict__ out, float* __restrict__ out32,
    float* __restrict__ lse) {
  const int64_t n = int64_t(n_q) * H;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < n;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t qi = t / H, h = t % H;
    float M = -INFINITY;
    for (int s = 0; s < n_split; ++s) M = fmaxf(M, part_ml[2 * ((s * H + h) * n_q + qi)]);
    float l = 0.f, acc[DH];
#pragma unroll
    for (int c = 0; c < DH; ++c) acc[c] = 0.f;
    for (int s = 0; s < n_split; ++s) {
      const int64_t r = (s * H + h) * n_q + qi;
      const float a = __expf(part_ml[2 * r] - M);
      l = fmaf(a, part_ml[2 * r + 1], l);
      float pa[DH];
      load_row<float, DH>(part_acc + (s * n_q + qi) * H * DH + h * DH, pa);
#pragma unroll
      for (int c = 0; c < DH; ++c) acc[c] = fmaf(a, pa[c], acc[c]);
    }
    const float inv = 1.0f / l;
#pragma unroll
    for (int c = 0; c < DH; ++c) acc[c] *= inv;
    store_row<T, DH>(out + t * DH, acc);
    if (out32) store_f32<DH>(out32 + t * DH, acc);
    lse[h * n_q + qi] = M + __logf(l);
  }
}

// node_score[j] = sum over rows of ns_part[:, j] / H.  A block of 1024
// threads takes 64 keys (lane = key) and splits the rows over its 16 waves
// (wave w: rows w, w + 16, ...); the waves' sums are added in wave order.
// One thread per key down all rows (2,000 at 16,000 nodes, 8 heads) left the
// loads' latency exposed: 466 us for 128 MB.
constexpr int kScoreThreads = 1024;
constexpr int kScoreWaves = kScoreThreads / kWave;
__global__ __launch_bounds__(kScoreThreads) void k_dense_scores(
    const float* __restrict__ part, int32_t rows, int32_t n_k, int32_t H, float* __restrict__ ns) {
  __shared__ float red[kScoreWaves][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x >> 6;
  const int64_t j = int64_t(blockIdx.x) * kWave + lane;
  float s = 0.f;
  if (j < n_k) {
#pragma unroll 8
    for (int r = w; r < rows; r += kScoreWaves) s += part[int64_t(r) * n_k + j];
  }
  red[w][lane] = s;
  __syncthreads();
  if (w == 0 && j < n_k) {
    float t = red[0][lane];
#pragma unroll
    for (int u = 1; u < kScoreWaves; ++u) t += red[u][lane];
    ns[j] = t / float(H);
  }
}

// ----------------------------------------------------------------- backward
// Blocks per key block of the dK/dV pass (one per half of the dK/dV columns).
template <typename T, int DH>
constexpr int kv_col_split() {
  return DH >= 64 && std::is_same<T, float>::value ? 2 : 1;
}

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

// Key-major pass: one block = 64 key rows (one per lane) of one head, in the
// forward's block order; its waves take the 16-query tiles in turn.  Each
// lane keeps K_j * scale and V_j; the query rows (Q, dO, lse, D) are read at
// wave-uniform addresses.  dK = scale sum_i dS_ij Q_i is summed unscaled and
// scaled once.
template <typename T, int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_dense_bwd_kv(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ g, const float* __restrict__ lse, const float* __restrict__ dsum,
    int32_t n_q, int32_t n_k, int32_t H, float scale, DropoutMask dm, T* __restrict__ grad_k,
    T* __restrict__ grad_v) {
  __shared__ float lds[kLdsFloats];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // fp32 at d >= 64: a block writes one half of the dK/dV columns (DC of
  // them); the lane keeps 64 + 64 registers of K and V rows for the dot
  // products but only 32 + 32 of dK and dV, 192 in all, so two waves fit a
  // SIMD (8,000 x 8,000 x 8 heads: 13.7 -> 11.8 ms).  The bf16 variant spills
  // scalar registers that way (12.5 -> 15.4 ms) and keeps one block per row.
  constexpr int kColSplit = kv_col_split<T, DH>();
  constexpr int DC = DH / kColSplit;
  const int h = __builtin_amdgcn_readfirstlane(blockIdx.x % H);
  const int rc = __builtin_amdgcn_readfirstlane(blockIdx.x / H);
  const int ch = __builtin_amdgcn_readfirstlane(rc % kColSplit);  // column half
  const int rb = __builtin_amdgcn_readfirstlane(rc / kColSplit);
  const int64_t kj = int64_t(rb) * kRowsPerBlock + lane;
  const bool k_ok = kj < n_k;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  float ks[DH], vr[DH], dk[DH], dv[DH];  // at d >= 64 dK, dV use their first DC entries
  if (k_ok) {
    load_row<T, DH>(k + (kj * H + h) * DH, ks);
    load_row<T, DH>(v + (kj * H + h) * DH, vr);
#pragma unroll
    for (int c = 0; c < DH; ++c) ks[c] *= scale;
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) ks[c] = vr[c] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) dk[c] = dv[c] = 0.f;
  const int hs = uniform_int(h);
  const int64_t HD = int64_t(H) * DH;
  const T* q_h = q + int64_t(hs) * DH;  // streamed rows of this head
  const T* g_h = g + int64_t(hs) * DH;
  const float* lse_h = lse + int64_t(hs) * n_q;
  const float* ds_h = dsum + int64_t(hs) * n_q;
  // one query's contribution, from its streamed rows (word: the dropout word
  // of (qi, this lane's key pair))
  auto contrib = [&](const float (&qr)[DH], const float (&gr)[DH], float L, float D,
                     uint32_t word) {
    const float p = __expf(dot1<DH>(qr, ks) - L);
    float mm = 1.f;
    if constexpr (DROP) mm = drop_scale(dm, word, uint32_t(kj));
    const float ds = p * (mm * dot1<DH>(gr, vr) - D);
    const float pm = p * mm;
#pragma unroll
    for (int c = 0; c < DH; ++c) {
      dv[c] = fmaf(pm, gr[c], dv[c]);
      dk[c] = fmaf(ds, qr[c], dk[c]);
    }
  };
  auto step = [&](int qi) {
    float qr[DH], gr[DH];
    load_row<T, DH>(q_h + int64_t(qi) * HD, qr);
    load_row<T, DH>(g_h + int64_t(qi) * HD, gr);
    contrib(qr, gr, lse_h[qi], ds_h[qi], DROP ? drop_word(dm, uint32_t(qi), uint32_t(kj)) : 0U);
  };
  // d = 64: a query's Q and dO rows (128 scalar registers together) do not
  // fit beside the kernel's other scalars; each is read in halves for the two
  // dot products and read again, through an opaque index (so the compiler
  // reloads from the scalar cache instead of keeping the rows), for the dV
  // and dK updates.
  auto step_halves = [&](int qi) {
    constexpr int HF = DH / 2;
    float s_ = 0.f, dp = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float r[HF];
      load_row<T, HF>(q_h + int64_t(uniform_int(qi)) * HD + hh * HF, r);
#pragma unroll
      for (int c = 0; c < HF; ++c) s_ = fmaf(r[c], ks[hh * HF + c], s_);
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float r[HF];
      load_row<T, HF>(g_h + int64_t(uniform_int(qi)) * HD + hh * HF, r);
#pragma unroll
      for (int c = 0; c < HF; ++c) dp = fmaf(r[c], vr[hh * HF + c], dp);
    }
    const float p = __expf(s_ - lse_h[qi]);
    float mm = 1.f;
    if constexpr (DROP)
      mm = drop_scale(dm, drop_word(dm, uint32_t(qi), uint32_t(kj)), uint32_t(kj));
    const float ds = p * (mm * dp - ds_h[qi]);
    const float pm = p * mm;
    {  // this block's columns ch * DC ..
      float r[DC];
      load_row<T, DC>(g_h + int64_t(uniform_int(qi)) * HD + ch * DC, r);
#pragma unroll
      for (int c = 0; c < DC; ++c) dv[c] = fmaf(pm, r[c], dv[c]);
    }
    {
      float r[DC];
      load_row<T, DC>(q_h + int64_t(uniform_int(qi)) * HD + ch * DC, r);
#pragma unroll
      for (int c = 0; c < DC; ++c) dk[c] = fmaf(ds, r[c], dk[c]);
    }
  };
  // Full tiles in groups of kGroup queries: a group's scalar loads are issued
  // together from an opaque copy of its first index and its results pinned
  // before the next group (else each load waits on its own).  At d = 64 the
  // lane's own K, V, dK, dV rows already take 256 registers.
  constexpr int kGroup = DH >= 16 ? 1 : 16 / DH;
  constexpr int kUnroll = DH >= 64 ? 2 : kStreamTile / kGroup;
  const int n_tiles = (n_q + kStreamTile - 1) / kStreamTile;
  for (int t = w; t < n_tiles; t += kWaves) {
    const int qb = t * kStreamTile;
    if constexpr (DH >= 64) {
      for (int i = 0; i < kStreamTile && qb + i < n_q; ++i) step_halves(qb + i);
    } else if (qb + kStreamTile <= n_q) {
#pragma unroll kUnroll
      for (int g0 = 0; g0 < kStreamTile; g0 += kGroup) {
        const int qg = uniform_int(qb + g0);
        float qr[kGroup][DH], gr[kGroup][DH], L[kGroup], D[kGroup];
#pragma unroll
        for (int i = 0; i < kGroup; ++i) {
          load_row<T, DH>(q_h + int64_t(qg + i) * HD, qr[i]);
          load_row<T, DH>(g_h + int64_t(qg + i) * HD, gr[i]);
          L[i] = lse_h[qg + i];
          D[i] = ds_h[qg + i];
        }
        uint32_t wd[kGroup] = {};
        if constexpr (DROP && kGroup % 2 == 0) {
          // Lanes 2m and 2m + 1 hold one key pair, hence one dropout word per
          // query: the even lane hashes query i's, the odd lane query i + 1's,
          // and they swap (DPP quad_perm [1, 0, 3, 2]).
          const bool odd = lane & 1;
#pragma unroll
          for (int i = 0; i < kGroup; i += 2) {
            const uint32_t mine = drop_word(dm, uint32_t(qg + i + odd), uint32_t(kj));
            const uint32_t other = static_cast<uint32_t>(
                __builtin_amdgcn_mov_dpp(static_cast<int>(mine), 0xB1, 0xf, 0xf, false));
            wd[i] = odd ? other : mine;
            wd[i + 1] = odd ? mine : other;
          }
        } else if constexpr (DROP) {
#pragma unroll
          for (int i = 0; i < kGroup; ++i) wd[i] = drop_word(dm, uint32_t(qg + i), uint32_t(kj));
        }
#pragma unroll
        for (int i = 0; i < kGroup; ++i) contrib(qr[i], gr[i], L[i], D[i], wd[i]);
#pragma unroll
        for (int c = 0; c < DH; ++c) {
          pin(dk[c]);
          pin(dv[c]);
        }
      }
    } else {
      for (int i = 0; qb + i < n_q; ++i) step(qb + i);
    }
  }
  float x[2 * DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    x[c] = dk[c];
    x[DC + c] = dv[c];
  }
  waves_sum<2 * DC>(x, lds, w, lane);
  if (w == 0 && k_ok) {
    float ok[DC], ov[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      ok[c] = x[c] * scale;
      ov[c] = x[DC + c];
    }
    store_row<T, DC>(grad_k + (kj * H + h) * DH + ch * DC, ok);
    store_row<T, DC>(grad_v + (kj * H + h) * DH + ch * DC, ov);
  }
}

// Query-major pass: one block = 64 query rows (one per lane) of one head; its
// waves take the 16-key tiles in turn, reading K/V rows at wave-uniform
// addresses.
template <typename T, int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_dense_bwd_q(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ g, const float* __restrict__ lse, const float* __restrict__ dsum,
    int32_t n_q, int32_t n_k, int32_t H, float scale, DropoutMask dm, T* __restrict__ grad_q) {
  __shared__ float lds[kLdsFloats];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = __builtin_amdgcn_readfirstlane(blockIdx.x % H);
  const int rb = __builtin_amdgcn_readfirstlane(blockIdx.x / H);
  const int64_t qi = int64_t(rb) * kRowsPerBlock + lane;
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
  const int hs = uniform_int(h);
  const int64_t HD = int64_t(H) * DH;
  const T* k_h = k + int64_t(hs) * DH;  // streamed rows of this head
  const T* v_h = v + int64_t(hs) * DH;
  // one key's contribution, from its streamed rows
  auto contrib = [&](int kj, const float (&kr)[DH], const float (&vr)[DH], uint32_t word) {
    const float p = __expf(dot1<DH>(qs, kr) - L);
    float mm = 1.f;
    if constexpr (DROP) mm = drop_scale(dm, word, uint32_t(kj));
    const float ds = p * (mm * dot1<DH>(gi, vr) - Dq);
#pragma unroll
    for (int c = 0; c < DH; ++c) dq[c] = fmaf(ds, kr[c], dq[c]);
  };
  auto step = [&](int kj, uint32_t word) {
    float kr[DH], vr[DH];
    load_row<T, DH>(k_h + int64_t(kj) * HD, kr);
    load_row<T, DH>(v_h + int64_t(kj) * HD, vr);
    contrib(kj, kr, vr, word);
  };
  // d = 64: a key's K and V rows are read in halves, and K again through an
  // opaque index for the dQ update (as in the dK/dV pass)
  auto step_halves = [&](int kj, uint32_t word) {
    constexpr int HF = DH / 2;
    float s_ = 0.f, dp = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float r[HF];
      load_row<T, HF>(k_h + int64_t(uniform_int(kj)) * HD + hh * HF, r);
#pragma unroll
      for (int c = 0; c < HF; ++c) s_ = fmaf(qs[hh * HF + c], r[c], s_);
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float r[HF];
      load_row<T, HF>(v_h + int64_t(uniform_int(kj)) * HD + hh * HF, r);
#pragma unroll
      for (int c = 0; c < HF; ++c) dp = fmaf(gi[hh * HF + c], r[c], dp);
    }
    const float p = __expf(s_ - L);
    float mm = 1.f;
    if constexpr (DROP) mm = drop_scale(dm, word, uint32_t(kj));
    const float ds = p * (mm * dp - Dq);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float r[HF];
      load_row<T, HF>(k_h + int64_t(uniform_int(kj)) * HD + hh * HF, r);
#pragma unroll
      for (int c = 0; c < HF; ++c) dq[hh * HF + c] = fmaf(ds, r[c], dq[hh * HF + c]);
    }
  };
  // full tiles in groups of kGroup keys (a key pair at least), loads issued
  // together and results pinned per group as in the dK/dV pass (at d = 8,
  // pairs: 1.72 ms at 16,000 x 16,000 x 8 heads, against 2.14 ms for groups
  // of 4, whose 64 scalar registers of rows stall the wave longer)
#ifndef NGT_DENSE_Q_GROUP
#define NGT_DENSE_Q_GROUP 2
#endif
  constexpr int kGroup = DH >= 16 ? 2 : NGT_DENSE_Q_GROUP;
  const int n_tiles = (n_k + kStreamTile - 1) / kStreamTile;
  for (int t = w; t < n_tiles; t += kWaves) {
    const int kb = t * kStreamTile;
    if constexpr (DH >= 64) {
      for (int i = 0; i < kStreamTile && kb + i < n_k; ++i) {
        const uint32_t word = DROP ? drop_word(dm, uint32_t(qi), uint32_t(kb + i)) : 0U;
        step_halves(kb + i, word);
      }
    } else if (kb + kStreamTile <= n_k) {
#pragma unroll
      for (int g0 = 0; g0 < kStreamTile; g0 += kGroup) {
        const int kg = uniform_int(kb + g0);
        float kr[kGroup][DH], vr[kGroup][DH];
#pragma unroll
        for (int i = 0; i < kGroup; ++i) {
          load_row<T, DH>(k_h + int64_t(kg + i) * HD, kr[i]);
          load_row<T, DH>(v_h + int64_t(kg + i) * HD, vr[i]);
        }
#pragma unroll
        for (int i = 0; i < kGroup; i += 2) {
          const uint32_t word = DROP ? drop_word(dm, uint32_t(qi), uint32_t(kb + g0 + i)) : 0U;
          contrib(kb + g0 + i, kr[i], vr[i], word);
          contrib(kb + g0 + i + 1, kr[i + 1], vr[i + 1], word);
        }
#pragma unroll
        for (int c = 0; c < DH; ++c) pin(dq[c]);
      }
    } else {
      for (int i = 0; kb + i < n_k; ++i) {
        const uint32_t word = DROP ? drop_word(dm, uint32_t(qi), uint32_t(kb + i)) : 0U;
        step(kb + i, word);
      }
    }
  }
  waves_sum<DH>(dq, lds, w, lane);
  if (w == 0 && q_ok) {
#pragma unroll
    for (int c = 0; c < DH; ++c) dq[c] *= scale;
    store_row<T, DH>(grad_q + (qi * H + h) * DH, dq);
  }
}

// ------------------------------------------------------------------ host side
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline int64_t qblocks(int32_t n) { return (int64_t(n) + kRowsPerBlock - 1) / kRowsPerBlock; }

// Key splits of the vector-ALU forward: about kSplitTarget blocks in all
// (several rounds of resident blocks, so the last round's idle tail stays
// small), at least kMinSplitKeys keys per split, splits whole key tiles.
constexpr int64_t kSplitTarget = 8192;
constexpr int kMinSplitKeys = 512;
struct KeySplit {
  int n_split, split_keys;
};
KeySplit key_split(int32_t n_q, int32_t n_k, int32_t H) {
  const int64_t units = qblocks(n_q) * H;
  int64_t want = units > 0 ? (kSplitTarget + units - 1) / units : 1;
  want = std::min<int64_t>(want, std::max<int64_t>(1, n_k / kMinSplitKeys));
  if (want <= 1 || n_k <= 0) return {1, std::max(n_k, 1)};
  int keys = static_cast<int>((n_k + want - 1) / want);
  keys = (keys + kKeyTile - 1) / kKeyTile * kKeyTile;
  return {static_cast<int>((n_k + keys - 1) / keys), keys};
}

size_t ns_part_bytes(int32_t n_q, int32_t n_k, int32_t H) {
  return align256(size_t(qblocks(n_q)) * H * size_t(n_k) * 4);
}
size_t split_bytes(int32_t n_q, int32_t n_k, int32_t H, int32_t d) {
  const KeySplit ks = key_split(n_q, n_k, H);
  if (ks.n_split <= 1) return 0;
  return align256(size_t(ks.n_split) * n_q * H * 8) + align256(size_t(ks.n_split) * n_q * H * d * 4);
}
size_t fwd_ws(int32_t n_q, int32_t n_k, int32_t H, int32_t d) {
  return ns_part_bytes(n_q, n_k, H) + split_bytes(n_q, n_k, H, d);
}
size_t bwd_ws(int32_t n_q, int32_t H) { return align256(size_t(n_q) * H * 4); }

template <typename T, int DH>
int launch_fwd(const void* q, const void* k, const void* v, int n_q, int n_k, int H, float scale,
               const DropoutMask* dm, void* out, float* out32, float* lse, float* ns, char* ws,
               hipStream_t st) {
  if (n_q == 0) return NGT_OK;
  float* part = ns ? reinterpret_cast<float*>(ws) : nullptr;
  const KeySplit ks = key_split(n_q, n_k, H);
  float* part_ml = ks.n_split > 1 ? reinterpret_cast<float*>(ws + ns_part_bytes(n_q, n_k, H))
                                  : nullptr;
  float* part_acc =
      ks.n_split > 1 ? part_ml + align256(size_t(ks.n_split) * n_q * H * 8) / 4 : nullptr;
  const dim3 grid(static_cast<unsigned>(qblocks(n_q) * H * ks.n_split));
  {
    KernelTimer timer_("dense_fwd", st);
    const DropoutMask m = dm ? *dm : DropoutMask{};
    if (dm)
      hipLaunchKernelGGL((k_dense_fwd<T, DH, true>), grid, dim3(kBlock), 0, st,
                         static_cast<const T*>(q), static_cast<const T*>(k),
                         static_cast<const T*>(v), n_q, n_k, H, scale, m, ks.n_split,
                         ks.split_keys, static_cast<T*>(out), out32, lse, part, part_ml, part_acc);
    else
      hipLaunchKernelGGL((k_dense_fwd<T, DH, false>), grid, dim3(kBlock), 0, st,
                         static_cast<const T*>(q), static_cast<const T*>(k),
                         static_cast<const T*>(v), n_q, n_k, H, scale, m, ks.n_split,
                         ks.split_keys, static_cast<T*>(out), out32, lse, part, part_ml, part_acc);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (ks.n_split > 1) {
    KernelTimer timer_("dense_combine", st);
    int64_t blocks = (int64_t(n_q) * H + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL((k_dense_combine<T, DH>), dim3(int(blocks)), dim3(kBlock), 0, st, part_ml,
                       part_acc, ks.n_split, n_q, H, static_cast<T*>(out), out32, lse);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (ns && n_k > 0) {
    const int rows = static_cast<int>(qblocks(n_q) * H);
    KernelTimer timer_("dense_scores", st);
    hipLaunchKernelGGL(k_dense_scores, dim3((n_k + kWave - 1) / kWave), dim3(kScoreThreads), 0, st,
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
    // fp32 at d >= 64: two blocks per key block, one per half of the dK/dV columns
    const dim3 grid(static_cast<unsigned>(qblocks(n_k) * H * kv_col_split<T, DH>()));
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
    const dim3 grid(static_cast<unsigned>(qblocks(n_q) * H));
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

// The bf16 path runs on the matrix cores (ngt_dense_mfma.hip) for d <= 32;
// NGT_DENSE_VALU=1 selects the vector-ALU kernels instead (for comparison).
bool use_mfma(int dtype, int d) {
  static const bool valu = getenv("NGT_DENSE_VALU") != nullptr;
  return dtype == NGT_BF16 && mfma_dense_supported(d) && !valu;
}

// Forward workspace: the matrix-core path needs H * n_k floats of node-score
// partials (only with node scores); the vector-ALU path needs per-block
// node-score partials (only with node scores) and, when it splits the keys,
// the split states behind them.
// The matrix-core path: [node-score partials H * n_k (with node scores)]
// [split states (m, l) and unnormalised outputs (with a key split)].
struct MfFwdLayout {
  size_t ml, acc, total;
  MfSplit sp;
};
MfFwdLayout mf_fwd_layout(int32_t n_q, int32_t n_k, int32_t H, int32_t d, bool node_scores) {
  MfFwdLayout L{};
  L.sp = mfma_fwd_split(n_q, n_k, H, node_scores);
  size_t off = node_scores ? align256(size_t(H) * n_k * 4) : 0;
  if (L.sp.n_split > 1) {
    L.ml = off;
    off += align256(size_t(L.sp.n_split) * n_q * H * 8);
    L.acc = off;
    off += align256(size_t(L.sp.n_split) * n_q * H * d * 4);
  }
  L.total = off;
  return L;
}

size_t fwd_need(int dtype, int32_t n_q, int32_t n_k, int32_t H, int32_t d, bool node_scores) {
  if (use_mfma(dtype, d)) return mf_fwd_layout(n_q, n_k, H, d, node_scores).total;
  return node_scores || key_split(n_q, n_k, H).n_split > 1 ? fwd_ws(n_q, n_k, H, d) : 0;
}

// Backward workspace: D_i [n_q, H] fp32, and on the matrix-core path after it
// the key splits' partial dQ (two passes) or the key blocks' partial dQ
// (single pass).
size_t bwd_need(int dtype, int32_t n_q, int32_t n_k, int32_t H, int32_t d) {
  size_t need = bwd_ws(n_q, H);
  if (use_mfma(dtype, d) && n_q > 0) {
    const int fb = mfma_fused_blocks(n_q, n_k, H, d);
    const MfSplit sq = mfma_dq_split(n_q, n_k, H);
    const int parts = fb > 0 ? fb : (sq.n_split > 1 ? sq.n_split : 0);
    if (parts > 0) need += align256(size_t(parts) * n_q * H * d * 4);
  }
  return need;
}

template <int DH>
void launch_mf_combine(const float* part_ml, const float* part_acc, int n_split, int n_q, int H,
                       void* out, float* out32, float* lse, hipStream_t st) {
  int64_t blocks = (int64_t(n_q) * H + kBlock - 1) / kBlock;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((k_dense_combine<bf16_t, DH>), dim3(int(blocks)), dim3(kBlock), 0, st,
                     part_ml, part_acc, n_split, n_q, H, static_cast<bf16_t*>(out), out32, lse);
}

__global__ void k_fill_zero(float* __restrict__ p, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_dense_workspace_bytes(int dtype, int32_t n_q, int32_t n_k, int32_t n_heads,
                                         int32_t head_dim, int32_t node_scores,
                                         size_t* fwd_bytes, size_t* bwd_bytes) {
  const int rc = check_args("ngt_dense_workspace_bytes", dtype, n_q, n_k, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (fwd_bytes) *fwd_bytes = n_q > 0 ? fwd_need(dtype, n_q, n_k, n_heads, head_dim, node_scores != 0) : 0;
  if (bwd_bytes) *bwd_bytes = bwd_need(dtype, n_q, n_k, n_heads, head_dim);
  return NGT_OK;
}

extern "C" int ngt_dense_fwd(int dtype, const void* q, const void* k, const void* v, int32_t n_q,
                             int32_t n_k, int32_t n_heads, int32_t head_dim, float scale,
                             float dropout_p, uint64_t seed, const uint64_t* seed_dev,
                             void* out, float* out_f32, float* lse, float* node_score,
                             void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_args("ngt_dense_fwd", dtype, n_q, n_k, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (!(scale > 0.f)) return set_error(NGT_ERR_ARG, "ngt_dense_fwd: scale must be > 0");
  DropoutMask dmv{};
  bool drop = false;
  NGT_CHECK_OK(make_dropout("ngt_dense_fwd", dropout_p, seed, seed_dev, n_q, n_k, &dmv, &drop));
  const DropoutMask* dm = drop ? &dmv : nullptr;
  if (n_q > 0 && (!q || !out || !lse)) return set_error(NGT_ERR_ARG, "ngt_dense_fwd: null q/out/lse");
  if (n_k > 0 && (!k || !v)) return set_error(NGT_ERR_ARG, "ngt_dense_fwd: null k/v");
  if (n_q > 0) {
    const size_t need = fwd_need(dtype, n_q, n_k, n_heads, head_dim, node_score != nullptr);
    if (need && (!workspace || workspace_bytes < need))
      return set_error(NGT_ERR_WORKSPACE, "ngt_dense_fwd: workspace %zu < %zu", workspace_bytes,
                       need);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (node_score && n_q == 0 && n_k > 0) {  // no queries: every column score is 0
    hipLaunchKernelGGL(k_fill_zero, dim3(unsigned((n_k + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                       st, node_score, int64_t(n_k));
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (use_mfma(dtype, head_dim)) {
    if (n_q == 0) return NGT_OK;
    float* part = node_score ? static_cast<float*>(workspace) : nullptr;
    const MfFwdLayout L = mf_fwd_layout(n_q, n_k, n_heads, head_dim, node_score != nullptr);
    char* ws = static_cast<char*>(workspace);
    float* part_ml = L.sp.n_split > 1 ? reinterpret_cast<float*>(ws + L.ml) : nullptr;
    float* part_acc = L.sp.n_split > 1 ? reinterpret_cast<float*>(ws + L.acc) : nullptr;
    rc = mfma_dense_fwd(head_dim, q, k, v, n_q, n_k, n_heads, scale, dm, out, out_f32, lse, part,
                        L.sp, part_ml, part_acc, st);
    if (rc != NGT_OK) return rc;
    if (L.sp.n_split > 1) {
      KernelTimer timer_("dense_combine", st);
      switch (head_dim) {
        case 8: launch_mf_combine<8>(part_ml, part_acc, L.sp.n_split, n_q, n_heads, out, out_f32, lse, st); break;
        case 16: launch_mf_combine<16>(part_ml, part_acc, L.sp.n_split, n_q, n_heads, out, out_f32, lse, st); break;
        case 24: launch_mf_combine<24>(part_ml, part_acc, L.sp.n_split, n_q, n_heads, out, out_f32, lse, st); break;
        default: launch_mf_combine<32>(part_ml, part_acc, L.sp.n_split, n_q, n_heads, out, out_f32, lse, st); break;
      }
      NGT_HIP_CHECK(hipGetLastError());
    }
    if (!node_score || n_k == 0) return NGT_OK;
    hipLaunchKernelGGL(k_dense_scores, dim3((n_k + kWave - 1) / kWave), dim3(kScoreThreads), 0, st,
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
                             float dropout_p, uint64_t seed, const uint64_t* seed_dev,
                             void* grad_q, void* grad_k, void* grad_v, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc = check_args("ngt_dense_bwd", dtype, n_q, n_k, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (!(scale > 0.f)) return set_error(NGT_ERR_ARG, "ngt_dense_bwd: scale must be > 0");
  DropoutMask dmv{};
  bool drop = false;
  NGT_CHECK_OK(make_dropout("ngt_dense_bwd", dropout_p, seed, seed_dev, n_q, n_k, &dmv, &drop));
  const DropoutMask* dm = drop ? &dmv : nullptr;
  if (n_q > 0 && (!q || (!out && !out_f32) || !grad_out || !lse || !grad_q))
    return set_error(NGT_ERR_ARG, "ngt_dense_bwd: null query-side pointer");
  if (n_k > 0 && (!k || !v || !grad_k || !grad_v))
    return set_error(NGT_ERR_ARG, "ngt_dense_bwd: null key-side pointer");
  const size_t need = bwd_need(dtype, n_q, n_k, n_heads, head_dim);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(NGT_ERR_WORKSPACE, "ngt_dense_bwd: workspace %zu < %zu", workspace_bytes,
                     need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_mfma(dtype, head_dim)) {
    float* dsum = static_cast<float*>(workspace);  // written by the dQ pass
    const MfSplit sq = n_q > 0 ? mfma_dq_split(n_q, n_k, n_heads) : MfSplit{1, 1};
    const int fb = mfma_fused_blocks(n_q, n_k, n_heads, head_dim);
    float* part_dq = sq.n_split > 1 || fb > 0
                         ? reinterpret_cast<float*>(static_cast<char*>(workspace) + bwd_ws(n_q, n_heads))
                         : nullptr;
    return mfma_dense_bwd(head_dim, q, k, v, grad_out, out, out_f32, lse, dsum, n_q, n_k,
                          n_heads, scale, dm, grad_q, grad_k, grad_v, sq, part_dq, fb, st);
  }
  return dispatch<BwdOp>(dtype, head_dim, q, k, v, out, out_f32, grad_out, lse, int(n_q), int(n_k),
                         int(n_heads), scale, dm, grad_q, grad_k, grad_v,
                         static_cast<char*>(workspace), st);
}
