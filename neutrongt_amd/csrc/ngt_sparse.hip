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
// fixed-size chunks whose partials a finalize kernel adds.
//
// Wave layout: lane = slot * L + hl with L = next_pow2(heads per pass) lanes
// per edge and S = 64 / L edge slots per wave.  Each lane owns one head of one
// edge and the d-element head slice of every gathered row, so the L lanes of a
// slot read one contiguous segment of a K/V row per edge.
//
// Head groups: a launch can walk the work list once per group of `hg` heads,
// so that one pass gathers only hg*d-element row slices (heads_per_pass has
// the per-kernel widths and the measurement behind them; virtual_wave the
// order in which groups are dealt to the XCDs).
#include "ngt_common.h"

#include <stdlib.h>

#include <type_traits>
#include <utility>

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kColTile = kWave;  // finalize: columns per block

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

// Sum of x[p * stride] for p = first, first + step, ... < n, added in that
// order.  The loads go out in batches of 8, so a split row's many partials
// are not one chain of dependent loads; the additions keep the plain loop's
// order (the same bits).
__device__ __forceinline__ float strided_sum(const float* __restrict__ x, int first, int n,
                                             int step, int64_t stride) {
  constexpr int B = 8;
  float a = 0.f;
  for (int p0 = first; p0 < n; p0 += B * step) {
    float v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int p = p0 + u * step;
      v[u] = p < n ? x[int64_t(p) * stride] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (p0 + u * step < n) a += v[u];
  }
  return a;
}

// Key rows: rows j < n_main of k/v, then rows j - n_main of k_ext/v_ext (a
// second buffer, e.g. the detached cache of related keys, so the caller need
// not concatenate it).  With one buffer k_ext = k, v_ext = v and n_main = n_k.
// Gradients exist only for the rows of k/v (the second buffer is constant).
// The per-edge gathers of the query-major kernels are instantiated with and
// without the second buffer (EXT): the select costs 2-5 % of the forward.
// With two buffers the forward takes 132 VGPRs against 108 (one wave less per
// SIMD; about 5 % of its time in the window step), whether the gathers select
// a base or branch; capping it at 128 spills.
template <typename T, bool EXT = true>
struct Keys {
  const T* k;
  const T* v;
  const T* k_ext;
  const T* v_ext;
  int64_t n_main;

  template <int DH>
  __device__ __forceinline__ const T* krow(int64_t j, int H, int h) const {
    if (!EXT || j < n_main) return k + (j * H + h) * DH;
    return k_ext + ((j - n_main) * H + h) * DH;
  }
  template <int DH>
  __device__ __forceinline__ const T* vrow(int64_t j, int H, int h) const {
    if (!EXT || j < n_main) return v + (j * H + h) * DH;
    return v_ext + ((j - n_main) * H + h) * DH;
  }
  // K and V words of key row j for head h
  template <int DH>
  __device__ __forceinline__ void load_kv(int64_t j, int H, int h, RowWords<T, DH>& kw,
                                          RowWords<T, DH>& vw) const {
    if (!EXT || j < n_main) {
      load_words<T, DH>(k + (j * H + h) * DH, kw);
      load_words<T, DH>(v + (j * H + h) * DH, vw);
    } else {
      load_words<T, DH>(k_ext + ((j - n_main) * H + h) * DH, kw);
      load_words<T, DH>(v_ext + ((j - n_main) * H + h) * DH, vw);
    }
  }
  template <int DH>
  __device__ __forceinline__ void load_k(int64_t j, int H, int h, RowWords<T, DH>& kw) const {
    if (!EXT || j < n_main)
      load_words<T, DH>(k + (j * H + h) * DH, kw);
    else
      load_words<T, DH>(k_ext + ((j - n_main) * H + h) * DH, kw);
  }
};

// Edges per slot whose row loads are issued together before any is used:
// as many as fit a budget of raw 16-byte words per lane (at most 4).
#ifndef NGT_FWD_WORDS
#define NGT_FWD_WORDS 16
#endif
#ifndef NGT_BWD_KV_WORDS
#define NGT_BWD_KV_WORDS 16
#endif
#ifndef NGT_BWD_Q_WORDS
#define NGT_BWD_Q_WORDS 16
#endif
constexpr int unroll_for(int words_per_edge, int budget) {
  return words_per_edge >= budget ? 1
                                  : (budget / words_per_edge >= 4 ? 4 : budget / words_per_edge);
}

// The key-major pass keeps at most 2 edges per slot in flight: on the
// high-degree window (bf16, d = 16, 4 words per edge) 4 took bwd_kv 100 ->
// 108 us per layer, GPH_Slim and the GT arxiv window read the same either way,
// and GPH_Large's 6-word edges already fit only 2.
constexpr int kv_unroll(int words_per_edge) {
  return unroll_for(words_per_edge, NGT_BWD_KV_WORDS) < 2 ? 1 : 2;
}

// Work decomposition shared by the edge kernels.
struct Lane {
  int slot;     // edge slot of this lane
  int S;        // edge slots per wave
  int h;        // head of this lane
  bool active;  // lane maps to a real head
};

// Wave id of this wave in the launch's work order [items of group 0 | items of
// group 1 | ... | packed waves of group 0 | ...], or -1 when it has none.
// xcd != 0 (n_groups divides 8): block b serves head group b % n_groups.  The
// dispatcher deals blocks to the eight XCDs round robin, so each XCD then
// gathers the row slices of one head group only and its L2 holds 8/n_groups
// times more rows of that slice.
__device__ __forceinline__ int64_t virtual_wave(int32_t n_items, int32_t n_pwaves,
                                                int32_t n_groups, int32_t xcd) {
  const int wv = threadIdx.x >> 6;
  if (!xcd) return int64_t(blockIdx.x) * kWavesPerBlock + wv;
  const int g = static_cast<int>(blockIdx.x % unsigned(n_groups));
  const int64_t w = int64_t(blockIdx.x / unsigned(n_groups)) * kWavesPerBlock + wv;
  if (w < n_items) return int64_t(g) * n_items + w;
  if (w - n_items < n_pwaves) return int64_t(n_items) * n_groups + int64_t(g) * n_pwaves + (w - n_items);
  return -1;
}

__device__ __forceinline__ bool wave_work(int64_t gw, int n_items, int n_groups, int hg, int L,
                                          int H, int& item, Lane& ln) {
  const int lane = threadIdx.x & (kWave - 1);
  if (n_items <= 0) return false;
  const int64_t group = gw / n_items;
  if (group >= n_groups) return false;
  item = static_cast<int>(gw - group * n_items);
  const int hl = lane & (L - 1);
  ln.slot = lane / L;
  ln.S = kWave / L;
  ln.h = static_cast<int>(group) * hg + hl;
  ln.active = hl < hg && ln.h < H;
  return true;
}

// Packed small rows: each edge slot of a wave owns one whole row.  Returns
// false for lanes without a row (they leave; packed mode uses no shuffles).
__device__ __forceinline__ bool packed_work(int64_t pw, int n_pwaves, int n_groups, int hg,
                                            int L, int H, const int32_t* __restrict__ packed,
                                            int n_packed, int64_t& row, int& h) {
  const int lane = threadIdx.x & (kWave - 1);
  if (n_pwaves <= 0) return false;
  const int64_t group = pw / n_pwaves;
  if (group >= n_groups) return false;
  const int64_t idx = pw - group * n_pwaves;
  const int hl = lane & (L - 1);
  const int64_t r_idx = idx * (kWave / L) + lane / L;
  h = static_cast<int>(group) * hg + hl;
  if (hl >= hg || h >= H || r_idx >= n_packed) return false;
  row = packed[r_idx];
  return true;
}

template <typename T, int DH, bool EXT, bool BIAS>
__device__ __forceinline__ float fwd_packed(const T* __restrict__ q, const Keys<T, EXT>& kv,
                                           const int32_t* __restrict__ rowptr,
                                           const int32_t* __restrict__ col, int64_t row, int h,
                                           int H, float inv_scale, float lo, float hi, float eps,
                                           T* __restrict__ out, float* __restrict__ rinv,
                                           float* __restrict__ zbuf, const float* __restrict__ eb) {
  RowWords<T, DH> qw;
  float acc[DH];
  float z = 0.f;
  load_words<T, DH>(q + (row * H + h) * DH, qw);
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  // U edges per round: their K/V loads are in flight together, and the
  // column indices of the next round are requested before this round's math.
  constexpr int U = unroll_for(2 * RowWords<T, DH>::NV, NGT_FWD_WORDS);
  const int beg = rowptr[row], end = rowptr[row + 1];
  int jn[U];
#pragma unroll
  for (int u = 0; u < U; ++u) jn[u] = beg + u < end ? col[beg + u] : -1;
  for (int e0 = beg; e0 < end; e0 += U) {
    RowWords<T, DH> kw[U], vw[U];
    int jc[U];
    float bu[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      jc[u] = jn[u];
      if (jc[u] >= 0) {
        kv.template load_kv<DH>(jc[u], H, h, kw[u], vw[u]);
        if constexpr (BIAS) bu[u] = eb[int64_t(e0 + u) * H + h];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) jn[u] = e0 + U + u < end ? col[e0 + U + u] : -1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (jc[u] >= 0) {
        float s = clampf(edge_dot<T, DH>(qw, kw[u]) * inv_scale, lo, hi);
        if constexpr (BIAS) s += bu[u];  // the bias is added after the clamp
        const float p = __expf(s);
        z += p;
#pragma unroll
        for (int c = 0; c < DH; ++c) acc[c] = fmaf(p, word_elem<T, DH>(vw[u], c), acc[c]);
      }
    }
  }
  const float den = z + eps;
  float o[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) o[c] = acc[c] / den;
  store_row<T, DH>(out + (row * H + h) * DH, o);
  rinv[row * H + h] = 1.0f / den;
  zbuf[row * H + h] = z;
  return z;
}

// ------------------------------------------------------------------ forward
// With one head group (every head of a row in one wave) the node score
// mean_h Z[i,h] of a row that is not split is reduced across the row's head
// lanes and written here; split rows get theirs in the finalize.  ns is null
// when no node scores are wanted or with several head groups (then the
// finalize launch computes them from zbuf).
template <typename T, int DH, bool EXT, bool BIAS>
__global__ __launch_bounds__(kBlock) void k_fwd(
    const T* __restrict__ q, const Keys<T, EXT> kv,
    const int32_t* __restrict__ col, const int4* __restrict__ items, int32_t n_items,
    int32_t n_groups, int32_t hg, int32_t H, int32_t L, float inv_scale, float lo, float hi,
    float eps, T* __restrict__ out, float* __restrict__ rinv, float* __restrict__ zbuf,
    float* __restrict__ part_acc, float* __restrict__ part_z, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ packed, int32_t n_packed, int32_t n_pwaves,
    float* __restrict__ ns, int32_t ns_len, int32_t xcd, const float* __restrict__ eb) {
  const int64_t gw = virtual_wave(n_items, n_pwaves, n_groups, xcd);
  if (gw < 0) return;
  if (gw >= int64_t(n_items) * n_groups) {
    int64_t prow = 0;
    int ph = 0;
    float z = 0.f;
    const bool has = packed_work(gw - int64_t(n_items) * n_groups, n_pwaves, n_groups, hg, L, H,
                                 packed, n_packed, prow, ph);
    if (has)
      z = fwd_packed<T, DH, EXT, BIAS>(q, kv, rowptr, col, prow, ph, H, inv_scale, lo, hi, eps,
                                       out, rinv, zbuf, eb);
    if (ns) {  // all lanes take part; lanes without a row add 0
      const float zs = reduce_heads(z, L);
      if (has && ph == 0 && prow < ns_len) ns[prow] = zs / float(H);
    }
    return;
  }
  int item;
  Lane ln;
  if (!wave_work(gw, n_items, n_groups, hg, L, H, item, ln)) return;
  const int4 it = items[item];
  const int64_t row = it.x;
  const int h = ln.h;
  const int S = ln.S;

  RowWords<T, DH> qw;
  float acc[DH];
  float z = 0.f;
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  if (ln.active)
    load_words<T, DH>(q + (row * H + h) * DH, qw);
  else
    zero_words<T, DH>(qw);

  // Column indices of 64 edges are loaded at once (one coalesced access) and
  // handed to the slots with ds_bpermute; then the K/V rows of U edges per
  // slot are requested before any of them is used.
  constexpr int NV = RowWords<T, DH>::NV;
  constexpr int U = unroll_for(2 * NV, NGT_FWD_WORDS);
  const int lane = threadIdx.x & (kWave - 1);
  // each 64-edge block's column indices are requested one block ahead
  int nx_j = lane < it.z - it.y ? col[it.y + lane] : 0;
  for (int blk = it.y; blk < it.z; blk += kWave) {
    const int nb = min(kWave, it.z - blk);
    const int my_j = nx_j;
    nx_j = lane < it.z - blk - kWave ? col[blk + kWave + lane] : 0;
    for (int t0 = 0; t0 < nb; t0 += S * U) {
      RowWords<T, DH> kw[U], vw[U];
      bool ok[U];
      float bu[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = t0 + u * S + ln.slot;
        ok[u] = t < nb && ln.active;
        const int64_t j = __shfl(my_j, t < nb ? t : 0, kWave);
        if (ok[u]) {
          kv.template load_kv<DH>(j, H, h, kw[u], vw[u]);
          if constexpr (BIAS) bu[u] = eb[int64_t(blk + t) * H + h];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (ok[u]) {
          float s = clampf(edge_dot<T, DH>(qw, kw[u]) * inv_scale, lo, hi);
          if constexpr (BIAS) s += bu[u];  // the bias is added after the clamp
          const float p = __expf(s);
          z += p;
#pragma unroll
          for (int c = 0; c < DH; ++c) acc[c] = fmaf(p, word_elem<T, DH>(vw[u], c), acc[c]);
        }
      }
    }
  }

  reduce_slots<DH>(acc, z, L);
  const float zs = ns && it.w < 0 ? reduce_heads(z, L) : 0.f;  // inactive lanes hold 0
  if (ln.slot != 0 || !ln.active) return;
  if (it.w < 0) {
    const float den = z + eps;
    float o[DH];
#pragma unroll
    for (int c = 0; c < DH; ++c) o[c] = acc[c] / den;
    store_row<T, DH>(out + (row * H + h) * DH, o);
    rinv[row * H + h] = 1.0f / den;
    zbuf[row * H + h] = z;
    if (ns && h == 0 && row < ns_len) ns[row] = zs / float(H);
  } else {
    const int64_t p = int64_t(it.w) * H + h;
    store_f32<DH>(part_acc + p * DH, acc);
    part_z[p] = z;
  }
}

// Split rows: column c of the H*DH output columns of row sp.x is the sum of
// that column over the row's partial slots.  Blocks [0, n_splits * tiles) take
// (split row, 64-column tile); the 4 waves of a block take every 4th part and
// meet in LDS.  Tile 0 of a split row also writes its node score from the
// parts' Z.  The launch's first ns_blocks blocks (dispatched first, so they
// overlap the tiles) write the node scores of the rows that are not split
// (degree <= chunk) from zbuf, which the forward kernel has completed; split
// rows are left to their tile 0.
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_fwd_finalize(
    const int4* __restrict__ splits, int32_t tiles, int32_t H, float eps,
    const float* __restrict__ part_acc, const float* __restrict__ part_z, T* __restrict__ out,
    float* __restrict__ rinv, float* __restrict__ zbuf, float* __restrict__ ns, int32_t ns_len,
    const int32_t* __restrict__ rowptr, int32_t chunk, int32_t ns_blocks) {
  __shared__ float red[3][kWavesPerBlock][kColTile];
  if (int32_t(blockIdx.x) < ns_blocks) {
    const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= ns_len || rowptr[i + 1] - rowptr[i] > chunk) return;
    ns[i] = strided_sum(zbuf + i * H, 0, H, 1, 1) / float(H);
    return;
  }
  const unsigned fb = blockIdx.x - unsigned(ns_blocks);
  const int split = int(fb / unsigned(tiles));
  const int tile = int(fb % unsigned(tiles));
  const int4 sp = splits[split];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  // node score of the split row (tile 0 only): lanes = heads (H <= 64), the 4
  // waves take every 4th part, meet in LDS below
  const bool want_ns = ns && tile == 0 && sp.x < ns_len;
  if (want_ns) {
    const float zh = lane < H ? strided_sum(part_z + int64_t(sp.y) * H + lane, wave, sp.z,
                                            kWavesPerBlock, H)
                              : 0.f;
    red[2][wave][lane] = zh;
  }
  const int ncols = H * DH;
  const int col = tile * kColTile + lane;
  const bool ok = col < ncols;
  const int h = ok ? col / DH : 0;
  float a = 0.f, z = 0.f;
  if (ok) {
    a = strided_sum(part_acc + int64_t(sp.y) * ncols + col, wave, sp.z, kWavesPerBlock, ncols);
    z = strided_sum(part_z + int64_t(sp.y) * H + h, wave, sp.z, kWavesPerBlock, H);
  }
  red[0][wave][lane] = a;
  red[1][wave][lane] = z;
  __syncthreads();
  if (want_ns && wave == kWavesPerBlock - 1) {
    float zh = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) zh += red[2][w][lane];
    for (int off = 1; off < kWave; off <<= 1) zh += shfl_xor(zh, off);
    if (lane == 0) ns[sp.x] = zh / float(H);
  }
  if (wave != 0 || !ok) return;
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) {
    a += red[0][w][lane];
    z += red[1][w][lane];
  }
  const int64_t row = sp.x;
  const float den = z + eps;
  elem<T>::store(out + row * ncols + col, a / den);
  if (col % DH == 0) {
    rinv[row * H + h] = 1.0f / den;
    zbuf[row * H + h] = z;
  }
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

// da_e into ds.  NT: as a non-temporal store, which keeps a large ds from
// streaming through the L2 and evicting the Q / dO rows the pass gathers (a
// template flag: chosen at run time, the two stores fold into one plain store).
template <bool NT>
__device__ __forceinline__ void store_da(float* __restrict__ ds, int64_t i, float da) {
  if constexpr (NT)
    __builtin_nontemporal_store(da, ds + i);
  else
    ds[i] = da;
}

// The per-row statistics {r, r D} of a query, D = dO . out per head: read
// from rd (k_rowstat's output), or with FOLD formed at the edge from the
// query's out row and rinv with k_rowstat's own arithmetic (the same bits),
// which saves the k_rowstat launch where a window's key-major pass is one
// round of waves and its time a launch's fixed cost.
struct FoldArgs {
  const void* out;     // [N_q, H, d] of the element type
  const float* rinv;   // 1 / (Z + eps) per (query, head)
};

template <typename T, int DH, bool FOLD>
struct RowStat {
  RowWords<T, DH> ow;
  float2 r;
  __device__ __forceinline__ void load(const float2* __restrict__ rd, const FoldArgs& fa,
                                       int64_t i, int H, int h) {
    if constexpr (FOLD) {
      load_words<T, DH>(static_cast<const T*>(fa.out) + (i * H + h) * DH, ow);
      r.x = fa.rinv[i * H + h];
    } else {
      r = rd[i * H + h];
    }
  }
  // {r, r D} once the row's dO words gw have arrived
  __device__ __forceinline__ float2 get(const RowWords<T, DH>& gw) const {
    if constexpr (FOLD) {
      float o[DH], gg[DH];
      words_to_f32<T, DH>(ow, o);
      words_to_f32<T, DH>(gw, gg);
      return make_float2(r.x, r.x * dot<DH>(o, gg));
    } else {
      return r;
    }
  }
};

template <typename T, int DH, bool BIAS, bool NT, bool FOLD>
__device__ __forceinline__ void bwd_kv_packed(
    const T* __restrict__ q, const Keys<T>& kv,
    const T* __restrict__ g, const float2* __restrict__ rd, const int32_t* __restrict__ t_rowptr,
    const int32_t* __restrict__ t_col, int64_t row, int h, int H, float inv_scale, float lo,
    float hi, T* __restrict__ grad_k, T* __restrict__ grad_v, int64_t ldg,
    float* __restrict__ ds, const float* __restrict__ eb, float* __restrict__ deb,
    const FoldArgs& fa) {
  RowWords<T, DH> krw, vrw;
  float dk[DH], dv[DH];
  load_words<T, DH>(kv.template krow<DH>(row, H, h), krw);
  load_words<T, DH>(kv.template vrow<DH>(row, H, h), vrw);
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dk[c] = 0.f;
    dv[c] = 0.f;
  }
  constexpr int U = kv_unroll(2 * RowWords<T, DH>::NV);
  const int beg = t_rowptr[row], end = t_rowptr[row + 1];
  int in_[U];
#pragma unroll
  for (int u = 0; u < U; ++u) in_[u] = beg + u < end ? t_col[beg + u] : -1;
  for (int e0 = beg; e0 < end; e0 += U) {
    RowWords<T, DH> qw[U], gw[U];
    RowStat<T, DH, FOLD> rs[U];
    int ic[U];
    float bu[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ic[u] = in_[u];
      if (ic[u] >= 0) {
        const int64_t i = ic[u];
        load_words<T, DH>(q + (i * H + h) * DH, qw[u]);
        load_words<T, DH>(g + (i * H + h) * DH, gw[u]);
        rs[u].load(rd, fa, i, H, h);
        if constexpr (BIAS) bu[u] = eb[int64_t(e0 + u) * H + h];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) in_[u] = e0 + U + u < end ? t_col[e0 + U + u] : -1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (ic[u] >= 0) {
        const float2 r = rs[u].get(gw[u]);
        const float a = edge_dot<T, DH>(qw[u], krw) * inv_scale;
        float s = clampf(a, lo, hi);
        if constexpr (BIAS) s += bu[u];
        const float p = __expf(s);
        const float dp = r.x * edge_dot<T, DH>(gw[u], vrw) - r.y;
        const float da = (a >= lo && a <= hi) ? dp * p : 0.f;
        if constexpr (BIAS) {  // the bias's gradient: the score's, without the clamp mask
          if (deb) deb[int64_t(e0 + u) * H + h] = dp * p;
        }
        const float pr = p * r.x;
#pragma unroll
        for (int c = 0; c < DH; ++c) {
          dk[c] = fmaf(da, word_elem<T, DH>(qw[u], c), dk[c]);
          dv[c] = fmaf(pr, word_elem<T, DH>(gw[u], c), dv[c]);
        }
        if (ds) store_da<NT>(ds, int64_t(e0 + u) * H + h, da);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) dk[c] *= inv_scale;
  if (row >= kv.n_main) return;  // constant key rows: no gradient
  store_row<T, DH>(grad_k + row * ldg + h * DH, dk);
  store_row<T, DH>(grad_v + row * ldg + h * DH, dv);
}

// Key-major pass: grad_k, grad_v of key row j and da_e for every edge of j
// (stored at the key-major edge position for the query-major pass; ds is null
// when that pass recomputes da_e itself).
template <typename T, int DH, bool BIAS, bool NT, bool FOLD>
__global__ __launch_bounds__(kBlock) void k_bwd_kv(
    const T* __restrict__ q, const Keys<T> kv,
    const T* __restrict__ g, const float2* __restrict__ rd, const int32_t* __restrict__ t_col,
    const int4* __restrict__ items, int32_t n_items, int32_t n_groups, int32_t hg, int32_t H,
    int32_t L, float inv_scale, float lo, float hi, T* __restrict__ grad_k,
    T* __restrict__ grad_v, int64_t ldg, float* __restrict__ ds, float* __restrict__ part_kv,
    const int32_t* __restrict__ t_rowptr, const int32_t* __restrict__ packed, int32_t n_packed,
    int32_t n_pwaves, int32_t xcd, const float* __restrict__ eb, float* __restrict__ deb,
    int32_t row_min, const FoldArgs fa) {
  // key rows < row_min are left to another pass (the tiled one)
  const int64_t gw0 = virtual_wave(n_items, n_pwaves, n_groups, xcd);
  if (gw0 < 0) return;
  if (gw0 >= int64_t(n_items) * n_groups) {
    int64_t prow;
    int ph;
    if (packed_work(gw0 - int64_t(n_items) * n_groups, n_pwaves, n_groups, hg, L, H, packed,
                    n_packed, prow, ph) && prow >= row_min)
      bwd_kv_packed<T, DH, BIAS, NT, FOLD>(q, kv, g, rd, t_rowptr, t_col, prow, ph, H, inv_scale,
                                           lo, hi, grad_k, grad_v, ldg, ds, eb, deb, fa);
    return;
  }
  int item;
  Lane ln;
  if (!wave_work(gw0, n_items, n_groups, hg, L, H, item, ln)) return;
  const int4 it = items[item];
  const int64_t row = it.x;
  if (row < row_min) return;  // uniform per wave
  const int h = ln.h;
  const int S = ln.S;

  RowWords<T, DH> krw, vrw;
  float dk[DH], dv[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dk[c] = 0.f;
    dv[c] = 0.f;
  }
  if (ln.active) {
    load_words<T, DH>(kv.template krow<DH>(row, H, h), krw);
    load_words<T, DH>(kv.template vrow<DH>(row, H, h), vrw);
  } else {
    zero_words<T, DH>(krw);
    zero_words<T, DH>(vrw);
  }
  constexpr int NV = RowWords<T, DH>::NV;
  constexpr int U = kv_unroll(2 * NV);
  const int lane = threadIdx.x & (kWave - 1);
  // each 64-edge block's row indices are requested one block ahead
  int nx_i = lane < it.z - it.y ? t_col[it.y + lane] : 0;
  for (int blk = it.y; blk < it.z; blk += kWave) {
    const int nb = min(kWave, it.z - blk);
    const int my_i = nx_i;
    nx_i = lane < it.z - blk - kWave ? t_col[blk + kWave + lane] : 0;
    for (int t0 = 0; t0 < nb; t0 += S * U) {
      RowWords<T, DH> qw[U], gw[U];
      RowStat<T, DH, FOLD> rs[U];
      bool ok[U];
      float bu[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = t0 + u * S + ln.slot;
        ok[u] = t < nb && ln.active;
        const int64_t i = __shfl(my_i, t < nb ? t : 0, kWave);
        if (ok[u]) {
          load_words<T, DH>(q + (i * H + h) * DH, qw[u]);
          load_words<T, DH>(g + (i * H + h) * DH, gw[u]);
          rs[u].load(rd, fa, i, H, h);
          if constexpr (BIAS) bu[u] = eb[int64_t(blk + t) * H + h];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (ok[u]) {
          // rows stay packed; elements are unpacked at each use
          const float2 r = rs[u].get(gw[u]);
          const float a = edge_dot<T, DH>(qw[u], krw) * inv_scale;
          float s = clampf(a, lo, hi);
          if constexpr (BIAS) s += bu[u];
          const float p = __expf(s);
          const float dp = r.x * edge_dot<T, DH>(gw[u], vrw) - r.y;
          const float da = (a >= lo && a <= hi) ? dp * p : 0.f;
          if constexpr (BIAS) {  // the bias's gradient: the score's, without the clamp mask
            if (deb) deb[int64_t(blk + t0 + u * S + ln.slot) * H + h] = dp * p;
          }
          const float pr = p * r.x;
#pragma unroll
          for (int c = 0; c < DH; ++c) {
            dk[c] = fmaf(da, word_elem<T, DH>(qw[u], c), dk[c]);
            dv[c] = fmaf(pr, word_elem<T, DH>(gw[u], c), dv[c]);
          }
          if (ds) store_da<NT>(ds, int64_t(blk + t0 + u * S + ln.slot) * H + h, da);
        }
      }
    }
  }
  reduce_slots2<DH>(dk, dv, L);
  if (ln.slot != 0 || !ln.active) return;
#pragma unroll
  for (int c = 0; c < DH; ++c) dk[c] *= inv_scale;
  if (it.w < 0) {
    if (row >= kv.n_main) return;  // constant key rows: no gradient
    store_row<T, DH>(grad_k + row * ldg + h * DH, dk);
    store_row<T, DH>(grad_v + row * ldg + h * DH, dv);
  } else {
    float* p = part_kv + (int64_t(it.w) * H + h) * (2 * DH);
    store_f32<DH>(p, dk);
    store_f32<DH>(p + DH, dv);
  }
}

// Split key rows: columns are (h, [dk | dv]) = 2*H*DH per part.
template <typename T, int DH>
__device__ __forceinline__ void bwd_kv_finalize_tile(const int4* __restrict__ splits, int32_t H,
                                                     const float* __restrict__ part_kv,
                                                     T* __restrict__ grad_k,
                                                     T* __restrict__ grad_v, int64_t ldg,
                                                     int64_t n_main, int split, int tile,
                                                     int32_t row_min) {
  __shared__ float red[kWavesPerBlock][kColTile];
  const int4 sp = splits[split];
  if (sp.x >= n_main) return;  // constant key row: no gradient (uniform per block)
  if (sp.x < row_min) return;  // a row another pass handles (uniform per block)
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int ncols = 2 * H * DH;
  const int col = tile * kColTile + lane;
  const bool ok = col < ncols;
  float a =
      ok ? strided_sum(part_kv + int64_t(sp.y) * ncols + col, wave, sp.z, kWavesPerBlock, ncols)
         : 0.f;
  red[wave][lane] = a;
  __syncthreads();
  if (wave != 0 || !ok) return;
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) a += red[w][lane];
  const int h = col / (2 * DH);
  const int c = col - h * 2 * DH;
  const int64_t at = int64_t(sp.x) * ldg + h * DH;
  if (c < DH)
    elem<T>::store(grad_k + at + c, a);
  else
    elem<T>::store(grad_v + at + (c - DH), a);
}

// The query-major pass either reads each edge's da from ds (written by the
// key-major pass) or, with RC, recomputes it from the row's q, dO and {r, rD}
// and the edge's K and V rows.  The recomputation repeats the key-major
// pass's operations on the same operands in the same order (edge_dot, clamp,
// exp, the clamp mask), so da and hence dQ come out bit for bit the same.
struct RecomputeArgs {
  const void* q;        // [N_q, H, d] of the element type
  const void* g;        // dO, same layout
  const float2* rd;     // {r, r (dO . O)} per (query, head)
  float lo, hi;         // the score clamp
};

template <typename T, int DH>
__device__ __forceinline__ float recompute_da(const RowWords<T, DH>& qw, const RowWords<T, DH>& gw,
                                              float2 rr, const RowWords<T, DH>& kw,
                                              const RowWords<T, DH>& vw, float inv_scale,
                                              float lo, float hi) {
  const float a = edge_dot<T, DH>(qw, kw) * inv_scale;
  const float p = __expf(clampf(a, lo, hi));
  const float dp = rr.x * edge_dot<T, DH>(gw, vw) - rr.y;
  return (a >= lo && a <= hi) ? dp * p : 0.f;
}

template <typename T, int DH, bool EXT, bool RC>
__device__ __forceinline__ void bwd_q_packed(const Keys<T, EXT>& kv,
                                             const int32_t* __restrict__ rowptr,
                                             const int32_t* __restrict__ col,
                                             const int32_t* __restrict__ q2t,
                                             const float* __restrict__ ds, int64_t row, int h,
                                             int H, float inv_scale, T* __restrict__ grad_q,
                                             int64_t ldg, const RecomputeArgs& rc) {
  float dq[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) dq[c] = 0.f;
  RowWords<T, DH> qw, gw;
  float2 rr = make_float2(0.f, 0.f);
  if constexpr (RC) {
    load_words<T, DH>(static_cast<const T*>(rc.q) + (row * H + h) * DH, qw);
    load_words<T, DH>(static_cast<const T*>(rc.g) + (row * H + h) * DH, gw);
    rr = rc.rd[row * H + h];
  }
  constexpr int U = unroll_for((RC ? 2 : 1) * RowWords<T, DH>::NV, NGT_BWD_Q_WORDS);
  const int beg = rowptr[row], end = rowptr[row + 1];
  int jn[U], tn[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    jn[u] = beg + u < end ? col[beg + u] : -1;
    tn[u] = beg + u < end ? q2t[beg + u] : 0;
  }
  for (int e0 = beg; e0 < end; e0 += U) {
    RowWords<T, DH> kw[U], vw[RC ? U : 1];
    float d[U];
    int jc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      jc[u] = jn[u];
      if (jc[u] >= 0) {
        if constexpr (RC) {
          kv.template load_kv<DH>(jc[u], H, h, kw[u], vw[u]);
        } else {
          kv.template load_k<DH>(jc[u], H, h, kw[u]);
          d[u] = ds[int64_t(tn[u]) * H + h];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      jn[u] = e0 + U + u < end ? col[e0 + U + u] : -1;
      tn[u] = e0 + U + u < end ? q2t[e0 + U + u] : 0;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (jc[u] >= 0) {
        if constexpr (RC) d[u] = recompute_da<T, DH>(qw, gw, rr, kw[u], vw[u], inv_scale, rc.lo, rc.hi);
#pragma unroll
        for (int c = 0; c < DH; ++c) dq[c] = fmaf(d[u], word_elem<T, DH>(kw[u], c), dq[c]);
      }
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) dq[c] *= inv_scale;
  store_row<T, DH>(grad_q + row * ldg + h * DH, dq);
}

// Query-major pass: grad_q[i] = sum_e da_e k_j / scale.
template <typename T, int DH, bool EXT, bool RC>
__global__ __launch_bounds__(kBlock) void k_bwd_q(
    const Keys<T, EXT> kv, const int32_t* __restrict__ col, const int32_t* __restrict__ q2t,
    const float* __restrict__ ds, const int4* __restrict__ items, int32_t n_items,
    int32_t n_groups, int32_t hg, int32_t H, int32_t L, float inv_scale, T* __restrict__ grad_q,
    int64_t ldg, float* __restrict__ part_q, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ packed, int32_t n_packed, int32_t n_pwaves, int32_t q_blocks,
    const int4* __restrict__ splits_k, int32_t kv_tiles, const float* __restrict__ part_kv,
    T* __restrict__ grad_k, T* __restrict__ grad_v, int32_t xcd, const RecomputeArgs rc,
    int32_t kv_row_min) {
  // Blocks past the dQ work finish the split key rows of bwd_kv (their dK/dV
  // partials; rows >= kv_row_min): that work is independent of dQ, so it
  // rides in this launch.
  if (int32_t(blockIdx.x) >= q_blocks) {
    const int f = int(blockIdx.x) - q_blocks;
    bwd_kv_finalize_tile<T, DH>(splits_k, H, part_kv, grad_k, grad_v, ldg, kv.n_main,
                                f / kv_tiles, f % kv_tiles, kv_row_min);
    return;
  }
  const int64_t gw0 = virtual_wave(n_items, n_pwaves, n_groups, xcd);
  if (gw0 < 0) return;
  if (gw0 >= int64_t(n_items) * n_groups) {
    int64_t prow;
    int ph;
    if (packed_work(gw0 - int64_t(n_items) * n_groups, n_pwaves, n_groups, hg, L, H, packed,
                    n_packed, prow, ph))
      bwd_q_packed<T, DH, EXT, RC>(kv, rowptr, col, q2t, ds, prow, ph, H, inv_scale, grad_q, ldg,
                                   rc);
    return;
  }
  int item;
  Lane ln;
  if (!wave_work(gw0, n_items, n_groups, hg, L, H, item, ln)) return;
  const int4 it = items[item];
  const int64_t row = it.x;
  const int h = ln.h;
  const int S = ln.S;
  float dq[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) dq[c] = 0.f;
  RowWords<T, DH> qw, gw;
  float2 rr = make_float2(0.f, 0.f);
  if constexpr (RC) {
    if (ln.active) {
      load_words<T, DH>(static_cast<const T*>(rc.q) + (row * H + h) * DH, qw);
      load_words<T, DH>(static_cast<const T*>(rc.g) + (row * H + h) * DH, gw);
      rr = rc.rd[row * H + h];
    } else {
      zero_words<T, DH>(qw);
      zero_words<T, DH>(gw);
    }
  }
  constexpr int NV = RowWords<T, DH>::NV;
  constexpr int U = unroll_for((RC ? 2 : 1) * NV, NGT_BWD_Q_WORDS);
  const int lane = threadIdx.x & (kWave - 1);
  // each 64-edge block's column and key-major indices are requested one block ahead
  int nx_j = lane < it.z - it.y ? col[it.y + lane] : 0;
  int nx_t = lane < it.z - it.y ? q2t[it.y + lane] : 0;
  for (int blk = it.y; blk < it.z; blk += kWave) {
    const int nb = min(kWave, it.z - blk);
    const int my_j = nx_j, my_t = nx_t;
    nx_j = lane < it.z - blk - kWave ? col[blk + kWave + lane] : 0;
    nx_t = lane < it.z - blk - kWave ? q2t[blk + kWave + lane] : 0;
    for (int t0 = 0; t0 < nb; t0 += S * U) {
      RowWords<T, DH> kw[U], vw[RC ? U : 1];
      float dsv[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = t0 + u * S + ln.slot;
        ok[u] = t < nb && ln.active;
        const int src = t < nb ? t : 0;
        const int64_t j = __shfl(my_j, src, kWave);
        const int64_t tp = RC ? 0 : __shfl(my_t, src, kWave);
        if (ok[u]) {
          if constexpr (RC) {
            kv.template load_kv<DH>(j, H, h, kw[u], vw[u]);
          } else {
            kv.template load_k<DH>(j, H, h, kw[u]);
            dsv[u] = ds[tp * H + h];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (ok[u]) {
          if constexpr (RC)
            dsv[u] = recompute_da<T, DH>(qw, gw, rr, kw[u], vw[u], inv_scale, rc.lo, rc.hi);
#pragma unroll
          for (int c = 0; c < DH; ++c) dq[c] = fmaf(dsv[u], word_elem<T, DH>(kw[u], c), dq[c]);
        }
      }
    }
  }
  reduce_slots1<DH>(dq, L);
  if (ln.slot != 0 || !ln.active) return;
#pragma unroll
  for (int c = 0; c < DH; ++c) dq[c] *= inv_scale;
  if (it.w < 0)
    store_row<T, DH>(grad_q + row * ldg + h * DH, dq);
  else
    store_f32<DH>(part_q + (int64_t(it.w) * H + h) * DH, dq);
}

template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_bwd_q_finalize(const int4* __restrict__ splits,
                                                           int32_t H,
                                                           const float* __restrict__ part_q,
                                                           T* __restrict__ grad_q, int64_t ldg) {
  __shared__ float red[kWavesPerBlock][kColTile];
  const int4 sp = splits[blockIdx.x];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int ncols = H * DH;
  const int col = blockIdx.y * kColTile + lane;
  const bool ok = col < ncols;
  float a = ok ? strided_sum(part_q + int64_t(sp.y) * ncols + col, wave, sp.z, kWavesPerBlock,
                            ncols)
               : 0.f;
  red[wave][lane] = a;
  __syncthreads();
  if (wave != 0 || !ok) return;
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) a += red[w][lane];
  elem<T>::store(grad_q + int64_t(sp.x) * ldg + col, a);
}

// ------------------------------------------------------ tiled (dense windows)
// On windows where a large share of the possible (query, key) pairs are edges
// (the high-degree GT windows: about 7 % of the in-window pairs), the
// work-list kernels' row gathers nearly all hit the L2 and run at its request
// rate.  The tiled kernels read each row slice once per block of rows
// instead.  A block owns QB = 4 * S rows (taken in descending degree order,
// so that its rows have similar degrees), one head group of hg heads and one
// part of the swept column range.  It walks the part in column blocks: the
// block first copies the column block's row slices into LDS with coalesced
// loads, then every edge slot walks its own row's edges into the column block
// (columns are sorted within a row) and reads the other side's slices from
// LDS.  A row's accumulators stay in registers for the whole part; the
// parts' sums are added in part order by a finalize kernel, so the result is
// deterministic and no atomics are used.  The number of parts of a row block
// follows the degree of its first (longest) row, about e_slot edges per slot
// and part, so that blocks of hub rows are cut finer than the rest.
//
// Query-major (k_q_tiled): rows are queries, columns keys, the swept columns
// [0, n_sweep) with n_sweep = min(n_q, n_k) (the window's own nodes); K and V
// slices are staged.  The sparse columns >= n_sweep (related keys) are
// gathered from global memory by the last part.  MODE 0 is the forward
// (partials of sum p v and Z), MODE 1 the dQ pass with each edge's da
// recomputed from K and V (partials of sum da k).
// Key-major (k_kv_tiled): rows are the keys j < n_sweep, columns every query;
// Q and dO slices and {r, rD} are staged.  Partials are indexed by the row's
// position in the degree order.

// First position p in [lo, hi) with col[p] >= x (hi if none); col sorted.
__device__ __forceinline__ int lower_bound_col(const int32_t* __restrict__ col, int lo, int hi,
                                               int x) {
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (col[mid] < x) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Parts of the row block whose first (longest) row sits at order position
// `first`: ceil(degree / e_slot), at least 1, at most p_max and the number
// of column blocks.
__device__ __forceinline__ int tile_row_parts(const int32_t* __restrict__ rowptr,
                                              const int32_t* __restrict__ order, int64_t first,
                                              int e_slot, int p_max, int n_cols, int kb) {
  const int64_t r0 = order[first];
  const int deg = rowptr[r0 + 1] - rowptr[r0];
  const int nb = (n_cols + kb - 1) / kb;
  int p = (deg + e_slot - 1) / e_slot;
  p = min(p, min(p_max, nb));
  return p < 1 ? 1 : p;
}

// Slot geometry of a tiled block: lane -> (slot, head); block -> (row block,
// part, head group) with the head group fastest.  Blocks past their row
// block's part count are empty (live false: they leave before any barrier).
struct TileTask {
  int g, part, n_parts, hl, h, slot, c0, c1;
  int64_t ridx;
  bool act, live;
};

__device__ __forceinline__ TileTask tile_task(const int32_t* __restrict__ rowptr,
                                              const int32_t* __restrict__ order, int n_rows,
                                              int n_cols, int n_groups, int p_max, int e_slot,
                                              int hg, int L, int kb) {
  TileTask t;
  const unsigned per_rb = unsigned(n_groups * p_max);
  const int gp = int(blockIdx.x % per_rb);
  const int64_t rb = int64_t(blockIdx.x / per_rb);
  t.g = gp % n_groups;
  t.part = gp / n_groups;
  const int S = kWave / L;
  const int64_t rows_per_block = int64_t(kWavesPerBlock) * S;
  t.n_parts = tile_row_parts(rowptr, order, rb * rows_per_block, e_slot, p_max, n_cols, kb);
  t.live = t.part < t.n_parts;
  int cols = (n_cols + t.n_parts - 1) / t.n_parts;
  cols = (cols + kb - 1) / kb * kb;
  t.c0 = min(n_cols, t.part * cols);
  t.c1 = min(n_cols, t.c0 + cols);
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  t.hl = lane & (L - 1);
  t.slot = lane / L;
  t.h = t.g * hg + t.hl;
  t.act = t.hl < hg;
  t.ridx = rb * rows_per_block + int64_t(wave) * S + t.slot;
  (void)n_rows;
  return t;
}

template <typename T, int DH>
__device__ __forceinline__ void lds_words(const uint4* __restrict__ p, RowWords<T, DH>& r) {
#pragma unroll
  for (int i = 0; i < RowWords<T, DH>::NV; ++i) r.w[i] = p[i];
}

// Loads per thread (of each staged tensor) in flight before the stores to LDS.
constexpr int kStageBatch = 4;

// Copies words t = threadIdx.x, + kBlock, ... < n of two tensors to LDS in
// batches of B per thread: load(t, a, b) reads them, store(t, a, b) writes
// them; the B loads of a batch are issued before its first store.
template <int B, typename Load, typename Store>
__device__ __forceinline__ void stage_words(int n, Load load, Store store) {
  for (int t0 = threadIdx.x; t0 < n; t0 += B * kBlock) {
    uint4 a0, b0, a1, b1, a2, b2, a3, b3;
    static_assert(B == 4, "four words per batch");
    const int t1 = t0 + kBlock, t2 = t0 + 2 * kBlock, t3 = t0 + 3 * kBlock;
    if (t0 < n) load(t0, a0, b0);
    if (t1 < n) load(t1, a1, b1);
    if (t2 < n) load(t2, a2, b2);
    if (t3 < n) load(t3, a3, b3);
    if (t0 < n) store(t0, a0, b0);
    if (t1 < n) store(t1, a1, b1);
    if (t2 < n) store(t2, a2, b2);
    if (t3 < n) store(t3, a3, b3);
  }
}

// Staged slices are padded by one 16-byte word per column, so that the
// slices of consecutive columns start in different LDS banks.
template <typename T, int DH>
__host__ __device__ constexpr int tile_stride(int hg) {
  return hg * RowWords<T, DH>::NV + 1;
}

template <typename T, int DH, bool EXT, int MODE>
__global__ __launch_bounds__(kBlock) void k_q_tiled(
    const T* __restrict__ q, const Keys<T, EXT> kv, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ col, const int32_t* __restrict__ order, int32_t n_q,
    int32_t n_sweep, int32_t H, int32_t hg, int32_t L, int32_t n_groups, int32_t p_max,
    int32_t e_slot, int32_t kb, float inv_scale, float lo, float hi, const RecomputeArgs rc,
    float* __restrict__ part_acc, float* __restrict__ part_z) {
  extern __shared__ uint4 stage[];
  constexpr int NV = RowWords<T, DH>::NV;
  constexpr int U = unroll_for(2 * NV, NGT_FWD_WORDS);
  const TileTask tk = tile_task(rowptr, order, n_q, n_sweep, n_groups, p_max, e_slot, hg, L, kb);
  if (!tk.live) return;  // uniform over the block
  const bool work = tk.ridx < n_q && tk.act;
  const int64_t row = work ? order[tk.ridx] : 0;
  const int h = tk.h;
  int pos = 0, pend = 0, tail_end = 0;
  if (work) {
    const int beg = rowptr[row], end = rowptr[row + 1];
    pos = lower_bound_col(col, beg, end, tk.c0);
    pend = lower_bound_col(col, pos, end, tk.c1);
    tail_end = tk.part == tk.n_parts - 1 ? end : pend;  // the last part: columns >= n_sweep
  }
  RowWords<T, DH> qw, gw;
  float2 rr = make_float2(0.f, 0.f);
  if (work) {
    load_words<T, DH>((MODE == 0 ? q : static_cast<const T*>(rc.q)) + (row * H + h) * DH, qw);
    if constexpr (MODE == 1) {
      load_words<T, DH>(static_cast<const T*>(rc.g) + (row * H + h) * DH, gw);
      rr = rc.rd[row * H + h];
    }
  } else {
    zero_words<T, DH>(qw);
    zero_words<T, DH>(gw);
  }
  float acc[DH];
  float z = 0.f;
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  auto edge = [&](const RowWords<T, DH>& kw, const RowWords<T, DH>& vw) {
    if constexpr (MODE == 0) {
      const float p = __expf(clampf(edge_dot<T, DH>(qw, kw) * inv_scale, lo, hi));
      z += p;
#pragma unroll
      for (int c = 0; c < DH; ++c) acc[c] = fmaf(p, word_elem<T, DH>(vw, c), acc[c]);
    } else {
      const float d = recompute_da<T, DH>(qw, gw, rr, kw, vw, inv_scale, lo, hi);
#pragma unroll
      for (int c = 0; c < DH; ++c) acc[c] = fmaf(d, word_elem<T, DH>(kw, c), acc[c]);
    }
  };
  const int slice = hg * NV;                  // 16-byte words of one column's K (or V) slice
  const int stride = tile_stride<T, DH>(hg);  // padded
  uint4* ks = stage;
  uint4* vs = stage + int64_t(kb) * stride;
  for (int cb = tk.c0; cb < tk.c1; cb += kb) {
    const int nc = min(kb, tk.c1 - cb);
    __syncthreads();  // the previous column block's readers are done
    // kStageBatch words of K and of V per thread in flight before any is stored
    stage_words<kStageBatch>(nc * slice, [&](int t, uint4& a, uint4& b) {
      const int jl = t / slice, w = t - jl * slice;
      a = reinterpret_cast<const uint4*>(kv.template krow<DH>(cb + jl, H, tk.g * hg))[w];
      b = reinterpret_cast<const uint4*>(kv.template vrow<DH>(cb + jl, H, tk.g * hg))[w];
    }, [&](int t, const uint4& a, const uint4& b) {
      const int jl = t / slice, w = t - jl * slice;
      ks[jl * stride + w] = a;
      vs[jl * stride + w] = b;
    });
    __syncthreads();
    if (!work) continue;
    const int cend = cb + nc;
    // this round's and the next round's columns are in registers; the
    // round after that is requested while this one runs
    int cur[U], nxt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      cur[u] = pos + u < pend ? col[pos + u] : INT32_MAX;
      nxt[u] = pos + U + u < pend ? col[pos + U + u] : INT32_MAX;
    }
    for (;;) {
      int nn[U];
#pragma unroll
      for (int u = 0; u < U; ++u) nn[u] = pos + 2 * U + u < pend ? col[pos + 2 * U + u] : INT32_MAX;
      RowWords<T, DH> kw[U], vw[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (cur[u] < cend) {
          const int o = (cur[u] - cb) * stride + tk.hl * NV;
          lds_words<T, DH>(ks + o, kw[u]);
          lds_words<T, DH>(vs + o, vw[u]);
        }
      int took = 0;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (cur[u] < cend) {
          edge(kw[u], vw[u]);
          ++took;
        }
      pos += took;
      if (took < U) break;  // the row's next edge is in a later column block
#pragma unroll
      for (int u = 0; u < U; ++u) {
        cur[u] = nxt[u];
        nxt[u] = nn[u];
      }
    }
  }
  if (!work) return;
  // columns >= n_sweep: gathered from global memory (the last part)
  for (int e0 = pend; e0 < tail_end; e0 += U) {
    RowWords<T, DH> kw[U], vw[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = e0 + u < tail_end;
      if (ok[u]) kv.template load_kv<DH>(col[e0 + u], H, h, kw[u], vw[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (ok[u]) edge(kw[u], vw[u]);
  }
  const int64_t pr = (int64_t(tk.part) * n_q + tk.ridx) * H + h;
  store_f32<DH>(part_acc + pr * DH, acc);
  if constexpr (MODE == 0) part_z[pr] = z;
}

// Forward finalize: one thread per (order position, head); the parts in order.
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_fwd_tiled_finalize(
    const float* __restrict__ part_acc, const float* __restrict__ part_z,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ order, int32_t n_q,
    int32_t n_sweep, int32_t H, int32_t rows_per_block, int32_t p_max, int32_t e_slot, int32_t kb,
    float eps, T* __restrict__ out, float* __restrict__ rinv, float* __restrict__ zbuf,
    float* __restrict__ ns, int32_t ns_len) {
  const int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t nrh = int64_t(n_q) * H;
  if (t >= nrh) return;
  const int64_t ridx = t / H;
  const int h = int(t - ridx * H);
  const int P = tile_row_parts(rowptr, order, ridx / rows_per_block * rows_per_block, e_slot,
                               p_max, n_sweep, kb);
  float acc[DH], z = 0.f;
#pragma unroll
  for (int c = 0; c < DH; ++c) acc[c] = 0.f;
  for (int p = 0; p < P; ++p) {
    float a[DH];
    load_f32<DH>(part_acc + (p * nrh + t) * DH, a);
#pragma unroll
    for (int c = 0; c < DH; ++c) acc[c] += a[c];
    z += part_z[p * nrh + t];
  }
  const int64_t row = order[ridx];
  const int64_t o = row * H + h;
  const float den = z + eps;
  float ov[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) ov[c] = acc[c] / den;
  store_row<T, DH>(out + o * DH, ov);
  rinv[o] = 1.0f / den;
  zbuf[o] = z;
  if (ns && h == 0 && row < ns_len) {
    float zs = 0.f;
    for (int hh = 0; hh < H; ++hh) {
      float zh = 0.f;
      for (int p = 0; p < P; ++p) zh += part_z[p * nrh + t + hh];
      zs += zh;
    }
    ns[row] = zs / float(H);
  }
}

// Key-major tiled pass: dK, dV partials of the keys j < n_sweep.
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_kv_tiled(
    const T* __restrict__ q, const Keys<T> kv, const T* __restrict__ g,
    const float2* __restrict__ rd, const int32_t* __restrict__ t_rowptr,
    const int32_t* __restrict__ t_col, const int32_t* __restrict__ order, int32_t n_rows,
    int32_t n_q, int32_t H, int32_t hg, int32_t L, int32_t n_groups, int32_t p_max,
    int32_t e_slot, int32_t kb, float inv_scale, float lo, float hi,
    float* __restrict__ part_kv) {
  extern __shared__ uint4 stage[];
  constexpr int NV = RowWords<T, DH>::NV;
  constexpr int U = unroll_for(2 * NV, NGT_BWD_KV_WORDS);
  const TileTask tk = tile_task(t_rowptr, order, n_rows, n_q, n_groups, p_max, e_slot, hg, L, kb);
  if (!tk.live) return;
  const bool work = tk.ridx < n_rows && tk.act;
  const int64_t row = work ? order[tk.ridx] : 0;
  const int h = tk.h;
  int pos = 0, pend = 0;
  if (work) {
    const int beg = t_rowptr[row], end = t_rowptr[row + 1];
    pos = lower_bound_col(t_col, beg, end, tk.c0);
    pend = lower_bound_col(t_col, pos, end, tk.c1);
  }
  RowWords<T, DH> krw, vrw;
  if (work) {
    load_words<T, DH>(kv.template krow<DH>(row, H, h), krw);
    load_words<T, DH>(kv.template vrow<DH>(row, H, h), vrw);
  } else {
    zero_words<T, DH>(krw);
    zero_words<T, DH>(vrw);
  }
  float dk[DH], dv[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dk[c] = 0.f;
    dv[c] = 0.f;
  }
  const int slice = hg * NV;
  const int stride = tile_stride<T, DH>(hg);
  uint4* qs = stage;
  uint4* gs = stage + int64_t(kb) * stride;
  float2* rs = reinterpret_cast<float2*>(stage + 2 * int64_t(kb) * stride);
  for (int cb = tk.c0; cb < tk.c1; cb += kb) {
    const int nc = min(kb, tk.c1 - cb);
    __syncthreads();
    stage_words<kStageBatch>(nc * slice, [&](int t, uint4& a, uint4& b) {
      const int il = t / slice, w = t - il * slice;
      const int64_t base = (int64_t(cb + il) * H + tk.g * hg) * DH;
      a = reinterpret_cast<const uint4*>(q + base)[w];
      b = reinterpret_cast<const uint4*>(g + base)[w];
    }, [&](int t, const uint4& a, const uint4& b) {
      const int il = t / slice, w = t - il * slice;
      qs[il * stride + w] = a;
      gs[il * stride + w] = b;
    });
    for (int t = threadIdx.x; t < nc * hg; t += kBlock) {
      const int il = t / hg, hh = t - il * hg;
      rs[t] = rd[int64_t(cb + il) * H + tk.g * hg + hh];
    }
    __syncthreads();
    if (!work) continue;
    const int cend = cb + nc;
    int cur[U], nxt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      cur[u] = pos + u < pend ? t_col[pos + u] : INT32_MAX;
      nxt[u] = pos + U + u < pend ? t_col[pos + U + u] : INT32_MAX;
    }
    for (;;) {
      int nn[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        nn[u] = pos + 2 * U + u < pend ? t_col[pos + 2 * U + u] : INT32_MAX;
      RowWords<T, DH> qw[U], gw[U];
      float2 r[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (cur[u] < cend) {
          const int il = cur[u] - cb;
          const int o = il * stride + tk.hl * NV;
          lds_words<T, DH>(qs + o, qw[u]);
          lds_words<T, DH>(gs + o, gw[u]);
          r[u] = rs[il * hg + tk.hl];
        }
      int took = 0;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (cur[u] < cend) {
          const float a = edge_dot<T, DH>(qw[u], krw) * inv_scale;
          const float p = __expf(clampf(a, lo, hi));
          const float dp = r[u].x * edge_dot<T, DH>(gw[u], vrw) - r[u].y;
          const float da = (a >= lo && a <= hi) ? dp * p : 0.f;
          const float pr = p * r[u].x;
#pragma unroll
          for (int c = 0; c < DH; ++c) {
            dk[c] = fmaf(da, word_elem<T, DH>(qw[u], c), dk[c]);
            dv[c] = fmaf(pr, word_elem<T, DH>(gw[u], c), dv[c]);
          }
          ++took;
        }
      pos += took;
      if (took < U) break;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        cur[u] = nxt[u];
        nxt[u] = nn[u];
      }
    }
  }
  if (!work) return;
  float* pp = part_kv + ((int64_t(tk.part) * n_rows + tk.ridx) * H + h) * (2 * DH);
  store_f32<DH>(pp, dk);
  store_f32<DH>(pp + DH, dv);
}

// Backward finalize of the tiled passes: threads [0, n_q * H) add the dQ
// parts (query order positions), threads past them the dK/dV parts of the
// keys j < n_rows_k (key order positions; keys >= n_main have no gradient);
// each in part order.
template <typename T, int DH>
__global__ __launch_bounds__(kBlock) void k_bwd_tiled_finalize(
    const float* __restrict__ part_q, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ order_q, int32_t n_q, const float* __restrict__ part_kv,
    const int32_t* __restrict__ t_rowptr, const int32_t* __restrict__ order_k, int32_t n_rows_k,
    int64_t n_main, int32_t n_sweep, int32_t H, int32_t rows_per_block, int32_t p_max,
    int32_t e_slot, int32_t kb_q, int32_t kb_k, float inv_scale, T* __restrict__ grad_q,
    T* __restrict__ grad_k, T* __restrict__ grad_v) {
  const int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t nq = int64_t(n_q) * H;
  if (t < nq) {
    const int64_t ridx = t / H;
    const int h = int(t - ridx * H);
    const int P = tile_row_parts(rowptr, order_q, ridx / rows_per_block * rows_per_block, e_slot,
                                 p_max, n_sweep, kb_q);
    float a[DH];
#pragma unroll
    for (int c = 0; c < DH; ++c) a[c] = 0.f;
    for (int p = 0; p < P; ++p) {
      float b[DH];
      load_f32<DH>(part_q + (p * nq + t) * DH, b);
#pragma unroll
      for (int c = 0; c < DH; ++c) a[c] += b[c];
    }
#pragma unroll
    for (int c = 0; c < DH; ++c) a[c] *= inv_scale;
    store_row<T, DH>(grad_q + (int64_t(order_q[ridx]) * H + h) * DH, a);
    return;
  }
  const int64_t u = t - nq;
  const int64_t nk = int64_t(n_rows_k) * H;
  if (u >= nk) return;
  const int64_t ridx = u / H;
  const int h = int(u - ridx * H);
  const int64_t key = order_k[ridx];
  if (key >= n_main) return;  // constant key row: no gradient
  const int P = tile_row_parts(t_rowptr, order_k, ridx / rows_per_block * rows_per_block, e_slot,
                               p_max, n_q, kb_k);
  float dk[DH], dv[DH];
#pragma unroll
  for (int c = 0; c < DH; ++c) {
    dk[c] = 0.f;
    dv[c] = 0.f;
  }
  for (int p = 0; p < P; ++p) {
    float b[DH], e[DH];
    load_f32<DH>(part_kv + (p * nk + u) * (2 * DH), b);
    load_f32<DH>(part_kv + (p * nk + u) * (2 * DH) + DH, e);
#pragma unroll
    for (int c = 0; c < DH; ++c) {
      dk[c] += b[c];
      dv[c] += e[c];
    }
  }
#pragma unroll
  for (int c = 0; c < DH; ++c) dk[c] *= inv_scale;
  const int64_t o = (key * H + h) * DH;
  store_row<T, DH>(grad_k + o, dk);
  store_row<T, DH>(grad_v + o, dv);
}

// ------------------------------------------------------------------ host side
inline int lanes_for(int n) {
  int L = 1;
  while (L < n) L <<= 1;
  return L;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Heads per pass, per kernel (0 forward, 1 key-major backward, 2 query-major
// backward).  Measured on the 32,768-query / 105K-key window (H = 32, d = 24,
// bf16, us per launch at 32 / 16 / 8 / 4 heads per pass):
//   forward        524 / 470 / 443 / 646
//   key-major bwd  673 / 661 / 787 / 1250
//   query-major    298 / 312 / 385 / 650
// A narrower pass gathers smaller row slices, so more rows of them stay in
// L2; it also runs more waves, each with a fixed cost (work item, q row,
// cross-slot reductions that grow with the slot count 64 / heads).  The
// backward kernels carry more per-wave reduction (dK and dV, or dQ, plus
// per-edge ds) and more per-edge scalars, so they keep wider passes.
// NGT_HEAD_GROUP (all kernels) or NGT_HEAD_GROUP_FWD / _KV / _Q override.
int heads_per_pass(int H, int kind) {
  static const char* const kEnv[3] = {"NGT_HEAD_GROUP_FWD", "NGT_HEAD_GROUP_KV",
                                      "NGT_HEAD_GROUP_Q"};
  const char* env = getenv(kEnv[kind]);
  if (!env) env = getenv("NGT_HEAD_GROUP");
  if (env) {
    const int v = atoi(env);
    if (v >= 1) return v < H ? v : H;
  }
  const int cap = kind == 0 ? 8 : kind == 1 ? 16 : H;
  return H > cap ? cap : H;
}

// dQ from recomputed da (RC) instead of the ds written by the key-major pass:
// the query-major pass then gathers each edge's V row next to its K row, and
// the key-major pass skips its ds writes.  That pays where the key rows are
// reused enough to stay in L2.  Measured, the two passes' time per layer (us,
// dS read -> recompute): the high-degree GT window (95 edges per key row)
// 222.6 -> 188.2 (the layer 303 -> 267), GPH_Slim (15) 33.7 -> 31.9, the GT
// arxiv window (5) 38.5 -> 40.2, GPH_Large (17; its K/V rows do not fit the
// L2s) 940 -> 1,148.  So it is chosen from 32 edges per key row on; the bias
// path keeps ds (its da carries the per-edge bias).
// NGT_DQ_RECOMPUTE=0/1 overrides the choice (not with a bias).
constexpr int64_t kRecomputeEdgesPerKey = 32;
bool dq_recompute(const ngt_window_csr* c, const float* eb) {
  if (eb) return false;
  if (const char* env = getenv("NGT_DQ_RECOMPUTE")) return atoi(env) != 0;
  return c->n_k > 0 && c->n_edges >= kRecomputeEdgesPerKey * c->n_k;
}

// k_rowstat folded into the key-major pass (RowStat<.., true>) on windows of
// at most kFoldEdges edges without a bias or a recomputed dQ: there the pass
// is one round of waves bound by its longest chain, so the extra out-row
// load per edge rides with the Q and dO loads, and the launch (with its gap)
// goes.  The dQ pass then reads ds and needs no statistics.
// NGT_FOLD_ROWSTAT=0/1 overrides the choice.
constexpr int64_t kFoldEdges = int64_t(1) << 19;
bool rowstat_fold(const ngt_window_csr* c, const float* eb, bool rc) {
  if (eb || rc) return false;
  if (const char* env = getenv("NGT_FOLD_ROWSTAT")) return atoi(env) != 0;
  return c->n_edges <= kFoldEdges;
}

// ds written with non-temporal stores when it is too large to stay cached for
// the query-major pass anyway (E * H * 4 bytes above 64 MB): GPH_Large's
// 228 MB, bwd_kv 640 -> 630 us per layer, bwd_q 296 -> 295.  On windows whose
// ds stays in the MALL the query-major pass loses more than the key-major one
// gains (GT arxiv, 7.7 MB: bwd_q 14.7 -> 15.2 us).  NGT_DS_NT=0/1 overrides.
bool ds_nontemporal(const ngt_window_csr* c, int H) {
  if (const char* env = getenv("NGT_DS_NT")) return atoi(env) != 0;
  return size_t(c->n_edges) * size_t(H) * 4 > (size_t(64) << 20);
}

// Head groups are dealt to XCDs (virtual_wave) when their count divides 8;
// NGT_XCD=0 turns that off for experiments.
int xcd_mapping(int groups) {
  if (groups <= 1 || 8 % groups != 0) return 0;
  if (const char* env = getenv("NGT_XCD")) return atoi(env) != 0;
  return 1;
}

// Tiled kernels (dense windows): run only when asked for (NGT_TILED=1), where
// the row orders are built, the head count splits into groups of 4 (or fits
// one group of at most 8) and the staged slices fit kTileLds bytes for at
// least 16 columns.  Measured on the high-degree GT window (7,280 queries,
// 3.67 M edges, H = 8, d = 16, bf16), µs per launch, work lists -> tiled at
// 64 / 128 / 256 edges per slot and part: forward 75 -> 674 / 884 / 1,200,
// key-major 100 -> 1,085 / 1,400 / 1,973, dQ 80 -> 814 / 1,058 / 1,484.  The
// counters show why: an LDS block of 64 KiB leaves 2 blocks (8 waves) per CU
// where the work-list kernels keep about 3 times as many waves in flight, and
// each block's column blocks run as a chain of stage -> barrier -> walk ->
// barrier episodes whose load latency nothing overlaps, with 8.2 M LDS bank
// conflict cycles and 1.6 x the VALU instructions of the work-list forward.
// They stay as a tested option; overlapping the staging of the next column
// block with the walk of the current one is what they would need.
// NGT_TILE_HEADS, NGT_TILE_EDGES, NGT_TILE_PARTS and NGT_TILE_LDS override
// the heads per group, the edges per slot and part, the most parts per row
// block and the LDS bytes per block.
constexpr size_t kTileLds = 65536;

struct TilePlan {
  bool on;
  int hg, groups, L, rows_per_block;
  int n_sweep;  // swept columns of the query-major passes: min(n_q, n_k)
  int p_max;    // most column parts of one row block
  int e_slot;   // edges per slot and part that a row block's parts aim at
};

int tiled_heads(int H) {
  if (const char* env = getenv("NGT_TILE_HEADS")) {
    const int v = atoi(env);
    if (v >= 1 && H % v == 0 && v <= 8) return v;
  }
  if (H % 4 == 0) return 4;
  return H <= 8 ? H : 0;
}

inline int env_int(const char* name, int dflt, int lo, int hi) {
  if (const char* env = getenv(name)) {
    const int v = atoi(env);
    if (v >= lo && v <= hi) return v;
  }
  return dflt;
}

TilePlan tile_plan(const ngt_window_csr* c, int H, int d) {
  TilePlan t{};
  t.on = false;
  t.n_sweep = c->n_q < c->n_k ? c->n_q : c->n_k;
  if (!c->order_q || !c->order_k || t.n_sweep < 1) return t;
  t.hg = tiled_heads(H);
  if (t.hg < 1) return t;
  // the largest staged slice per column (key-major: Q, dO and {r, rD}, fp32, padded)
  if ((size_t(t.hg) * (2 * size_t(d) * 4 + 8) + 32) * 16 > kTileLds) return t;
  const char* env = getenv("NGT_TILED");
  if (!env || atoi(env) == 0) return t;
  t.groups = H / t.hg;
  t.L = lanes_for(t.hg);
  t.rows_per_block = kWavesPerBlock * (kWave / t.L);
  t.p_max = env_int("NGT_TILE_PARTS", 16, 1, 64);
  t.e_slot = env_int("NGT_TILE_EDGES", 256, 1, 1 << 20);
  t.on = true;
  return t;
}

// Columns per staged block for a slice of bytes_per_col bytes per column, in
// kTileLds bytes of LDS (NGT_TILE_LDS overrides, 8-64 KiB).
inline int tile_cols(size_t bytes_per_col) {
  const size_t lds = size_t(env_int("NGT_TILE_LDS", int(kTileLds), 8192, int(kTileLds)));
  int kb = int(lds / bytes_per_col);
  if (kb > 512) kb = 512;
  return kb & ~15;
}

template <typename T, int DH>
size_t tile_q_col_bytes(int hg) {
  return 2 * size_t(tile_stride<T, DH>(hg)) * 16;
}
template <typename T, int DH>
size_t tile_kv_col_bytes(int hg) {
  return 2 * size_t(tile_stride<T, DH>(hg)) * 16 + size_t(hg) * 8;
}

struct FwdLayout {
  size_t part_acc, part_z, zbuf, total;
};
struct BwdLayout {
  size_t rd, ds, part_kv, part_q, part_tk, total;
};

FwdLayout fwd_layout(const ngt_window_csr* c, int H, int d) {
  FwdLayout L{};
  const TilePlan tp = tile_plan(c, H, d);
  const size_t parts = tp.on ? size_t(tp.p_max) * c->n_q : size_t(c->n_parts_q);
  const size_t split = size_t(c->n_parts_q);
  const size_t n = parts > split ? parts : split;  // (partial rows) x H, either kernel family
  size_t off = 0;
  L.part_acc = off;
  off += align256(n * H * d * 4);
  L.part_z = off;
  off += align256(n * H * 4);
  L.zbuf = off;
  off += align256(size_t(c->n_q) * H * 4);
  L.total = off;
  return L;
}

BwdLayout bwd_layout(const ngt_window_csr* c, int H, int d) {
  BwdLayout L{};
  const TilePlan tp = tile_plan(c, H, d);
  size_t nq = size_t(c->n_parts_q), ntk = 0;
  if (tp.on) {
    const size_t tq = size_t(tp.p_max) * c->n_q;  // the tiled dQ parts share part_q
    nq = tq > nq ? tq : nq;
    ntk = size_t(tp.p_max) * tp.n_sweep;
  }
  size_t off = 0;
  L.rd = off;
  off += align256(size_t(c->n_q) * H * 8);
  L.ds = off;
  off += align256(size_t(c->n_edges) * H * 4);
  L.part_kv = off;
  off += align256(size_t(c->n_parts_k) * H * 2 * d * 4);
  L.part_q = off;
  off += align256(nq * H * d * 4);
  L.part_tk = off;
  off += align256(ntk * H * 2 * d * 4);
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
      csr->n_splits_k > csr->max_splits_k || csr->n_parts_q > csr->n_items_q ||
      csr->n_parts_k > csr->n_items_k || csr->n_packed_q < 0 || csr->n_packed_q > csr->n_q ||
      csr->n_packed_k < 0 || csr->n_packed_k > csr->n_k ||
      csr->n_items_q + csr->n_packed_q < csr->n_q - csr->n_splits_q ||
      csr->n_items_k + csr->n_packed_k < csr->n_k - csr->n_splits_k)
    return set_error(NGT_ERR_ARG, "%s: csr counters not filled from info[]", fn);
  return NGT_OK;
}

// Waves for the packed list: 64 / L rows (one per edge slot) per wave.
inline int packed_waves(int n_packed, int L) {
  const int per = kWave / L;
  return (n_packed + per - 1) / per;
}

inline unsigned blocks_for(int64_t waves) {
  return static_cast<unsigned>((waves + kWavesPerBlock - 1) / kWavesPerBlock);
}

// Blocks of an edge-kernel launch over n_items items and pw packed waves per
// head group (see virtual_wave for the xcd order).
inline unsigned edge_blocks(int n_items, int pw, int groups, int xcd) {
  const int64_t per_group = int64_t(n_items) + pw;
  if (per_group <= 0) return 0;
  return xcd ? unsigned(groups) * blocks_for(per_group) : blocks_for(per_group * groups);
}

template <typename T, int DH, bool EXT = true>
Keys<T, EXT> make_keys(const void* k, const void* v, const void* k_ext, const void* v_ext,
                       int64_t n_main, int H) {
  (void)H;
  const T* kk = static_cast<const T*>(k);
  const T* vv = static_cast<const T*>(v);
  return Keys<T, EXT>{kk, vv, k_ext ? static_cast<const T*>(k_ext) : kk,
                      v_ext ? static_cast<const T*>(v_ext) : vv, n_main};
}

// Tiled forward: k_q_tiled<MODE 0> over (row block, part, head group), then
// the finalize over (query, head).
template <typename T, int DH>
int launch_fwd_tiled(const ngt_window_csr* c, const TilePlan& tp, const void* q, const void* k,
                     const void* v, const void* k_ext, const void* v_ext, int64_t n_main, int H,
                     float inv_scale, float lo, float hi, float eps, void* out, float* rinv,
                     float* ns, int ns_len, char* ws, hipStream_t st) {
  const FwdLayout lay = fwd_layout(c, H, DH);
  float* part_acc = reinterpret_cast<float*>(ws + lay.part_acc);
  float* part_z = reinterpret_cast<float*>(ws + lay.part_z);
  float* zbuf = reinterpret_cast<float*>(ws + lay.zbuf);
  const size_t per_col = tile_q_col_bytes<T, DH>(tp.hg);
  const int kb = tile_cols(per_col);
  const int64_t rblocks = (int64_t(c->n_q) + tp.rows_per_block - 1) / tp.rows_per_block;
  const int64_t blocks = rblocks * tp.groups * tp.p_max;
  if (blocks > 0) {
    KernelTimer timer_("sparse_fwd", st);
    const RecomputeArgs none{nullptr, nullptr, nullptr, lo, hi};
    auto launch = [&](auto ext) {
      constexpr bool E = decltype(ext)::value;
      hipLaunchKernelGGL((k_q_tiled<T, DH, E, 0>), dim3(unsigned(blocks)), dim3(kBlock),
                         size_t(kb) * per_col, st, static_cast<const T*>(q),
                         make_keys<T, DH, E>(k, v, k_ext, v_ext, n_main, H), c->rowptr, c->col,
                         c->order_q, c->n_q, tp.n_sweep, H, tp.hg, tp.L, tp.groups, tp.p_max,
                         tp.e_slot, kb, inv_scale, lo, hi, none, part_acc, part_z);
    };
    if (n_main < c->n_k) launch(std::true_type{});
    else launch(std::false_type{});
    NGT_HIP_CHECK(hipGetLastError());
  }
  const int64_t nrh = int64_t(c->n_q) * H;
  if (nrh > 0) {
    KernelTimer timer_("sparse_fwd_finalize", st);
    hipLaunchKernelGGL((k_fwd_tiled_finalize<T, DH>), dim3(unsigned((nrh + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, st, part_acc, part_z, c->rowptr, c->order_q, c->n_q,
                       tp.n_sweep, H, tp.rows_per_block, tp.p_max, tp.e_slot, kb, eps,
                       static_cast<T*>(out), rinv, zbuf, ns_len > 0 ? ns : nullptr, ns_len);
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

template <typename T, int DH>
int launch_fwd(const ngt_window_csr* c, const void* q, const void* k, const void* v,
               const void* k_ext, const void* v_ext, int64_t n_main, int H, float inv_scale,
               float lo, float hi, float eps, void* out, float* rinv, float* ns, int ns_len,
               char* ws, hipStream_t st, const float* eb) {
  if (!eb) {
    const TilePlan tp = tile_plan(c, H, DH);
    if (tp.on)
      return launch_fwd_tiled<T, DH>(c, tp, q, k, v, k_ext, v_ext, n_main, H, inv_scale, lo, hi,
                                     eps, out, rinv, ns, ns_len, ws, st);
  }
  const int hg = heads_per_pass(H, 0);
  const int groups = (H + hg - 1) / hg;
  const int L = lanes_for(hg);
  const FwdLayout lay = fwd_layout(c, H, DH);
  float* part_acc = reinterpret_cast<float*>(ws + lay.part_acc);
  float* part_z = reinterpret_cast<float*>(ws + lay.part_z);
  float* zbuf = reinterpret_cast<float*>(ws + lay.zbuf);
  const int xcd = xcd_mapping(groups);
  const int pw_q = packed_waves(c->n_packed_q, L);
  const unsigned blocks_q = edge_blocks(c->n_items_q, pw_q, groups, xcd);
  // one head group: the forward kernels write the node scores themselves
  float* ns_direct = groups == 1 && ns && ns_len > 0 ? ns : nullptr;
  if (blocks_q > 0) {
    KernelTimer timer_("sparse_fwd", st);
    auto launch = [&](auto ext, auto bias) {
      constexpr bool E = decltype(ext)::value;
      constexpr bool B = decltype(bias)::value;
      hipLaunchKernelGGL((k_fwd<T, DH, E, B>), dim3(blocks_q), dim3(kBlock), 0, st,
                         static_cast<const T*>(q), make_keys<T, DH, E>(k, v, k_ext, v_ext, n_main, H),
                         c->col, reinterpret_cast<const int4*>(c->items_q), c->n_items_q, groups,
                         hg, H, L, inv_scale, lo, hi, eps, static_cast<T*>(out), rinv, zbuf,
                         part_acc, part_z, c->rowptr, c->packed_q, c->n_packed_q, pw_q,
                         ns_direct, ns_len, xcd, eb);
    };
    const bool ext = n_main < c->n_k;
    if (eb) {
      if (ext) launch(std::true_type{}, std::true_type{});
      else launch(std::false_type{}, std::true_type{});
    } else {
      if (ext) launch(std::true_type{}, std::false_type{});
      else launch(std::false_type{}, std::false_type{});
    }
    NGT_HIP_CHECK(hipGetLastError());
  }
  // Split rows' finalize; with several head groups the node scores of the
  // other rows ride in the same launch as extra blocks.
  const int tiles = (H * DH + kColTile - 1) / kColTile;
  const int64_t fin_blocks = int64_t(c->n_splits_q) * tiles;
  const bool ns_late = ns && ns_len > 0 && !ns_direct;
  const int64_t ns_blocks = ns_late ? (ns_len + kBlock - 1) / kBlock : 0;
  if (fin_blocks + ns_blocks > 0) {
    KernelTimer timer_("sparse_fwd_finalize", st);
    hipLaunchKernelGGL((k_fwd_finalize<T, DH>), dim3(unsigned(fin_blocks + ns_blocks)),
                       dim3(kBlock), 0, st, reinterpret_cast<const int4*>(c->splits_q), tiles, H,
                       eps, part_acc, part_z, static_cast<T*>(out), rinv, zbuf,
                       ns_direct ? ns_direct : (ns_late ? ns : nullptr), ns_len, c->rowptr,
                       c->chunk_q, int32_t(ns_blocks));
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

// Tiled backward (after k_rowstat, with each edge's da recomputed in the dQ
// pass): k_kv_tiled over the key rows j < n_sweep, the work-list key-major
// pass over the key rows j >= n_sweep that have a gradient (with the finalize
// of its split rows), k_q_tiled<MODE 1> over the queries, then one finalize
// for the tiled parts.
template <typename T, int DH>
int launch_bwd_tiled(const ngt_window_csr* c, const TilePlan& tp, const void* q, const void* k,
                     const void* v, const void* k_ext, const void* v_ext, int64_t n_main,
                     const void* g, const float2* rd, int H, float inv_scale, float lo, float hi,
                     void* gq, void* gk, void* gv, const BwdLayout& lay, char* ws,
                     hipStream_t st) {
  float* part_q = reinterpret_cast<float*>(ws + lay.part_q);
  float* part_kv = reinterpret_cast<float*>(ws + lay.part_kv);
  float* part_tk = reinterpret_cast<float*>(ws + lay.part_tk);
  const int rows_k = tp.n_sweep;
  const size_t kv_col = tile_kv_col_bytes<T, DH>(tp.hg);
  const int kb_k = tile_cols(kv_col);
  const int64_t blocks_k =
      (int64_t(rows_k) + tp.rows_per_block - 1) / tp.rows_per_block * tp.groups * tp.p_max;
  if (blocks_k > 0) {
    KernelTimer timer_("sparse_bwd_kv", st);
    hipLaunchKernelGGL((k_kv_tiled<T, DH>), dim3(unsigned(blocks_k)), dim3(kBlock),
                       size_t(kb_k) * kv_col, st, static_cast<const T*>(q),
                       make_keys<T, DH>(k, v, k_ext, v_ext, n_main, H), static_cast<const T*>(g),
                       rd, c->t_rowptr, c->t_col, c->order_k, rows_k, c->n_q, H, tp.hg, tp.L,
                       tp.groups, tp.p_max, tp.e_slot, kb_k, inv_scale, lo, hi, part_tk);
    NGT_HIP_CHECK(hipGetLastError());
  }
  const bool rest = n_main > rows_k;  // key rows past the sweep with a gradient
  if (rest) {
    const int hg = heads_per_pass(H, 1);
    const int groups = (H + hg - 1) / hg;
    const int L = lanes_for(hg);
    const int xcd = xcd_mapping(groups);
    const int pw_k = packed_waves(c->n_packed_k, L);
    const unsigned blocks = edge_blocks(c->n_items_k, pw_k, groups, xcd);
    if (blocks > 0) {
      KernelTimer timer_("sparse_bwd_kv_rest", st);
      hipLaunchKernelGGL((k_bwd_kv<T, DH, false, false, false>), dim3(blocks), dim3(kBlock), 0, st,
                         static_cast<const T*>(q), make_keys<T, DH>(k, v, k_ext, v_ext, n_main, H),
                         static_cast<const T*>(g), rd, c->t_col,
                         reinterpret_cast<const int4*>(c->items_k), c->n_items_k, groups, hg, H,
                         L, inv_scale, lo, hi, static_cast<T*>(gk), static_cast<T*>(gv),
                         int64_t(H) * DH, nullptr, part_kv, c->t_rowptr, c->packed_k,
                         c->n_packed_k, pw_k, xcd, nullptr, nullptr, rows_k,
                         FoldArgs{nullptr, nullptr});
      NGT_HIP_CHECK(hipGetLastError());
    }
  }
  const size_t q_col = tile_q_col_bytes<T, DH>(tp.hg);
  const int kb_q = tile_cols(q_col);
  const int64_t blocks_q =
      (int64_t(c->n_q) + tp.rows_per_block - 1) / tp.rows_per_block * tp.groups * tp.p_max;
  const int kv_tiles = (2 * H * DH + kColTile - 1) / kColTile;
  const int64_t fin_rest = rest ? int64_t(c->n_splits_k) * kv_tiles : 0;
  if (blocks_q > 0) {
    KernelTimer timer_("sparse_bwd_q", st);
    const RecomputeArgs rca{q, g, rd, lo, hi};
    auto launch = [&](auto ext) {
      constexpr bool E = decltype(ext)::value;
      hipLaunchKernelGGL((k_q_tiled<T, DH, E, 1>), dim3(unsigned(blocks_q)), dim3(kBlock),
                         size_t(kb_q) * q_col, st, static_cast<const T*>(q),
                         make_keys<T, DH, E>(k, v, k_ext, v_ext, n_main, H), c->rowptr, c->col,
                         c->order_q, c->n_q, tp.n_sweep, H, tp.hg, tp.L, tp.groups, tp.p_max,
                         tp.e_slot, kb_q, inv_scale, lo, hi, rca, part_q, nullptr);
    };
    if (n_main < c->n_k) launch(std::true_type{});
    else launch(std::false_type{});
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (fin_rest > 0) {
    // split key rows past the sweep: k_bwd_q's finalize blocks alone (no dQ blocks)
    KernelTimer timer_("sparse_bwd_kv_rest_finalize", st);
    const RecomputeArgs none{nullptr, nullptr, nullptr, lo, hi};
    hipLaunchKernelGGL((k_bwd_q<T, DH, false, false>), dim3(unsigned(fin_rest)), dim3(kBlock), 0,
                       st, make_keys<T, DH, false>(k, v, k_ext, v_ext, n_main, H), c->col, c->q2t,
                       nullptr, reinterpret_cast<const int4*>(c->items_q), 0, 1, H, H, 1, inv_scale,
                       static_cast<T*>(gq), int64_t(H) * DH, nullptr, c->rowptr, c->packed_q, 0, 0,
                       0,
                       reinterpret_cast<const int4*>(c->splits_k), kv_tiles, part_kv,
                       static_cast<T*>(gk), static_cast<T*>(gv), 0, none, rows_k);
    NGT_HIP_CHECK(hipGetLastError());
  }
  const int64_t threads = int64_t(c->n_q) * H + int64_t(rows_k) * H;
  if (threads > 0) {
    KernelTimer timer_("sparse_bwd_q_finalize", st);
    hipLaunchKernelGGL((k_bwd_tiled_finalize<T, DH>),
                       dim3(unsigned((threads + kBlock - 1) / kBlock)), dim3(kBlock), 0, st,
                       part_q, c->rowptr, c->order_q, c->n_q, part_tk, c->t_rowptr, c->order_k,
                       rows_k, n_main, tp.n_sweep, H, tp.rows_per_block, tp.p_max, tp.e_slot,
                       kb_q, kb_k, inv_scale, static_cast<T*>(gq), static_cast<T*>(gk),
                       static_cast<T*>(gv));
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

template <typename T, int DH>
int launch_bwd(const ngt_window_csr* c, const void* q, const void* k, const void* v,
               const void* k_ext, const void* v_ext, int64_t n_main, const void* out,
               const void* g, const float* rinv, int H, float inv_scale, float lo, float hi,
               void* gq, void* gk, void* gv, int64_t ldg, char* ws, hipStream_t st,
               const float* eb, float* deb) {
  const BwdLayout lay = bwd_layout(c, H, DH);
  float2* rd = reinterpret_cast<float2*>(ws + lay.rd);
  float* ds = reinterpret_cast<float*>(ws + lay.ds);
  float* part_kv = reinterpret_cast<float*>(ws + lay.part_kv);
  float* part_q = reinterpret_cast<float*>(ws + lay.part_q);
  const bool rc = dq_recompute(c, eb);
  const bool fold = rowstat_fold(c, eb, rc);
  const int64_t nrh = int64_t(c->n_q) * H;
  if (nrh > 0 && !fold) {
    int64_t blocks = (nrh + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    KernelTimer timer_("sparse_rowstat", st);
    hipLaunchKernelGGL((k_rowstat<T, DH>), dim3(int(blocks)), dim3(kBlock), 0, st,
                       static_cast<const T*>(out), static_cast<const T*>(g), rinv, nrh, rd);
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (rc && ldg == int64_t(H) * DH) {  // the tiled passes recompute each edge's da in the dQ pass
    const TilePlan tp = tile_plan(c, H, DH);
    if (tp.on)
      return launch_bwd_tiled<T, DH>(c, tp, q, k, v, k_ext, v_ext, n_main, g, rd, H, inv_scale,
                                     lo, hi, gq, gk, gv, lay, ws, st);
  }
  int hg = heads_per_pass(H, 1);
  int groups = (H + hg - 1) / hg;
  int L = lanes_for(hg);
  int xcd = xcd_mapping(groups);
  const int pw_k = packed_waves(c->n_packed_k, L);
  const unsigned blocks_k = edge_blocks(c->n_items_k, pw_k, groups, xcd);
  if (blocks_k > 0) {
    KernelTimer timer_("sparse_bwd_kv", st);
    const FoldArgs fa{out, rinv};
    auto launch = [&](auto bias, auto nt, auto fold_t) {
      constexpr bool B = decltype(bias)::value;
      constexpr bool N = decltype(nt)::value;
      constexpr bool F = decltype(fold_t)::value;
      hipLaunchKernelGGL((k_bwd_kv<T, DH, B, N, F>), dim3(blocks_k), dim3(kBlock), 0, st,
                         static_cast<const T*>(q), make_keys<T, DH>(k, v, k_ext, v_ext, n_main, H),
                         static_cast<const T*>(g), rd, c->t_col,
                         reinterpret_cast<const int4*>(c->items_k), c->n_items_k, groups, hg, H,
                         L, inv_scale, lo, hi, static_cast<T*>(gk), static_cast<T*>(gv), ldg,
                         rc ? nullptr : ds, part_kv, c->t_rowptr, c->packed_k, c->n_packed_k,
                         pw_k, xcd, eb, deb, 0, fa);
    };
    const bool nt = !rc && ds_nontemporal(c, H);
    if (fold) {  // no bias and no recomputed dQ
      if (nt) launch(std::false_type{}, std::true_type{}, std::true_type{});
      else launch(std::false_type{}, std::false_type{}, std::true_type{});
    } else if (eb) {
      if (nt) launch(std::true_type{}, std::true_type{}, std::false_type{});
      else launch(std::true_type{}, std::false_type{}, std::false_type{});
    } else {
      if (nt) launch(std::false_type{}, std::true_type{}, std::false_type{});
      else launch(std::false_type{}, std::false_type{}, std::false_type{});
    }
    NGT_HIP_CHECK(hipGetLastError());
  }
  hg = heads_per_pass(H, 2);
  groups = (H + hg - 1) / hg;
  L = lanes_for(hg);
  xcd = xcd_mapping(groups);
  const int pw_q = packed_waves(c->n_packed_q, L);
  const int kv_tiles = (2 * H * DH + kColTile - 1) / kColTile;
  const int64_t q_blocks = edge_blocks(c->n_items_q, pw_q, groups, xcd);
  const int64_t fin_blocks = int64_t(c->n_splits_k) * kv_tiles;
  if (q_blocks + fin_blocks > 0) {
    KernelTimer timer_("sparse_bwd_q", st);
    const RecomputeArgs rca{q, g, rd, lo, hi};
    auto launch = [&](auto ext, auto recomp) {
      constexpr bool E = decltype(ext)::value;
      constexpr bool R = decltype(recomp)::value;
      hipLaunchKernelGGL((k_bwd_q<T, DH, E, R>), dim3(unsigned(q_blocks + fin_blocks)), dim3(kBlock),
                         0, st, make_keys<T, DH, E>(k, v, k_ext, v_ext, n_main, H), c->col, c->q2t, ds,
                         reinterpret_cast<const int4*>(c->items_q), c->n_items_q, groups, hg, H,
                         L, inv_scale, static_cast<T*>(gq), ldg, part_q, c->rowptr, c->packed_q,
                         c->n_packed_q, pw_q, int32_t(q_blocks),
                         reinterpret_cast<const int4*>(c->splits_k), kv_tiles, part_kv,
                         static_cast<T*>(gk), static_cast<T*>(gv), xcd, rca, 0);
    };
    const bool ext = n_main < c->n_k;
    if (rc) {
      if (ext) launch(std::true_type{}, std::true_type{});
      else launch(std::false_type{}, std::true_type{});
    } else {
      if (ext) launch(std::true_type{}, std::false_type{});
      else launch(std::false_type{}, std::false_type{});
    }
    NGT_HIP_CHECK(hipGetLastError());
  }
  if (c->n_splits_q > 0) {
    KernelTimer timer_("sparse_bwd_q_finalize", st);
    dim3 grid(c->n_splits_q, (H * DH + kColTile - 1) / kColTile);
    hipLaunchKernelGGL((k_bwd_q_finalize<T, DH>), grid, dim3(kBlock), 0, st,
                       reinterpret_cast<const int4*>(c->splits_q), H, part_q,
                       static_cast<T*>(gq), ldg);
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

// ------------------------------------- dense per-pair bias <-> per-edge bias
// The reference's optional attn_bias is a dense [H, N, N] term indexed
// [h, src, dst] and added to each edge's clamped score
// (graphormer_dist_node_level.py:81-84).  The kernels read it per edge in CSR
// order: eb_q[pos][h] for the query-major edge at pos and eb_t[q2t[pos]][h]
// for its key-major position.  One thread per query-major edge; its row
// (query) is the largest r with rowptr[r] <= pos.
__device__ __forceinline__ int32_t row_of(const int32_t* __restrict__ rowptr, int32_t n_rows,
                                          int64_t pos) {
  int32_t lo = 0, hi = n_rows;  // rowptr[lo] <= pos < rowptr[hi]
  while (hi - lo > 1) {
    const int32_t mid = lo + (hi - lo) / 2;
    if (rowptr[mid] <= pos)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kBlock) void k_edge_bias_gather(
    const int32_t* __restrict__ rowptr, int32_t n_q, const int32_t* __restrict__ col,
    const int32_t* __restrict__ q2t, int64_t n_edges, int32_t H, const float* __restrict__ bias,
    int64_t sh, int64_t ss, int64_t sd, float* __restrict__ eb_q, float* __restrict__ eb_t) {
  for (int64_t pos = int64_t(blockIdx.x) * kBlock + threadIdx.x; pos < n_edges;
       pos += int64_t(gridDim.x) * kBlock) {
    const int64_t dst = row_of(rowptr, n_q, pos);
    const int64_t src = col[pos];
    const int64_t tp = q2t[pos];
    for (int h = 0; h < H; ++h) {
      const float b = bias[h * sh + src * ss + dst * sd];
      eb_q[pos * H + h] = b;
      eb_t[tp * H + h] = b;
    }
  }
}

// Gradient of the dense bias: grad[h, src, dst] = the sum of deb_t over the
// edges (src -> dst), added in key-major order (edges with the same pair are
// adjacent there); pairs without an edge are left as they are.  One thread
// per key-major edge; the first edge of each pair's run writes the sum.
__global__ __launch_bounds__(kBlock) void k_edge_bias_grad(
    const int32_t* __restrict__ t_rowptr, int32_t n_k, const int32_t* __restrict__ t_col,
    int64_t n_edges, int32_t H, const float* __restrict__ deb_t, float* __restrict__ grad,
    int64_t sh, int64_t ss, int64_t sd) {
  for (int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x; t < n_edges;
       t += int64_t(gridDim.x) * kBlock) {
    const int32_t key = row_of(t_rowptr, n_k, t);
    const int32_t qi = t_col[t];
    const int64_t beg = t_rowptr[key], end = t_rowptr[key + 1];
    if (t > beg && t_col[t - 1] == qi) continue;  // not the first edge of its pair
    int64_t last = t + 1;
    while (last < end && t_col[last] == qi) ++last;
    for (int h = 0; h < H; ++h) {
      float a = 0.f;
      for (int64_t u = t; u < last; ++u) a += deb_t[u * H + h];
      grad[h * sh + int64_t(key) * ss + int64_t(qi) * sd] = a;
    }
  }
}

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

static int sparse_fwd(int dtype, const void* q, const void* k, const void* v, const void* k_ext,
                      const void* v_ext, int32_t n_k_main, const ngt_window_csr* csr,
                      int32_t n_heads, int32_t head_dim, float scale, float clamp_lo,
                      float clamp_hi, float eps, const float* edge_bias, void* out, float* rinv,
                      float* node_score, int32_t node_score_len, void* workspace,
                      size_t workspace_bytes, void* stream) {
  int rc = check_common("ngt_sparse_fwd", dtype, csr, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  if (!(scale > 0.f)) return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: scale must be > 0");
  if (csr->n_q > 0 && (!q || !out || !rinv))
    return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: null q/out/rinv");
  if (n_k_main < 0 || n_k_main > csr->n_k)
    return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: n_k_main=%d outside [0, n_k=%d]", n_k_main,
                     csr->n_k);
  if (csr->n_edges > 0 && ((n_k_main > 0 && (!k || !v)) ||
                           (n_k_main < csr->n_k && (!k_ext || !v_ext))))
    return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: null k/v");
  if (node_score_len < 0 || node_score_len > csr->n_q)
    return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: node_score_len out of range");
  const size_t need = fwd_layout(csr, n_heads, head_dim).total;
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(NGT_ERR_WORKSPACE, "ngt_sparse_fwd: workspace %zu < %zu", workspace_bytes,
                     need);
  return dispatch<FwdOp>(dtype, head_dim, csr, q, k, v, k_ext, v_ext, int64_t(n_k_main),
                         int(n_heads), 1.0f / scale, clamp_lo, clamp_hi, eps, out, rinv,
                         node_score, int(node_score_len), static_cast<char*>(workspace),
                         static_cast<hipStream_t>(stream), edge_bias);
}

extern "C" int ngt_sparse_fwd_ext(int dtype, const void* q, const void* k, const void* v,
                                  const void* k_ext, const void* v_ext, int32_t n_k_main,
                                  const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                                  float scale, float clamp_lo, float clamp_hi, float eps,
                                  void* out, float* rinv, float* node_score,
                                  int32_t node_score_len, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  return sparse_fwd(dtype, q, k, v, k_ext, v_ext, n_k_main, csr, n_heads, head_dim, scale,
                    clamp_lo, clamp_hi, eps, nullptr, out, rinv, node_score, node_score_len,
                    workspace, workspace_bytes, stream);
}

extern "C" int ngt_sparse_fwd_bias(int dtype, const void* q, const void* k, const void* v,
                                   const void* k_ext, const void* v_ext, int32_t n_k_main,
                                   const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                                   float scale, float clamp_lo, float clamp_hi, float eps,
                                   const float* edge_bias, void* out, float* rinv,
                                   float* node_score, int32_t node_score_len, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (csr && csr->n_edges > 0 && !edge_bias)
    return set_error(NGT_ERR_ARG, "ngt_sparse_fwd_bias: null edge_bias");
  return sparse_fwd(dtype, q, k, v, k_ext, v_ext, n_k_main, csr, n_heads, head_dim, scale,
                    clamp_lo, clamp_hi, eps, csr && csr->n_edges > 0 ? edge_bias : nullptr, out,
                    rinv, node_score, node_score_len, workspace, workspace_bytes, stream);
}

extern "C" int ngt_sparse_fwd(int dtype, const void* q, const void* k, const void* v,
                              const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                              float scale, float clamp_lo, float clamp_hi, float eps, void* out,
                              float* rinv, float* node_score, int32_t node_score_len,
                              void* workspace, size_t workspace_bytes, void* stream) {
  if (!csr) return set_error(NGT_ERR_ARG, "ngt_sparse_fwd: null csr");
  return ngt_sparse_fwd_ext(dtype, q, k, v, nullptr, nullptr, csr->n_k, csr, n_heads, head_dim,
                            scale, clamp_lo, clamp_hi, eps, out, rinv, node_score,
                            node_score_len, workspace, workspace_bytes, stream);
}

static int sparse_bwd(int dtype, const void* q, const void* k, const void* v, const void* k_ext,
                      const void* v_ext, int32_t n_k_main, const void* out, const void* grad_out,
                      const float* rinv, const ngt_window_csr* csr, int32_t n_heads,
                      int32_t head_dim, float scale, float clamp_lo, float clamp_hi,
                      const float* edge_bias_t, float* grad_edge_bias_t, void* grad_q,
                      void* grad_k, void* grad_v, int64_t grad_row_stride, void* workspace,
                      size_t workspace_bytes, void* stream) {
  int rc = check_common("ngt_sparse_bwd", dtype, csr, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  const int64_t row_elems = int64_t(n_heads) * head_dim;
  const int64_t ldg = grad_row_stride == 0 ? row_elems : grad_row_stride;
  const int64_t esize = dtype == NGT_F32 ? 4 : 2;
  if (ldg < row_elems || (ldg * esize) % 16)
    return set_error(NGT_ERR_ARG,
                     "ngt_sparse_bwd: gradient row stride %lld elements (at least %lld, a "
                     "multiple of 16 bytes)",
                     static_cast<long long>(ldg), static_cast<long long>(row_elems));
  if ((reinterpret_cast<uintptr_t>(grad_q) | reinterpret_cast<uintptr_t>(grad_k) |
       reinterpret_cast<uintptr_t>(grad_v)) & 15)
    return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: gradients must be 16-byte aligned");
  if (!(scale > 0.f)) return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: scale must be > 0");
  if (csr->n_q > 0 && (!q || !out || !grad_out || !rinv || !grad_q))
    return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: null query-side pointer");
  if (n_k_main < 0 || n_k_main > csr->n_k)
    return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: n_k_main=%d outside [0, n_k=%d]", n_k_main,
                     csr->n_k);
  if ((n_k_main > 0 && (!k || !v || !grad_k || !grad_v)) ||
      (n_k_main < csr->n_k && (!k_ext || !v_ext)))
    return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: null key-side pointer");
  const size_t need = bwd_layout(csr, n_heads, head_dim).total;
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(NGT_ERR_WORKSPACE, "ngt_sparse_bwd: workspace %zu < %zu", workspace_bytes,
                     need);
  return dispatch<BwdOp>(dtype, head_dim, csr, q, k, v, k_ext, v_ext, int64_t(n_k_main), out,
                         grad_out, rinv, int(n_heads), 1.0f / scale, clamp_lo, clamp_hi, grad_q,
                         grad_k, grad_v, ldg, static_cast<char*>(workspace),
                         static_cast<hipStream_t>(stream), edge_bias_t, grad_edge_bias_t);
}

extern "C" int ngt_sparse_bwd_ext(int dtype, const void* q, const void* k, const void* v,
                                  const void* k_ext, const void* v_ext, int32_t n_k_main,
                                  const void* out, const void* grad_out, const float* rinv,
                                  const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                                  float scale, float clamp_lo, float clamp_hi, void* grad_q,
                                  void* grad_k, void* grad_v, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  return sparse_bwd(dtype, q, k, v, k_ext, v_ext, n_k_main, out, grad_out, rinv, csr, n_heads,
                    head_dim, scale, clamp_lo, clamp_hi, nullptr, nullptr, grad_q, grad_k,
                    grad_v, 0, workspace, workspace_bytes, stream);
}

extern "C" int ngt_sparse_bwd_strided(int dtype, const void* q, const void* k, const void* v,
                                      const void* k_ext, const void* v_ext, int32_t n_k_main,
                                      const void* out, const void* grad_out, const float* rinv,
                                      const ngt_window_csr* csr, int32_t n_heads,
                                      int32_t head_dim, float scale, float clamp_lo,
                                      float clamp_hi, void* grad_q, void* grad_k, void* grad_v,
                                      int64_t grad_row_stride, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  return sparse_bwd(dtype, q, k, v, k_ext, v_ext, n_k_main, out, grad_out, rinv, csr, n_heads,
                    head_dim, scale, clamp_lo, clamp_hi, nullptr, nullptr, grad_q, grad_k,
                    grad_v, grad_row_stride, workspace, workspace_bytes, stream);
}

extern "C" int ngt_sparse_bwd_bias(int dtype, const void* q, const void* k, const void* v,
                                   const void* k_ext, const void* v_ext, int32_t n_k_main,
                                   const void* out, const void* grad_out, const float* rinv,
                                   const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                                   float scale, float clamp_lo, float clamp_hi,
                                   const float* edge_bias_t, float* grad_edge_bias_t,
                                   void* grad_q, void* grad_k, void* grad_v, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (csr && csr->n_edges > 0 && !edge_bias_t)
    return set_error(NGT_ERR_ARG, "ngt_sparse_bwd_bias: null edge_bias_t");
  const bool any = csr && csr->n_edges > 0;
  return sparse_bwd(dtype, q, k, v, k_ext, v_ext, n_k_main, out, grad_out, rinv, csr, n_heads,
                    head_dim, scale, clamp_lo, clamp_hi, any ? edge_bias_t : nullptr,
                    any ? grad_edge_bias_t : nullptr, grad_q, grad_k, grad_v, 0, workspace,
                    workspace_bytes, stream);
}

static unsigned edge_grid(int64_t n) {
  return unsigned(std::min<int64_t>((n + kBlock - 1) / kBlock, 1 << 16));
}

extern "C" int ngt_edge_bias_gather(const ngt_window_csr* csr, int32_t n_heads, const float* bias,
                                    int64_t stride_h, int64_t stride_src, int64_t stride_dst,
                                    float* edge_bias_q, float* edge_bias_t, void* stream) {
  int rc = check_common("ngt_edge_bias_gather", NGT_F32, csr, n_heads, 8);
  if (rc != NGT_OK) return rc;
  if (csr->n_edges == 0) return NGT_OK;
  if (!bias || !edge_bias_q || !edge_bias_t)
    return set_error(NGT_ERR_ARG, "ngt_edge_bias_gather: null pointer");
  if (stride_h < 0 || stride_src < 0 || stride_dst < 0)
    return set_error(NGT_ERR_ARG, "ngt_edge_bias_gather: negative stride");
  hipLaunchKernelGGL(k_edge_bias_gather, dim3(edge_grid(csr->n_edges)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), csr->rowptr, csr->n_q, csr->col, csr->q2t,
                     csr->n_edges, n_heads, bias, stride_h, stride_src, stride_dst, edge_bias_q,
                     edge_bias_t);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_edge_bias_grad(const ngt_window_csr* csr, int32_t n_heads,
                                  const float* grad_edge_bias_t, float* grad_bias,
                                  int64_t stride_h, int64_t stride_src, int64_t stride_dst,
                                  void* stream) {
  int rc = check_common("ngt_edge_bias_grad", NGT_F32, csr, n_heads, 8);
  if (rc != NGT_OK) return rc;
  if (csr->n_edges == 0) return NGT_OK;
  if (!grad_edge_bias_t || !grad_bias)
    return set_error(NGT_ERR_ARG, "ngt_edge_bias_grad: null pointer");
  if (stride_h < 0 || stride_src < 0 || stride_dst < 0)
    return set_error(NGT_ERR_ARG, "ngt_edge_bias_grad: negative stride");
  hipLaunchKernelGGL(k_edge_bias_grad, dim3(edge_grid(csr->n_edges)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), csr->t_rowptr, csr->n_k, csr->t_col,
                     csr->n_edges, n_heads, grad_edge_bias_t, grad_bias, stride_h, stride_src,
                     stride_dst);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_sparse_bwd(int dtype, const void* q, const void* k, const void* v,
                              const void* out, const void* grad_out, const float* rinv,
                              const ngt_window_csr* csr, int32_t n_heads, int32_t head_dim,
                              float scale, float clamp_lo, float clamp_hi, void* grad_q,
                              void* grad_k, void* grad_v, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (!csr) return set_error(NGT_ERR_ARG, "ngt_sparse_bwd: null csr");
  return ngt_sparse_bwd_ext(dtype, q, k, v, nullptr, nullptr, csr->n_k, out, grad_out, rinv, csr,
                            n_heads, head_dim, scale, clamp_lo, clamp_hi, grad_q, grad_k, grad_v,
                            workspace, workspace_bytes, stream);
}

// ------------------------------------------------ allocation-free forward
// ngt_sparse_fwd for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc): its scratch (the
// split rows' fp32 partials and the per-(row, head) Z buffer, the forward's
// workspace) lives in a static device array of kNoAllocScratchBytes that every
// device holds until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and is kept per device.  Nothing in the scratch has to start
// at zero: every word a kernel reads was written earlier in the same call
// (each split item writes its partial slot, every row -- empty rows included,
// through the packed list -- writes its Z), so the last call's contents are
// never read.  Calls that overlap on one device share the array and race.
#include <mutex>

constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;  // 32 MiB per device
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call there).  hipGetSymbolAddress answers for the current device, so a
// stream of another device is refused: its kernels would be handed this
// device's copy of the array.
int scratch_ptr(hipStream_t stream, void** out) {
  int dev = -1;
  NGT_HIP_CHECK(hipGetDevice(&dev));
  hipDevice_t sdev = -1;
  NGT_HIP_CHECK(hipStreamGetDevice(stream, &sdev));
  if (sdev != dev)
    return set_error(NGT_ERR_ARG,
                     "ngt_sparse_fwd_noalloc: the stream belongs to device %d, the current device "
                     "is %d (make the stream's device current)", int(sdev), dev);
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_sparse_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    NGT_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_error(NGT_ERR_HIP, "ngt_sparse_fwd_noalloc: no address for scratch");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NGT_OK;
}
}  // namespace

extern "C" int ngt_sparse_fwd_noalloc(int dtype, const void* q, const void* k, const void* v,
                                      const ngt_window_csr* csr, int32_t n_heads,
                                      int32_t head_dim, float scale, float clamp_lo,
                                      float clamp_hi, float eps, void* out, float* rinv,
                                      float* node_score, int32_t node_score_len, void* stream) {
  const int rc = check_common("ngt_sparse_fwd_noalloc", dtype, csr, n_heads, head_dim);
  if (rc != NGT_OK) return rc;
  const size_t need = fwd_layout(csr, n_heads, head_dim).total;
  if (need > kNoAllocScratchBytes)
    return set_error(NGT_ERR_UNSUPPORTED,
                     "ngt_sparse_fwd_noalloc: the window needs %zu bytes of scratch; the static "
                     "buffer holds %zu (use ngt_sparse_fwd with a workspace)",
                     need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) NGT_CHECK_OK(scratch_ptr(static_cast<hipStream_t>(stream), &ws));
  return ngt_sparse_fwd(dtype, q, k, v, csr, n_heads, head_dim, scale, clamp_lo, clamp_hi, eps,
                        out, rinv, node_score, node_score_len, ws, need, stream);
}
