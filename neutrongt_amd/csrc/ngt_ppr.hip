// APPNP personalised PageRank with per-row top-k, on the GPU.
//
// One propagation step of personal_pagerank_appnp
// (NeutronGT/core/ppr_backends/appnp_backend.py:179-224 with the SpGEMM of
// cusparse_spgemm.cu:65-267) for a batch of seed rows:
//   next[r, :] = topk_K( (1 - alpha) * (state[r, :] P) + alpha * e_seed(r) )
// with P[c, n] = 1 / max(deg(c), 1) for every edge c -> n of the graph CSR.
//
// The state is fixed-width: row r holds cnt[r] <= K entries (col, val) in
// rank order (value descending, then column ascending).  Two forms of the
// step give the same bits: the direct evaluation further down
// (ngt_ppr_step_direct, no product list) and the sorted product list
// (ngt_ppr_step), which is
//   1. count:   per row, the number of products sum_j deg(col_j) plus one
//               teleport entry; an exclusive scan gives each row's range;
//   2. expand:  one wave per row writes, in order j = 0 .. cnt-1 and CSR order
//               of the neighbours, the key (row, n, 0) and the product
//               val_j * P[col_j, n]; then the teleport key (row, seed, 1) with
//               value 0.  Keys are packed as narrow as the ids allow (32 bits
//               when they fit), so the sort makes as few passes as it can;
//   3. sort:    rocPRIM radix sort of (key, value) -- stable, so the products
//               of one (row, column) stay in the order they were generated and
//               the teleport entry comes last;
//   4. reduce:  segment starts (key >> 1 changes), a scan, and one thread per
//               segment adding its products one by one from 0.0f, then
//               value = sum * keep (+ alpha when the teleport is there), with
//               keep = fp32(1 - alpha) rounded from double as the reference's
//               tensor-times-Python-float does: its product scaling followed
//               by its scatter_add of the teleport term;
//   5. top-K:   one wave per row picks K times the best remaining (value
//               descending, column ascending) segment of the row.
// Every sum has a fixed order, so the result is deterministic; the reference's
// order (cuSPARSE, then an atomic scatter_add) is not, and its torch.topk tie
// order is implementation-defined.
#include "ngt_common.h"

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxK = 64;
constexpr int kFastK = 8;  // K up to this takes the one-pass register top-K

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline unsigned grid_waves(int64_t waves) {
  return static_cast<unsigned>((waves + kWaves - 1) / kWaves);
}

// status[0]: bad node ids / row pointers met.  Thread n_rows zeroes the
// extra count slot the scan turns into the total.
__global__ void k_ppr_count(const int64_t* __restrict__ rowptr, int64_t n_nodes,
                            const int32_t* __restrict__ st_col, const int32_t* __restrict__ st_cnt,
                            int32_t n_rows, int32_t K, int64_t* __restrict__ cnt,
                            int32_t* status) {
  const int64_t r = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (r > n_rows) return;
  if (r == n_rows) {
    cnt[r] = 0;
    return;
  }
  int64_t c = 1;  // the teleport entry
  const int n = st_cnt[r];
  if (n < 0 || n > K) {
    atomicAdd(status, 1);
  } else {
    for (int j = 0; j < n; ++j) {
      const int32_t col = st_col[r * K + j];
      if (col < 0 || col >= n_nodes) {
        atomicAdd(status, 1);
        continue;
      }
      const int64_t d = rowptr[col + 1] - rowptr[col];
      if (d < 0)
        atomicAdd(status, 1);
      else
        c += d;
    }
  }
  cnt[r] = c;
}

// Key layout: (row << rs) | (column << 1) | teleport, rs = 1 + cb where cb
// column bits leave the all-ones column free: an out-of-range id gets that
// dead column, which sorts last in its row and is dropped.  Keys are 32 bits
// wide when row and column fit, else 64.
struct KeyFmt {
  int32_t rs;        // row shift
  uint32_t deadcol;  // (1 << cb) - 1
};

// One wave per state row: products in order (j, CSR position), teleport last.
template <typename KeyT>
__global__ __launch_bounds__(kBlock) void k_ppr_expand(
    const int64_t* __restrict__ rowptr, const int64_t* __restrict__ col,
    const float* __restrict__ inv_deg, int64_t n_nodes, const int32_t* __restrict__ st_col,
    const float* __restrict__ st_val, const int32_t* __restrict__ st_cnt,
    const int64_t* __restrict__ seeds, int32_t n_rows, int32_t K,
    const int64_t* __restrict__ row_off, int64_t total, KeyFmt f, KeyT* __restrict__ keys,
    float* __restrict__ vals, int32_t* status) {
  const int64_t r = blockIdx.x * int64_t(kWaves) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & (kWave - 1);
  if (r >= n_rows) return;
  if (row_off[n_rows] > total) {  // the product list would overrun the workspace
    if (r == 0 && lane == 0) atomicAdd(status, 1);
    return;
  }
  int64_t at = row_off[r];
  const KeyT rk = KeyT(r) << f.rs;
  const KeyT dead = rk | (KeyT(f.deadcol) << 1);
  const int n = st_cnt[r];
  if (n >= 0 && n <= K) {
    for (int j = 0; j < n; ++j) {
      const int32_t c = st_col[r * K + j];
      if (c < 0 || c >= n_nodes) continue;  // counted by k_ppr_count
      const int64_t b = rowptr[c], e = rowptr[c + 1];
      if (e < b) continue;
      const float w = st_val[r * K + j] * inv_deg[c];
      for (int64_t p = b + lane; p < e; p += kWave) {
        const int64_t nb = col[p];
        const bool ok = nb >= 0 && nb < n_nodes;
        if (!ok) atomicAdd(status, 1);
        keys[at + (p - b)] = ok ? (rk | (KeyT(nb) << 1)) : dead;
        vals[at + (p - b)] = w;
      }
      at += e - b;
    }
  }
  if (lane == 0) {
    const int64_t sd = seeds[r];
    const bool ok = sd >= 0 && sd < n_nodes;
    if (!ok) atomicAdd(status, 1);
    keys[at] = ok ? (rk | (KeyT(sd) << 1) | KeyT(1)) : dead;
    vals[at] = 0.f;
  }
}

template <typename KeyT>
__global__ void k_ppr_starts(const KeyT* __restrict__ keys, int64_t n, KeyFmt f,
                             int32_t* __restrict__ flag) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  const KeyT k = keys[i] >> 1;
  const bool real = uint32_t(k & KeyT(f.deadcol)) != f.deadcol;
  flag[i] = real && (i == 0 || (keys[i - 1] >> 1) != k) ? 1 : 0;
}

// s * keep, then + alpha when the teleport is present, with two roundings
// (no fused multiply-add): the reference scales one tensor, then adds.
__device__ __forceinline__ float scale_then_add(float s, float keep, float alpha, bool tele) {
#pragma clang fp contract(off)
  const float scaled = s * keep;
  return tele ? scaled + alpha : scaled;
}

template <typename KeyT>
__global__ void k_ppr_segsum(const KeyT* __restrict__ keys, const float* __restrict__ vals,
                             int64_t n, KeyFmt f, const int32_t* __restrict__ flag,
                             const int32_t* __restrict__ pos, float alpha, float keep,
                             int32_t* __restrict__ seg_row, int32_t* __restrict__ seg_col,
                             float* __restrict__ seg_val) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n || !flag[i]) return;
  const KeyT k = keys[i] >> 1;
  float s = 0.f;
  bool tele = false;
  for (int64_t p = i; p < n && (keys[p] >> 1) == k; ++p) {
    s += vals[p];
    tele |= (keys[p] & KeyT(1)) != 0;
  }
  const int32_t at = pos[i];
  seg_row[at] = int32_t(keys[i] >> f.rs);
  seg_col[at] = int32_t(k & KeyT(f.deadcol));
  seg_val[at] = scale_then_add(s, keep, alpha, tele);
}

// (v, c) ranks before (bv, bc): value descending, then column ascending
__device__ __forceinline__ bool better(float v, int32_t c, float bv, int32_t bc) {
  return v > bv || (v == bv && c < bc);
}

// One wave per row: K rounds of "best segment ranked after the last pick".
__global__ __launch_bounds__(kBlock) void k_ppr_topk(
    const int32_t* __restrict__ seg_row, const int32_t* __restrict__ seg_col,
    const float* __restrict__ seg_val, const int32_t* __restrict__ n_seg_p, int32_t n_rows,
    int32_t K, int32_t* __restrict__ out_col, float* __restrict__ out_val,
    int32_t* __restrict__ out_cnt) {
  const int64_t r = blockIdx.x * int64_t(kWaves) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & (kWave - 1);
  if (r >= n_rows) return;
  const int32_t n_seg = *n_seg_p;
  // the row's segments: [lower_bound(r), lower_bound(r + 1)) of seg_row
  int32_t lo = 0, hi = n_seg;
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (seg_row[mid] < r) lo = mid + 1; else hi = mid;
  }
  const int32_t b = lo;
  hi = n_seg;
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (seg_row[mid] <= r) lo = mid + 1; else hi = mid;
  }
  const int32_t e = lo;
  if (K <= kFastK) {
    // one pass: every lane keeps its best K of a strided share in registers
    // (insertion by compare-and-swap down the list), then K rounds of a wave
    // arg-max over the lanes' heads, the winner popping its head
    float lv[kFastK];
    int32_t lc[kFastK];
#pragma unroll
    for (int i = 0; i < kFastK; ++i) {
      lv[i] = -INFINITY;
      lc[i] = INT32_MAX;
    }
    for (int32_t s = b + lane; s < e; s += kWave) {
      float tv = seg_val[s];
      int32_t tc = seg_col[s];
#pragma unroll
      for (int i = 0; i < kFastK; ++i) {
        if (i < K && better(tv, tc, lv[i], lc[i])) {
          const float sv = lv[i];
          const int32_t sc = lc[i];
          lv[i] = tv;
          lc[i] = tc;
          tv = sv;
          tc = sc;
        }
      }
    }
    const int n_out = e - b < K ? e - b : K;
    for (int t = 0; t < n_out; ++t) {
      float bv = lv[0];
      int32_t bc = lc[0];
      for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const int32_t oc = __shfl_xor(bc, off, kWave);
        if (better(ov, oc, bv, bc)) {
          bv = ov;
          bc = oc;
        }
      }
      if (lc[0] == bc && lv[0] == bv) {  // (value, column) pairs are unique in a row
#pragma unroll
        for (int i = 0; i + 1 < kFastK; ++i) {
          lv[i] = lv[i + 1];
          lc[i] = lc[i + 1];
        }
        lv[kFastK - 1] = -INFINITY;
        lc[kFastK - 1] = INT32_MAX;
      }
      if (lane == 0) {
        out_col[r * K + t] = bc;
        out_val[r * K + t] = bv;
      }
    }
    if (lane == 0) out_cnt[r] = n_out;
    return;
  }
  float pv = INFINITY;
  int32_t pc = -1;  // last pick: everything ranks after (+inf, -1)
  int picked = 0;
  for (int t = 0; t < K && t < e - b; ++t) {
    float bv = -INFINITY;
    int32_t bc = INT32_MAX;
    for (int32_t s = b + lane; s < e; s += kWave) {
      const float v = seg_val[s];
      const int32_t c = seg_col[s];
      if (better(pv, pc, v, c) && better(v, c, bv, bc)) {
        bv = v;
        bc = c;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, kWave);
      const int32_t oc = __shfl_xor(bc, off, kWave);
      if (better(ov, oc, bv, bc)) {
        bv = ov;
        bc = oc;
      }
    }
    if (lane == 0) {
      out_col[r * K + t] = bc;
      out_val[r * K + t] = bv;
    }
    pv = bv;
    pc = bc;
    ++picked;
  }
  if (lane == 0) out_cnt[r] = picked;
}

struct PprLayout {
  size_t cnt, keys_a, keys_b, vals_a, vals_b, flag, pos, seg_row, seg_col, seg_val, n_seg, temp,
      temp_bytes, total;
};

int ppr_layout(int64_t T, int32_t n_rows, PprLayout* L) {
  const size_t t = size_t(T > 0 ? T : 1);
  const size_t m = size_t(n_rows > 0 ? n_rows : 1);
  size_t sort_bytes = 0, scan_bytes = 0, scan2 = 0;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, sort_bytes, (uint64_t*)nullptr,
                                          (uint64_t*)nullptr, (float*)nullptr, (float*)nullptr,
                                          t, 0u, 64u, hipStream_t(0)));
  size_t sort32 = 0;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, sort32, (uint32_t*)nullptr,
                                          (uint32_t*)nullptr, (float*)nullptr, (float*)nullptr,
                                          t, 0u, 32u, hipStream_t(0)));
  if (sort32 > sort_bytes) sort_bytes = sort32;
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan_bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                        int32_t(0), t, rocprim::plus<int32_t>(), hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan2, (int64_t*)nullptr, (int64_t*)nullptr,
                                        int64_t(0), m + 1, rocprim::plus<int64_t>(),
                                        hipStream_t(0)));
  size_t off = 0;
  auto take = [&](size_t b) {
    const size_t at = off;
    off += align256(b);
    return at;
  };
  L->cnt = take((m + 1) * 8);
  L->keys_a = take(t * 8);
  L->keys_b = take(t * 8);
  L->vals_a = take(t * 4);
  L->vals_b = take(t * 4);
  L->flag = take(t * 4);
  L->pos = take(t * 4);
  L->seg_row = take(t * 4);
  L->seg_col = take(t * 4);
  L->seg_val = take(t * 4);
  L->n_seg = take(8);
  L->temp_bytes = sort_bytes > scan_bytes ? sort_bytes : scan_bytes;
  if (scan2 > L->temp_bytes) L->temp_bytes = scan2;
  L->temp = take(L->temp_bytes);
  L->total = off;
  return NGT_OK;
}

__global__ void k_ppr_nseg(const int32_t* __restrict__ flag, const int32_t* __restrict__ pos,
                           int64_t n, int32_t* __restrict__ n_seg) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *n_seg = n > 0 ? pos[n - 1] + flag[n - 1] : 0;
}

template <typename KeyT>
int ppr_sort_reduce(const int64_t* rowptr, const int64_t* col, const float* inv_deg,
                    int64_t n_nodes, const int32_t* st_col, const float* st_val,
                    const int32_t* st_cnt, const int64_t* seeds, int32_t n_rows, int32_t K,
                    float alpha, float keep, const int64_t* row_off, int64_t total, KeyFmt f,
                    unsigned end_bit, int32_t* status, char* ws, const PprLayout& L,
                    hipStream_t s) {
  KeyT* keys_a = reinterpret_cast<KeyT*>(ws + L.keys_a);
  KeyT* keys_b = reinterpret_cast<KeyT*>(ws + L.keys_b);
  float* vals_a = reinterpret_cast<float*>(ws + L.vals_a);
  float* vals_b = reinterpret_cast<float*>(ws + L.vals_b);
  int32_t* flag = reinterpret_cast<int32_t*>(ws + L.flag);
  int32_t* pos = reinterpret_cast<int32_t*>(ws + L.pos);
  hipLaunchKernelGGL(k_ppr_expand<KeyT>, dim3(grid_waves(n_rows)), dim3(kBlock), 0, s, rowptr,
                     col, inv_deg, n_nodes, st_col, st_val, st_cnt, seeds, n_rows, K, row_off, total, f,
                     keys_a, vals_a, status);
  NGT_HIP_CHECK(hipGetLastError());
  size_t tb = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(ws + L.temp, tb, keys_a, keys_b, vals_a, vals_b,
                                          size_t(total), 0u, end_bit, s));
  const unsigned g = static_cast<unsigned>((total + kBlock - 1) / kBlock);
  hipLaunchKernelGGL(k_ppr_starts<KeyT>, dim3(g), dim3(kBlock), 0, s, keys_b, total, f, flag);
  tb = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::exclusive_scan(ws + L.temp, tb, flag, pos, int32_t(0), size_t(total),
                                        rocprim::plus<int32_t>(), s));
  hipLaunchKernelGGL(k_ppr_nseg, dim3(1), dim3(64), 0, s, flag, pos, total,
                     reinterpret_cast<int32_t*>(ws + L.n_seg));
  hipLaunchKernelGGL(k_ppr_segsum<KeyT>, dim3(g), dim3(kBlock), 0, s, keys_b, vals_b, total, f,
                     flag, pos, alpha, keep, reinterpret_cast<int32_t*>(ws + L.seg_row),
                     reinterpret_cast<int32_t*>(ws + L.seg_col),
                     reinterpret_cast<float*>(ws + L.seg_val));
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

// ---------------------------------------------------------------------------
// Direct evaluation: no product list, no sort.  For row r with state lists
// L_j = the CSR row of st_col[r, j] (columns ascending) and weights
// w_j = st_val[r, j] * inv_deg[st_col[r, j]], the sum of column n is
//   s = 0; for j in rank order: for every occurrence of n in L_j: s += w_j,
// which is exactly the additions, in the same order, that the stable sort of
// the product list (j, CSR position) gives one (row, n) segment.  Position p
// of list j is evaluated by the lane that owns it: the first occurrence of n
// in the first list holding it (searches in the other lists decide).
//
// Work: one wave per chunk of kDirChunk consecutive entries of one list (a
// row's chunks are its lists' chunks in rank order, at least one per row for
// the teleport entry).  A chunk's columns lie in [vmin, vmax], its first and
// last entry, so each other list is searched once per chunk for the slice of
// entries in that interval (a cooperative search, all lists at once); the
// per-column lookups then run inside those slices.  The columns a bound does
// not rule out are compacted and summed exactly.  Each chunk keeps its best K
// (value descending, column ascending); a per-row merge takes the best K of
// its chunks', which is the best K of the row whatever the chunking.
//
// Pruning, which changes no result.  With nonnegative weights, keep and
// alpha, a column's value is at least fl(w_j * keep) for every list j that
// holds it (fp32 sums of nonnegative terms only grow), and a list of L
// entries holds at least ceil(L / M) distinct columns, M the most repeats of
// one column within a CSR row.  So if the i heaviest lists together are sure
// to hold K distinct columns (the most of their ceil(L / M), plus the seed
// when no list holds it and alpha is at least the bound), the row's K-th best
// value is at least tau = fl(w_(i) * keep) for the first such i.  A column
// whose value is shown to lie below tau cannot be among the row's best K.
// A column's upper bound is keep times: M * w_j for its own list, plus the
// exact share of the lists whose slice holds at most kDirRev entries
// (each slice entry looked up among the chunk's columns adds its w), plus
// M * w for every larger non-empty slice; fp32's rounding of the exact sum
// (at most K * M + 1 roundings) is covered by a factor 1 + 2^-10.

constexpr int kDirU = 8;                                 // entries per lane
constexpr int64_t kDirChunk = int64_t(kWave) * kDirU;    // entries per chunk
constexpr int kDirRev = 256;  // slices up to this size are looked up from the slice's side

__device__ __forceinline__ int64_t lane_i64(int64_t v, int src) {  // src wave-uniform
  const uint64_t u = uint64_t(v);
  const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u)), src));
  const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u >> 32)), src));
  return int64_t((uint64_t(hi) << 32) | lo);
}

__device__ __forceinline__ float lane_f32(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

__device__ __forceinline__ int32_t clamp_i32(int64_t v) {
  return v < INT32_MIN ? INT32_MIN : (v > INT32_MAX ? INT32_MAX : int32_t(v));
}

// cnt[u] = the number of entries equal to x[u] in the m >= 1 sorted columns
// col[lo ..], for every u with act[u].  Branchless lower bounds with one trip
// count for all u, so the U searches' loads are in flight together (the
// slices stay in L2 and L1; staging them in LDS first measured slower).
template <int U>
__device__ __forceinline__ void slice_counts(const int64_t* __restrict__ col, int64_t lo,
                                             int64_t m, const int32_t (&x)[U],
                                             const bool (&act)[U], int32_t (&cnt)[U]) {
  int64_t a[U];
#pragma unroll
  for (int u = 0; u < U; ++u) a[u] = lo;
  for (int64_t len = m; len > 1;) {
    const int64_t half = len >> 1;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (act[u]) a[u] = col[a[u] + half] < x[u] ? a[u] + half : a[u];
    len -= half;
  }
  const int64_t e = lo + m;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    cnt[u] = 0;
    if (!act[u]) continue;
    int64_t q = a[u] + (col[a[u]] < x[u] ? 1 : 0);
    for (; q < e && col[q] == x[u]; ++q) ++cnt[u];
  }
}

// For every list l < n whose lane sets `need`: slo and shi on lane l become
// the first entry of list l (col[lb, lb + ll), ascending) >= vlo and > vhi;
// 0 on the other lanes.  With n <= 32, G lanes per (list, bound) run a
// (G+1)-way search together, each round testing G pivots of the open range;
// above that, each lane runs both binary searches itself.  Every lane takes
// part in every shuffle.
__device__ __forceinline__ void coop_slices(const int64_t* __restrict__ col, int n, bool need,
                                            int64_t lb, int64_t ll, int64_t vlo, int64_t vhi,
                                            int lane, int64_t& slo, int64_t& shi) {
  slo = shi = 0;
  if (n <= kWave / 2) {
    const int G = kWave / (2 * (n > 0 ? n : 1));
    const int g = lane / G, k = lane % G;
    const int jj = g >> 1, bnd = g & 1;  // group 2 jj + b: list jj, bound b (0: >= vlo, 1: > vhi)
    const bool mine = g < 2 * n;
    const int src = mine ? jj : 0;
    const bool nd = __shfl(int(need), src, kWave) != 0 && mine;
    int64_t L = __shfl(lb, src, kWave);
    const int64_t len = __shfl(ll, src, kWave);
    int64_t R = nd ? L + len : L;
    const int64_t x = bnd ? vhi : vlo;
    const uint64_t gmask = mine ? (((1ull << G) - 1ull) << (g * G)) : 0ull;
    while (__ballot(R > L)) {
      const int64_t piv = L + ((R - L) * (k + 1)) / (G + 1);  // in [L, R) when R > L
      bool right = false;  // the answer lies after piv
      if (R > L) {
        const int64_t v = col[piv];
        right = bnd ? v <= x : v < x;
      }
      const uint64_t bal = __ballot(right) & gmask;
      const int cnt = __popcll(bal);  // the group's pivots ascend: a prefix goes right
      const int64_t lo_p = __shfl(piv, g * G + (cnt > 0 ? cnt - 1 : 0), kWave);
      const int64_t hi_p = __shfl(piv, g * G + (cnt < G ? cnt : G - 1), kWave);
      if (R > L) {
        if (cnt > 0) L = lo_p + 1;
        if (cnt < G) R = hi_p;
      }
    }
    slo = __shfl(L, (2 * lane) * G < kWave ? (2 * lane) * G : 0, kWave);
    shi = __shfl(L, (2 * lane + 1) * G < kWave ? (2 * lane + 1) * G : 0, kWave);
    if (!need) slo = shi = 0;
  } else if (need) {
    int64_t a = lb, c = lb;
    for (int64_t len = ll; len > 1;) {
      const int64_t half = len >> 1;
      a = col[a + half] < vlo ? a + half : a;
      c = col[c + half] <= vhi ? c + half : c;
      len -= half;
    }
    slo = a + (col[a] < vlo ? 1 : 0);
    shi = c + (col[c] <= vhi ? 1 : 0);
  }
}

// Per row, one wave: the table of its state lists (begin, length, first and
// last column, weight w_j = st_val * inv_deg, the same fp32 product the chunks
// would form), the lower bound tau of its K-th best value (-inf: no bound),
// the lists it skips, its chunk count (the sum over the other lists of
// ceil(length / kDirChunk), at least 1 for the teleport entry), whether a
// list it keeps holds the seed, and the seed's exact value.  A list is
// skipped when it is among the lightest whose keep * sum of M * w stays below
// tau: a column that only skipped lists hold is worth less than tau, so its
// entries need no chunk; columns a kept list holds are still summed over
// every list.  Wave n_rows writes the count slot the scan turns into the
// total.
__global__ __launch_bounds__(kBlock) void k_ppr_rows(
    const int64_t* __restrict__ rowptr, const int64_t* __restrict__ col,
    const float* __restrict__ inv_deg, int64_t n_nodes, const int32_t* __restrict__ st_col,
    const float* __restrict__ st_val, const int32_t* __restrict__ st_cnt,
    const int64_t* __restrict__ seeds, int32_t n_rows, int32_t K, float alpha, float keep,
    int32_t max_mult, int64_t* __restrict__ tl_b, int64_t* __restrict__ tl_len,
    int64_t* __restrict__ tl_first, int64_t* __restrict__ tl_last, float* __restrict__ tl_w,
    int32_t* __restrict__ tl_skip, int32_t* __restrict__ nch, int32_t* __restrict__ seed_in,
    float* __restrict__ seed_val, float* __restrict__ row_tau, int32_t* status) {
#pragma clang fp contract(off)
  const int32_t r = __builtin_amdgcn_readfirstlane(int(blockIdx.x * kWaves + (threadIdx.x >> 6)));
  const int lane = threadIdx.x & (kWave - 1);
  if (r > n_rows) return;
  if (r == n_rows) {
    if (lane == 0) nch[r] = 0;
    return;
  }
  int n = __builtin_amdgcn_readfirstlane(st_cnt[r]);
  if (n < 0 || n > K) n = 0;
  int64_t lb = 0, ll = 0, lfirst = 0, llast = -1;
  float lw = 0.f;
  if (lane < n) {
    const int32_t c = st_col[int64_t(r) * K + lane];
    if (c >= 0 && c < n_nodes) {
      const int64_t b = rowptr[c], e = rowptr[c + 1];
      if (e > b) {
        lb = b;
        ll = e - b;
        lw = st_val[int64_t(r) * K + lane] * inv_deg[c];
        lfirst = col[b];
        llast = col[e - 1];
      }
    }
    const int64_t at = int64_t(r) * K + lane;
    tl_b[at] = lb;
    tl_len[at] = ll;
    tl_first[at] = lfirst;
    tl_last[at] = llast;
    tl_w[at] = lw;
  }
  const int64_t sd = seeds[r];
  const bool seed_ok = sd >= 0 && sd < n_nodes;
  int64_t slo, shi;  // the seed's entries in list `lane`
  coop_slices(col, n, seed_ok && lane < n && ll > 0 && sd >= lfirst && sd <= llast, lb, ll, sd,
              sd, lane, slo, shi);
  const bool held_any = __ballot(shi > slo) != 0;

  bool prune = max_mult > 0 && int64_t(max_mult) * K <= 4096 && keep >= 0.f && alpha >= 0.f;
  if (__ballot(lane < n && !(lw >= 0.f && lw <= __FLT_MAX__))) prune = false;  // < 0, inf, NaN
  float tau = -INFINITY;
  bool skip = false;
  if (prune) {
    // lists by weight, heaviest first: lane i of `order` names the list of rank i
    int rank = lane;
    if (lane < n) {
      rank = 0;
      for (int i = 0; i < n; ++i) {
        const float wi = lane_f32(lw, i);
        rank += (wi > lw || (wi == lw && i < lane)) ? 1 : 0;
      }
    }
    const int order = __builtin_amdgcn_ds_permute(rank * 4, lane);
    // tau: the union of the i heaviest lists holds at least max ceil(length / M)
    // distinct columns, each worth at least fl(w_(i) * keep); a seed that no
    // list holds is one more, worth alpha
    const bool seed_alone = seed_ok && !held_any;
    int64_t dmax = 0;
    for (int i = 0; i < n; ++i) {
      const int jj = __builtin_amdgcn_readlane(order, i);
      const int64_t d = (lane_i64(ll, jj) + max_mult - 1) / max_mult;
      dmax = d > dmax ? d : dmax;
      const float v = lane_f32(lw, jj) * keep;
      if (dmax + ((seed_alone && alpha >= v) ? 1 : 0) >= K) {
        tau = v;
        break;
      }
    }
    if (tau > 0.f) {
      // the lightest lists whose keep * sum of M * w, rounding covered as in the
      // chunks, stays below tau
      const double cut = double(tau) / (double(keep) * (1.0 + 1.0 / 1024.0));
      double acc = 0.0;
      int nskip = 0;
      for (int i = n - 1; i >= 0; --i) {
        acc += double(max_mult) * double(lane_f32(lw, __builtin_amdgcn_readlane(order, i)));
        if (acc * (1.0 + 0x1p-40) >= cut) break;
        ++nskip;
      }
      skip = lane < n && rank >= n - nskip;
    }
  }
  int64_t c = skip ? 0 : (ll + kDirChunk - 1) / kDirChunk;
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, kWave);
  const bool held_live = __ballot(shi > slo && !skip) != 0;
  // the seed's value: its entries' products in list order, scaled, plus alpha
  float sv = 0.f;
  for (int jj = 0; jj < n; ++jj) {
    const int32_t cnt = __builtin_amdgcn_readlane(int(shi - slo), jj);
    const float wj = lane_f32(lw, jj);
    for (int32_t k = 0; k < cnt; ++k) sv += wj;
  }
  if (lane < n) tl_skip[int64_t(r) * K + lane] = skip ? 1 : 0;
  if (lane == 0) {
    nch[r] = c > 0 ? int32_t(c) : 1;
    seed_in[r] = held_live ? 1 : 0;
    seed_val[r] = scale_then_add(sv, keep, alpha, true);
    row_tau[r] = prune ? tau : -INFINITY;
    if (!seed_ok) atomicAdd(status, 1);
  }
}

// row_of[c] = the row of chunk c (c < max_chunks), one thread per row
__global__ void k_ppr_chunk_rows(const int32_t* __restrict__ chunk_off, int32_t n_rows,
                                 int32_t max_chunks, int32_t* __restrict__ row_of) {
  const int64_t r = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (r >= n_rows) return;
  const int32_t e = chunk_off[r + 1] < max_chunks ? chunk_off[r + 1] : max_chunks;
  for (int32_t c = chunk_off[r]; c < e; ++c) row_of[c] = int32_t(r);
}

// What a chunk's survivors need: the per-list values every lane holds for
// list `lane` (slice begin and size, weight, skipped) and the chunk's context.
struct ChunkCtx {
  const int64_t* col;
  const int32_t* own_lds;  // the chunk's columns, position t at [t]
  const int32_t* surv;     // the surviving positions, S of them
  int32_t S;
  int n, j, lane;
  int64_t p0, ej;
  float wj_own, keep, alpha;
  bool seed_ok, extra;  // extra: this lane adds the seed's teleport entry
  int64_t sd;
  int32_t K, w;
  int64_t sm, slo;
  float lw;
  bool lsk;      // list `lane` is skipped: it owns no column
  float seed_v;  // the seed's value, for the teleport entry
};

// The exact sums of the chunk's surviving positions, 64 at a time (one per
// lane; lists in order, a column an earlier list holds belongs to that list),
// kept in LDS: the column in surv[i] (-1: another list's) and the value's
// bits in own_lds[i], whose column survivor i has read by then (survivors
// ascend, so survivor i's position is at least i).  Then the chunk's best K of
// them and the teleport entry into part_*.
__device__ __forceinline__ void chunk_survivors(const ChunkCtx& x, int32_t* surv, int32_t* vals,
                                                float* __restrict__ part_val,
                                                int32_t* __restrict__ part_col,
                                                int32_t* __restrict__ part_cnt) {
#pragma clang fp contract(off)
  int real = 0;
  for (int32_t base = 0; base < x.S; base += kWave) {  // uniform
    const int32_t idx = base + x.lane;
    bool own[1] = {idx < x.S};
    const int32_t t = own[0] ? surv[idx] : 0;
    const int32_t nv[1] = {own[0] ? x.own_lds[t] : 0};
    int32_t rep = 0;
    if (own[0]) {
      rep = 1;
      for (int64_t q = x.p0 + t + 1; q < x.ej && x.col[q] == nv[0]; ++q) ++rep;
    }
    float s = 0.f;
    for (int jj = 0; jj < x.n; ++jj) {
      if (jj == x.j) {
        if (own[0])
          for (int32_t c = 0; c < rep; ++c) s += x.wj_own;
        continue;
      }
      const int64_t m = lane_i64(x.sm, jj);
      if (m == 0) continue;
      const int64_t lo_ = lane_i64(x.slo, jj);
      const float wj = lane_f32(x.lw, jj);
      int32_t cnt[1];
      slice_counts<1>(x.col, lo_, m, nv, own, cnt);
      if (!own[0] || cnt[0] == 0) continue;
      if (jj < x.j && !__builtin_amdgcn_readlane(int(x.lsk), jj)) {
        own[0] = false;  // an earlier list that is not skipped holds it
        continue;
      }
      for (int32_t k = 0; k < cnt[0]; ++k) s += wj;
    }
    real += __popcll(__ballot(own[0]));
    if (idx < x.S) {
      vals[idx] = __float_as_int(
          own[0] ? scale_then_add(s, x.keep, x.alpha, x.seed_ok && nv[0] == x.sd) : 0.f);
      surv[idx] = own[0] ? nv[0] : -1;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float ev = x.extra ? x.seed_v : -INFINITY;
  const int32_t ec = x.extra ? int32_t(x.sd) : INT32_MAX;
  real += __popcll(__ballot(x.extra));
  const int n_out = real < x.K ? real : x.K;
  float pv = INFINITY;
  int32_t pc = -1;  // the last pick: everything ranks after (+inf, -1)
  for (int t = 0; t < n_out; ++t) {
    float bv = -INFINITY;
    int32_t bc = INT32_MAX;
    if (better(pv, pc, ev, ec) && better(ev, ec, bv, bc)) {
      bv = ev;
      bc = ec;
    }
    for (int32_t i = x.lane; i < x.S; i += kWave) {
      const int32_t c = surv[i];
      if (c < 0) continue;
      const float v = __int_as_float(vals[i]);
      if (better(pv, pc, v, c) && better(v, c, bv, bc)) {
        bv = v;
        bc = c;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, kWave);
      const int32_t oc = __shfl_xor(bc, off, kWave);
      if (better(ov, oc, bv, bc)) {
        bv = ov;
        bc = oc;
      }
    }
    if (x.lane == 0) {
      part_val[int64_t(x.w) * x.K + t] = bv;
      part_col[int64_t(x.w) * x.K + t] = bc;
    }
    pv = bv;
    pc = bc;
  }
  if (x.lane == 0) part_cnt[x.w] = n_out;
}

// One chunk w (uniform) of the direct step, on one wave with two LDS arrays
// of kDirChunk slots (the chunk's columns, then the survivors' values; the
// pruning bound's small-slice sums, then the compacted survivors).
// status[0]: bad neighbour ids; status[1]: CSR rows out of order or a column
// repeated more than max_mult times.
__device__ __forceinline__ void ppr_chunk(
    const int64_t* __restrict__ col, int64_t n_nodes, const int32_t* __restrict__ st_cnt,
    const int64_t* __restrict__ seeds, int32_t K, float alpha, float keep, int32_t max_mult,
    const int32_t* __restrict__ chunk_off, const int32_t* __restrict__ row_of,
    const int64_t* __restrict__ tl_b, const int64_t* __restrict__ tl_len,
    const int64_t* __restrict__ tl_first, const int64_t* __restrict__ tl_last,
    const float* __restrict__ tl_w, const int32_t* __restrict__ tl_skip,
    const int32_t* __restrict__ seed_in, const float* __restrict__ seed_val,
    const float* __restrict__ row_tau, float* __restrict__ part_val,
    int32_t* __restrict__ part_col, int32_t* __restrict__ part_cnt, int32_t* status,
    const int32_t w, const int lane, int32_t* own_lds, float* small_sum) {
#pragma clang fp contract(off)
  const int32_t r = __builtin_amdgcn_readfirstlane(row_of[w]);
  const int32_t ci = w - __builtin_amdgcn_readfirstlane(chunk_off[r]);
  int n = __builtin_amdgcn_readfirstlane(st_cnt[r]);
  if (n < 0 || n > K) n = 0;
  // lane j < n holds list j: begin, length, weight, first and last column
  int64_t lb = 0, ll = 0, lfirst = 0, llast = -1;
  float lw = 0.f;
  bool lsk = false;  // skipped: no chunks of its own, and it owns no column
  if (lane < n) {
    const int64_t at = int64_t(r) * K + lane;
    lb = tl_b[at];
    ll = tl_len[at];
    lfirst = tl_first[at];
    llast = tl_last[at];
    lw = tl_w[at];
    lsk = tl_skip[at] != 0;
  }
  // this chunk's list j: the last list with chunks whose first chunk is <= ci
  const int32_t cj = lsk ? 0 : int32_t((ll + kDirChunk - 1) / kDirChunk);
  int32_t cinc = cj;
  for (int off = 1; off < kWave; off <<= 1) {
    const int32_t v = __shfl_up(cinc, off, kWave);
    if (lane >= off) cinc += v;
  }
  const uint64_t jm = __ballot(cj > 0 && cinc - cj <= ci);
  const int j = jm ? 63 - __clzll(jm) : -1;  // -1: no list (the teleport chunk of an empty row)
  int64_t p0 = 0, ej = 0, vmin = 0, vmax = -1;
  if (j >= 0) {
    const int32_t sub = ci - (__builtin_amdgcn_readlane(cinc, j) - __builtin_amdgcn_readlane(cj, j));
    const int64_t bj = lane_i64(lb, j);
    p0 = bj + int64_t(sub) * kDirChunk;
    ej = bj + lane_i64(ll, j);
    const int64_t pe = p0 + kDirChunk < ej ? p0 + kDirChunk : ej;
    vmin = col[p0];
    vmax = col[pe - 1];
  }
  const float wj_own = j >= 0 ? lane_f32(lw, j) : 0.f;
  const int64_t sd = seeds[r];
  const bool seed_ok = sd >= 0 && sd < n_nodes;

  // every other list's slice [slo, shi) of columns in [vmin, vmax]
  int64_t slo = 0, shi = 0;
  const bool need = j >= 0 && lane < n && lane != j && ll > 0 && vmax >= lfirst && vmin <= llast;
  coop_slices(col, n, need, lb, ll, vmin, vmax, lane, slo, shi);
  if (shi < slo) shi = slo;  // rows out of order (flagged where they are read)
  const int64_t sm = shi - slo;

  // this chunk's entries: column (also into LDS) and whether this entry owns it
  int32_t nv[kDirU];
  bool own[kDirU];
#pragma unroll
  for (int u = 0; u < kDirU; ++u) {
    const int64_t p = p0 + lane + u * kWave;
    own[u] = false;
    nv[u] = 0;
    own_lds[lane + u * kWave] = INT32_MAX;  // past the list: above every column
    small_sum[lane + u * kWave] = 0.f;
    if (j < 0 || p >= ej) continue;
    const int64_t x = col[p];
    own_lds[lane + u * kWave] = clamp_i32(x);
    bool o = x >= 0 && x < n_nodes;
    if (!o) atomicAdd(status, 1);
    const int64_t bj = ej - lane_i64(ll, j);
    if (p > bj) {
      const int64_t prev = col[p - 1];
      if (prev > x) atomicAdd(status + 1, 1);
      if (prev == x) o = false;  // a repeat: its first occurrence owns it
    }
    if (max_mult > 0 && p - max_mult >= bj && col[p - max_mult] == x) atomicAdd(status + 1, 1);
    if (o) nv[u] = int32_t(x);
    own[u] = o;
  }

  const float tau = row_tau[r];  // -inf: no bound for this row
  if (j >= 0 && tau > 0.f) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // slices of at most kDirRev entries: each entry is looked up among the
    // chunk's own (ascending) columns and adds its list's w to the slot of the
    // column's first occurrence, so small_sum holds those lists' exact share
    // of each column's sum (fp32 adds in any order: a bound, not the value);
    // larger slices count M * w until a lookup rules them out
    double big = 0.0, all = double(max_mult) * double(wj_own);
    for (int jj = 0; jj < n; ++jj) {
      const int64_t m = lane_i64(sm, jj);
      if (jj == j || m == 0) continue;
      const float wjj = lane_f32(lw, jj);
      all += double(max_mult) * double(wjj);
      if (m > kDirRev) {
        big += double(max_mult) * double(wjj);
        continue;
      }
      const int64_t lo_ = lane_i64(slo, jj);
      for (int32_t k0 = 0; k0 < int32_t(m); k0 += kWave) {
        const int32_t k = k0 + lane;
        if (k >= int32_t(m)) continue;
        const int32_t x = clamp_i32(col[lo_ + k]);
        int32_t a = 0;
        for (int32_t len = int32_t(kDirChunk); len > 1;) {
          const int32_t half = len >> 1;
          a = own_lds[a + half - 1] < x ? a + half : a;
          len -= half;
        }
        if (own_lds[a] < x) ++a;
        if (a < int32_t(kDirChunk) && own_lds[a] == x) atomicAdd(small_sum + a, wjj);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const double err = all * 0x1p-40;
    // a column survives while keep * (bound + rounding of the double sums)
    // * (1 + 2^-10) reaches tau; the seed always survives (alpha).  The fp32
    // share of the small slices is raised by 2^-16 to cover its roundings.
    const double cut = double(tau) / (double(keep) * (1.0 + 1.0 / 1024.0));
    const double fixed = double(max_mult) * double(wj_own) + big + err;  // own list: <= M repeats
#pragma unroll
    for (int u = 0; u < kDirU; ++u) {
      const double bnd = fixed + double(small_sum[lane + u * kWave]) * (1.0 + 0x1p-16);
      own[u] = own[u] && (bnd >= cut || (seed_ok && nv[u] == sd));
    }
  }

  // the surviving positions, compacted (small_sum's slots are free again)
  int32_t* surv = reinterpret_cast<int32_t*>(small_sum);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  int32_t S = 0;
#pragma unroll
  for (int u = 0; u < kDirU; ++u) {
    const uint64_t mk = __ballot(own[u]);
    if (own[u]) surv[S + __popcll(mk & below)] = lane + u * kWave;
    S += __popcll(mk);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  ChunkCtx x;
  x.col = col;
  x.own_lds = own_lds;
  x.surv = surv;
  x.S = S;
  x.n = n;
  x.j = j;
  x.lane = lane;
  x.p0 = p0;
  x.ej = ej;
  x.wj_own = wj_own;
  x.keep = keep;
  x.alpha = alpha;
  x.seed_ok = seed_ok;
  // the seed, when no list with chunks holds it, with its exact value
  x.extra = ci == 0 && seed_ok && !seed_in[r] && lane == 0;
  x.seed_v = seed_val[r];
  x.lsk = lsk;
  x.sd = sd;
  x.K = K;
  x.w = w;
  x.sm = sm;
  x.slo = slo;
  x.lw = lw;
  chunk_survivors(x, surv, own_lds, part_val, part_col, part_cnt);
}

// One wave per chunk.  status[1] also flags chunk counts past the bound the
// workspace was sized for (nothing is then written).
__global__ __launch_bounds__(kBlock) void k_ppr_direct(
    const int64_t* __restrict__ col, int64_t n_nodes, const int32_t* __restrict__ st_cnt,
    const int64_t* __restrict__ seeds, int32_t n_rows, int32_t K, float alpha, float keep,
    int32_t max_mult, const int32_t* __restrict__ chunk_off, int32_t max_chunks,
    const int32_t* __restrict__ row_of, const int64_t* __restrict__ tl_b,
    const int64_t* __restrict__ tl_len, const int64_t* __restrict__ tl_first,
    const int64_t* __restrict__ tl_last, const float* __restrict__ tl_w,
    const int32_t* __restrict__ tl_skip, const int32_t* __restrict__ seed_in,
    const float* __restrict__ seed_val, const float* __restrict__ row_tau,
    float* __restrict__ part_val, int32_t* __restrict__ part_col, int32_t* __restrict__ part_cnt,
    int32_t* status) {
  __shared__ int32_t own_all[kWaves][kDirChunk];
  __shared__ float small_all[kWaves][kDirChunk];
  const int32_t w = __builtin_amdgcn_readfirstlane(int(blockIdx.x * kWaves + (threadIdx.x >> 6)));
  const int lane = threadIdx.x & (kWave - 1);
  const int32_t n_chunks = __builtin_amdgcn_readfirstlane(chunk_off[n_rows]);
  if (n_chunks > max_chunks) {
    if (w == 0 && lane == 0) atomicAdd(status + 1, 1);
    return;
  }
  if (w >= n_chunks) return;
  ppr_chunk(col, n_nodes, st_cnt, seeds, K, alpha, keep, max_mult, chunk_off, row_of, tl_b, tl_len,
            tl_first, tl_last, tl_w, tl_skip, seed_in, seed_val, row_tau, part_val, part_col,
            part_cnt, status, w, lane, own_all[threadIdx.x >> 6], small_all[threadIdx.x >> 6]);
}

// One wave per row: the best K of its chunks' best K.
__global__ __launch_bounds__(kBlock) void k_ppr_merge(
    const int32_t* __restrict__ chunk_off, int32_t max_chunks, const float* __restrict__ part_val,
    const int32_t* __restrict__ part_col, const int32_t* __restrict__ part_cnt, int32_t n_rows,
    int32_t K, int32_t* __restrict__ out_col, float* __restrict__ out_val,
    int32_t* __restrict__ out_cnt) {
  const int32_t r = __builtin_amdgcn_readfirstlane(int(blockIdx.x * kWaves + (threadIdx.x >> 6)));
  const int lane = threadIdx.x & (kWave - 1);
  if (r >= n_rows || chunk_off[n_rows] > max_chunks) return;  // the latter flagged above
  const int32_t c0 = chunk_off[r], c1 = chunk_off[r + 1];
  if (c1 - c0 == 1) {
    const int32_t cnt = part_cnt[c0];
    if (lane < cnt) {
      out_col[int64_t(r) * K + lane] = part_col[int64_t(c0) * K + lane];
      out_val[int64_t(r) * K + lane] = part_val[int64_t(c0) * K + lane];
    }
    if (lane == 0) out_cnt[r] = cnt;
    return;
  }
  int32_t have = 0;
  for (int32_t c = c0 + lane; c < c1; c += kWave) have += part_cnt[c];
  for (int off = 32; off > 0; off >>= 1) have += __shfl_xor(have, off, kWave);
  const int n_out = have < K ? have : K;
  const int64_t m = int64_t(c1 - c0) * K;
  float pv = INFINITY;
  int32_t pc = -1;
  for (int t = 0; t < n_out; ++t) {
    float bv = -INFINITY;
    int32_t bc = INT32_MAX;
    for (int64_t i = lane; i < m; i += kWave) {
      const int32_t c = c0 + int32_t(i / K);
      const int32_t k = int32_t(i % K);
      if (k >= part_cnt[c]) continue;
      const float v = part_val[int64_t(c) * K + k];
      const int32_t cl = part_col[int64_t(c) * K + k];
      if (better(pv, pc, v, cl) && better(v, cl, bv, bc)) {
        bv = v;
        bc = cl;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, kWave);
      const int32_t oc = __shfl_xor(bc, off, kWave);
      if (better(ov, oc, bv, bc)) {
        bv = ov;
        bc = oc;
      }
    }
    if (lane == 0) {
      out_col[int64_t(r) * K + t] = bc;
      out_val[int64_t(r) * K + t] = bv;
    }
    pv = bv;
    pc = bc;
  }
  if (lane == 0) out_cnt[r] = n_out;
}

struct DirectLayout {
  size_t nch, chunk_off, temp, temp_bytes, row_of, tl_b, tl_len, tl_first, tl_last, tl_w, tl_skip,
      seed_in, seed_val, row_tau, part_val, part_col, part_cnt, total;
  int64_t max_chunks;
};

int direct_layout(int64_t total, int32_t n_rows, int32_t K, DirectLayout* L) {
  const size_t m = size_t(n_rows > 0 ? n_rows : 1);
  // a row's chunks: at most 1 + sum over its <= K lists of (length / kDirChunk + 1)
  L->max_chunks = int64_t(m) * (K + 1) + (total > 0 ? total : 0) / kDirChunk + 1;
  const size_t c = size_t(L->max_chunks);
  size_t scan_bytes = 0;
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan_bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                        int32_t(0), m + 1, rocprim::plus<int32_t>(),
                                        hipStream_t(0)));
  size_t off = 0;
  auto take = [&](size_t b) {
    const size_t at = off;
    off += align256(b);
    return at;
  };
  L->nch = take((m + 1) * 4);
  L->chunk_off = take((m + 1) * 4);
  L->temp_bytes = scan_bytes;
  L->temp = take(scan_bytes);
  L->row_of = take(c * 4);
  L->tl_b = take(m * size_t(K) * 8);
  L->tl_len = take(m * size_t(K) * 8);
  L->tl_first = take(m * size_t(K) * 8);
  L->tl_last = take(m * size_t(K) * 8);
  L->tl_w = take(m * size_t(K) * 4);
  L->tl_skip = take(m * size_t(K) * 4);
  L->seed_in = take(m * 4);
  L->seed_val = take(m * 4);
  L->row_tau = take(m * 4);
  L->part_val = take(c * size_t(K) * 4);
  L->part_col = take(c * size_t(K) * 4);
  L->part_cnt = take(c * 4);
  L->total = off;
  return NGT_OK;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_ppr_count_workspace_bytes(int32_t n_rows, size_t* bytes) {
  if (!bytes || n_rows < 0)
    return set_error(NGT_ERR_ARG, "ngt_ppr_count_workspace_bytes: bad arguments");
  size_t need = 0;
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, need, (int64_t*)nullptr, (int64_t*)nullptr,
                                        int64_t(0), size_t(n_rows) + 1,
                                        rocprim::plus<int64_t>(), hipStream_t(0)));
  *bytes = align256((size_t(n_rows) + 1) * 8) + need;
  return NGT_OK;
}

extern "C" int ngt_ppr_count(const int64_t* rowptr, int64_t n_nodes, const int32_t* st_col,
                             const int32_t* st_cnt, int32_t n_rows, int32_t K, int64_t* row_off,
                             int32_t* status, void* workspace, size_t workspace_bytes,
                             void* stream) {
  if (n_nodes < 0 || n_rows < 0 || K < 1 || K > kMaxK || !row_off || !status ||
      (n_rows > 0 && (!rowptr || !st_col || !st_cnt)))
    return set_error(NGT_ERR_ARG, "ngt_ppr_count: bad arguments (1 <= K <= %d)", kMaxK);
  size_t need = 0;
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, need, (int64_t*)nullptr, (int64_t*)nullptr,
                                        int64_t(0), size_t(n_rows) + 1,
                                        rocprim::plus<int64_t>(), hipStream_t(0)));
  const size_t cnt_bytes = align256((size_t(n_rows) + 1) * 8);
  if (!workspace || workspace_bytes < cnt_bytes + need)
    return set_error(NGT_ERR_WORKSPACE, "ngt_ppr_count: workspace %zu < %zu", workspace_bytes,
                     cnt_bytes + need);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int64_t* cnt = static_cast<int64_t*>(workspace);
  KernelTimer timer_("ppr_count", s);
  hipLaunchKernelGGL(k_ppr_count, dim3((n_rows + kBlock) / kBlock), dim3(kBlock), 0, s, rowptr,
                     n_nodes, st_col, st_cnt, n_rows, K, cnt, status);
  NGT_HIP_CHECK(hipGetLastError());
  // row_off[i] = sum of cnt[0..i), row_off[n_rows] = the total
  NGT_HIP_CHECK(rocprim::exclusive_scan(static_cast<char*>(workspace) + cnt_bytes, need, cnt,
                                        row_off, int64_t(0), size_t(n_rows) + 1,
                                        rocprim::plus<int64_t>(), s));
  return NGT_OK;
}

extern "C" int ngt_ppr_step_workspace_bytes(int64_t total, int32_t n_rows, size_t* bytes) {
  if (!bytes || total < 0 || n_rows < 0)
    return set_error(NGT_ERR_ARG, "ngt_ppr_step_workspace_bytes: bad arguments");
  PprLayout L;
  NGT_CHECK_OK(ppr_layout(total, n_rows, &L));
  *bytes = L.total;
  return NGT_OK;
}

extern "C" int ngt_ppr_step(const int64_t* rowptr, const int64_t* col, const float* inv_deg,
                            int64_t n_nodes, const int32_t* st_col, const float* st_val,
                            const int32_t* st_cnt, const int64_t* seeds, int32_t n_rows,
                            int32_t K, float alpha, float keep, const int64_t* row_off,
                            int64_t total, int32_t* out_col, float* out_val, int32_t* out_cnt,
                            int32_t* status, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (n_nodes < 0 || n_rows < 0 || K < 1 || K > kMaxK || total < n_rows ||
      (n_rows > 0 && (!rowptr || !inv_deg || !st_col || !st_val || !st_cnt || !seeds ||
                      !row_off || !out_col || !out_val || !out_cnt || !status)))
    return set_error(NGT_ERR_ARG, "ngt_ppr_step: bad arguments");
  if (n_nodes >= (int64_t(1) << 31) || n_rows >= (1 << 30) || total >= (int64_t(1) << 31))
    return set_error(NGT_ERR_UNSUPPORTED,
                     "ngt_ppr_step: node, row or product count too large (split the batch)");
  if (n_rows == 0) return NGT_OK;
  PprLayout L;
  NGT_CHECK_OK(ppr_layout(total, n_rows, &L));
  if (!workspace || workspace_bytes < L.total)
    return set_error(NGT_ERR_WORKSPACE, "ngt_ppr_step: workspace %zu < %zu", workspace_bytes,
                     L.total);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* seg_row = reinterpret_cast<int32_t*>(ws + L.seg_row);
  int32_t* seg_col = reinterpret_cast<int32_t*>(ws + L.seg_col);
  float* seg_val = reinterpret_cast<float*>(ws + L.seg_val);
  int32_t* n_seg = reinterpret_cast<int32_t*>(ws + L.n_seg);
  KernelTimer timer_("ppr_step", s);
  KeyFmt f;
  int cb = 1;  // column bits, leaving the all-ones column unused
  while ((int64_t(1) << cb) - 1 < n_nodes) ++cb;
  f.rs = cb + 1;
  f.deadcol = uint32_t((uint64_t(1) << cb) - 1);
  int row_bits = 1;
  while ((int64_t(1) << row_bits) < n_rows) ++row_bits;
  const unsigned end_bit = unsigned(f.rs + row_bits);
  if (end_bit <= 32)
    NGT_CHECK_OK(ppr_sort_reduce<uint32_t>(rowptr, col, inv_deg, n_nodes, st_col, st_val, st_cnt,
                                           seeds, n_rows, K, alpha, keep, row_off, total, f,
                                           end_bit, status, ws, L, s));
  else
    NGT_CHECK_OK(ppr_sort_reduce<uint64_t>(rowptr, col, inv_deg, n_nodes, st_col, st_val, st_cnt,
                                           seeds, n_rows, K, alpha, keep, row_off, total, f,
                                           end_bit, status, ws, L, s));
  hipLaunchKernelGGL(k_ppr_topk, dim3(grid_waves(n_rows)), dim3(kBlock), 0, s, seg_row, seg_col,
                     seg_val, n_seg, n_rows, K, out_col, out_val, out_cnt);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_ppr_step_direct_workspace_bytes(int64_t total, int32_t n_rows, int32_t K,
                                                   size_t* bytes) {
  if (!bytes || total < 0 || n_rows < 0 || K < 1 || K > kMaxK)
    return set_error(NGT_ERR_ARG, "ngt_ppr_step_direct_workspace_bytes: bad arguments");
  DirectLayout L;
  NGT_CHECK_OK(direct_layout(total, n_rows, K, &L));
  *bytes = L.total;
  return NGT_OK;
}

extern "C" int ngt_ppr_step_direct(const int64_t* rowptr, const int64_t* col,
                                   const float* inv_deg, int64_t n_nodes, const int32_t* st_col,
                                   const float* st_val, const int32_t* st_cnt,
                                   const int64_t* seeds, int32_t n_rows, int32_t K, float alpha,
                                   float keep, int32_t max_mult, int64_t total,
                                   int32_t* out_col, float* out_val,
                                   int32_t* out_cnt, int32_t* status, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (n_nodes < 0 || n_rows < 0 || K < 1 || K > kMaxK || total < n_rows || max_mult < 0 ||
      (n_rows > 0 && (!rowptr || !col || !inv_deg || !st_col || !st_val || !st_cnt || !seeds ||
                      !out_col || !out_val || !out_cnt || !status)))
    return set_error(NGT_ERR_ARG, "ngt_ppr_step_direct: bad arguments");
  if (n_nodes >= (int64_t(1) << 31) || n_rows >= (1 << 30) ||
      total / kDirChunk + int64_t(n_rows) * (K + 1) >= (int64_t(1) << 31) - 1)
    return set_error(NGT_ERR_UNSUPPORTED,
                     "ngt_ppr_step_direct: node, row or product count too large (split the batch)");
  if (n_rows == 0) return NGT_OK;
  DirectLayout L;
  NGT_CHECK_OK(direct_layout(total, n_rows, K, &L));
  if (!workspace || workspace_bytes < L.total)
    return set_error(NGT_ERR_WORKSPACE, "ngt_ppr_step_direct: workspace %zu < %zu",
                     workspace_bytes, L.total);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* nch = reinterpret_cast<int32_t*>(ws + L.nch);
  int32_t* chunk_off = reinterpret_cast<int32_t*>(ws + L.chunk_off);
  float* part_val = reinterpret_cast<float*>(ws + L.part_val);
  int32_t* part_col = reinterpret_cast<int32_t*>(ws + L.part_col);
  int32_t* part_cnt = reinterpret_cast<int32_t*>(ws + L.part_cnt);
  KernelTimer timer_("ppr_step", s);
  int64_t* tl_b = reinterpret_cast<int64_t*>(ws + L.tl_b);
  int64_t* tl_len = reinterpret_cast<int64_t*>(ws + L.tl_len);
  int64_t* tl_first = reinterpret_cast<int64_t*>(ws + L.tl_first);
  int64_t* tl_last = reinterpret_cast<int64_t*>(ws + L.tl_last);
  float* tl_w = reinterpret_cast<float*>(ws + L.tl_w);
  int32_t* seed_in = reinterpret_cast<int32_t*>(ws + L.seed_in);
  int32_t* tl_skip = reinterpret_cast<int32_t*>(ws + L.tl_skip);
  float* seed_val = reinterpret_cast<float*>(ws + L.seed_val);
  float* row_tau = reinterpret_cast<float*>(ws + L.row_tau);
  int32_t* row_of = reinterpret_cast<int32_t*>(ws + L.row_of);
  const int32_t max_chunks = int32_t(L.max_chunks);
  hipLaunchKernelGGL(k_ppr_rows, dim3(grid_waves(int64_t(n_rows) + 1)), dim3(kBlock), 0, s,
                     rowptr, col, inv_deg, n_nodes, st_col, st_val, st_cnt, seeds, n_rows, K,
                     alpha, keep, max_mult, tl_b, tl_len, tl_first, tl_last, tl_w, tl_skip, nch,
                     seed_in, seed_val, row_tau, status);
  NGT_HIP_CHECK(hipGetLastError());
  size_t tb = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::exclusive_scan(ws + L.temp, tb, nch, chunk_off, int32_t(0),
                                        size_t(n_rows) + 1, rocprim::plus<int32_t>(), s));
  hipLaunchKernelGGL(k_ppr_chunk_rows, dim3((n_rows + kBlock - 1) / kBlock), dim3(kBlock), 0, s,
                     chunk_off, n_rows, max_chunks, row_of);
  NGT_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(k_ppr_direct, dim3(grid_waves(L.max_chunks)), dim3(kBlock), 0, s, col,
                     n_nodes, st_cnt, seeds, n_rows, K, alpha, keep,
                     max_mult, chunk_off, max_chunks, row_of, tl_b, tl_len, tl_first, tl_last,
                     tl_w, tl_skip, seed_in, seed_val, row_tau, part_val, part_col, part_cnt,
                     status);
  NGT_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(k_ppr_merge, dim3(grid_waves(n_rows)), dim3(kBlock), 0, s, chunk_off,
                     int32_t(L.max_chunks), part_val, part_col, part_cnt, n_rows, K, out_col,
                     out_val, out_cnt);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}
