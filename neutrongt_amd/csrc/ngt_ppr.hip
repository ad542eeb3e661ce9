// APPNP personalised PageRank with per-row top-k, on the GPU.
//
// One propagation step of personal_pagerank_appnp
// (NeutronGT/core/ppr_backends/appnp_backend.py:179-224 with the SpGEMM of
// cusparse_spgemm.cu:65-267) for a batch of seed rows:
//   next[r, :] = topk_K( (1 - alpha) * (state[r, :] P) + alpha * e_seed(r) )
// with P[c, n] = 1 / max(deg(c), 1) for every edge c -> n of the graph CSR.
//
// The state is fixed-width: row r holds cnt[r] <= K entries (col, val) in
// rank order (value descending, then column ascending).  A step is
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
    const int64_t* __restrict__ row_off, KeyFmt f, KeyT* __restrict__ keys,
    float* __restrict__ vals, int32_t* status) {
  const int64_t r = blockIdx.x * int64_t(kWaves) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & (kWave - 1);
  if (r >= n_rows) return;
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
                     col, inv_deg, n_nodes, st_col, st_val, st_cnt, seeds, n_rows, K, row_off, f,
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
