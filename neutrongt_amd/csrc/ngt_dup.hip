// Duplicate-node layout of a rank's windows on the GPU
// (_compute_local_duplicate_nodes, NeutronGT/core/node_level_pipeline/
// window_state.py:52-73, and build_dup_cache_metadata, :181-205).
//
// The rank's W windows arrive as one int64 array of T node ids with window
// offsets win_ptr[0..W].  A node is a duplicate when it occurs at least
// min_count times in the whole array (2 for the rerange; 1 makes every node
// a cache entry, which is the cache metadata of a given set of duplicate
// lists).  Everything follows from one stable sort of the ids:
//   - runs of equal ids in sorted order give each id's count, so an element
//     is a duplicate when its run is at least min_count long;
//   - the duplicate runs, in sorted order, are the cache: cache_ids is the
//     sorted unique duplicate ids and an element's cache index is its run's
//     rank among the duplicate runs (what searchsorted returns for it);
//   - an exclusive scan of the per-element duplicate flags, taken in the
//     original order, places each window's duplicates first and the rest
//     after them, both in original order (a stable split), and lists every
//     window's cache indices back to back.
#include "ngt_common.h"

#include <algorithm>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

namespace ngt {
namespace {

constexpr int kBlock = 256;

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline unsigned grid_for(int64_t n) {
  int64_t g = (n + kBlock - 1) / kBlock;
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

// idx = 0..T-1 (the sort's values), info = 0, and flag[T] = 0, which closes
// the exclusive scan of the flags: its entry T is the number of duplicates.
__global__ void k_dup_iota(int32_t* __restrict__ idx, int64_t T, int64_t* __restrict__ info,
                           int32_t* __restrict__ flag) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i < T) idx[i] = static_cast<int32_t>(i);
  if (i < 3) info[i] = 0;
  if (i == 0) flag[T] = 0;
}

// Over the sorted ids: flag[pos] = 1 for elements of runs of >= min_count
// equal ids; head[s] = 1 at the first element of each such run.  An element
// counts its equal neighbours up to min_count - 1 on each side.
__global__ void k_dup_mark(const int64_t* __restrict__ key, const int32_t* __restrict__ pos,
                           int64_t T, int32_t min_count, int32_t* __restrict__ flag,
                           int32_t* __restrict__ head) {
  const int64_t s = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (s >= T) return;
  const int64_t k = key[s];
  const int64_t need = int64_t(min_count) - 1;
  int64_t back = 0, ahead = 0;
  while (back < need && s - back - 1 >= 0 && key[s - back - 1] == k) ++back;
  while (ahead < need && s + ahead + 1 < T && key[s + ahead + 1] == k) ++ahead;
  const bool dup = back + ahead >= need;
  const bool first = s == 0 || key[s - 1] != k;
  flag[pos[s]] = dup ? 1 : 0;
  head[s] = dup && first ? 1 : 0;
}

// cache_ids[run rank] = id at each duplicate run's head; every duplicate
// element gets its run's rank as its cache index (in original order);
// info[0] = number of cache entries.
__global__ void k_dup_cache(const int64_t* __restrict__ key, const int32_t* __restrict__ pos,
                            const int32_t* __restrict__ head, const int32_t* __restrict__ run,
                            const int32_t* __restrict__ flag, int64_t T,
                            int64_t* __restrict__ cache_ids, int32_t* __restrict__ cidx,
                            int64_t* __restrict__ info) {
  const int64_t s = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (s >= T) return;
  const int32_t p = pos[s];
  const int32_t r = run[s] - 1;  // inclusive scan of head: this run's rank
  if (head[s]) cache_ids[r] = key[s];
  cidx[p] = flag[p] ? r : -1;
  if (s + 1 == T) info[0] = run[s];
}

// The window of element p: the w with win_ptr[w] <= p < win_ptr[w+1], or -1.
__device__ __forceinline__ int32_t window_of(const int64_t* __restrict__ win_ptr, int32_t W,
                                             int64_t p) {
  int32_t lo = 0, hi = W;  // invariant: answer in [lo, hi)
  while (hi - lo > 1) {
    const int32_t mid = (lo + hi) >> 1;
    if (win_ptr[mid] <= p) lo = mid; else hi = mid;
  }
  return (W > 0 && win_ptr[lo] <= p && p < win_ptr[lo + 1]) ? lo : -1;
}

// Stable split of each window into [duplicates, the rest] and the
// back-to-back list of the windows' cache indices.  dscan = exclusive scan of
// flag over [0, T]; info[1] = total duplicates, info[2] = elements whose
// window offsets were malformed (nothing is written for them).
__global__ void k_dup_emit(const int64_t* __restrict__ nodes, const int64_t* __restrict__ win_ptr,
                           int32_t W, int64_t T, const int32_t* __restrict__ flag,
                           const int32_t* __restrict__ dscan, const int32_t* __restrict__ cidx,
                           int64_t* __restrict__ reranged, int64_t* __restrict__ dup_index,
                           int64_t* __restrict__ info) {
  const int64_t p = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (p == 0) info[1] = dscan[T];
  if (p >= T) return;
  const int32_t w = window_of(win_ptr, W, p);
  if (w < 0) {
    atomicAdd(reinterpret_cast<unsigned long long*>(info + 2), 1ull);
    return;
  }
  const int64_t a = win_ptr[w], b = win_ptr[w + 1];
  if (a < 0 || b > T) {
    atomicAdd(reinterpret_cast<unsigned long long*>(info + 2), 1ull);
    return;
  }
  const int64_t da = dscan[a], nd = int64_t(dscan[b]) - da, before = int64_t(dscan[p]) - da;
  const int64_t at = flag[p] ? a + before : a + nd + (p - a) - before;
  reranged[at] = nodes[p];
  if (flag[p]) dup_index[dscan[p]] = cidx[p];
}

// dup_ptr[w] = offset of window w's cache indices (w <= W).
__global__ void k_dup_ptr(const int64_t* __restrict__ win_ptr, int32_t W,
                          const int32_t* __restrict__ dscan, int64_t T,
                          int64_t* __restrict__ dup_ptr) {
  const int64_t w = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (w > W) return;
  int64_t o = win_ptr[w];
  o = o < 0 ? 0 : (o > T ? T : o);
  dup_ptr[w] = dscan[o];
}

struct DupLayout {
  size_t key_b, idx_a, pos, flag, head, run, dscan, cidx, temp, total, temp_bytes;
};

int dup_layout(int64_t T, DupLayout* L) {
  const size_t t = size_t(T > 0 ? T : 1);
  size_t sort = 0, scan_a = 0, scan_b = 0;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, sort, (int64_t*)nullptr, (int64_t*)nullptr,
                                          (int32_t*)nullptr, (int32_t*)nullptr, t, 0u, 64u,
                                          hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::inclusive_scan(nullptr, scan_a, (int32_t*)nullptr, (int32_t*)nullptr, t,
                                        rocprim::plus<int32_t>(), hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan_b, (int32_t*)nullptr, (int32_t*)nullptr, 0,
                                        t + 1, rocprim::plus<int32_t>(), hipStream_t(0)));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  };
  L->key_b = take(t * 8);
  L->idx_a = take(t * 4);
  L->pos = take(t * 4);
  L->flag = take((t + 1) * 4);
  L->head = take(t * 4);
  L->run = take(t * 4);
  L->dscan = take((t + 1) * 4);
  L->cidx = take(t * 4);
  L->temp_bytes = std::max(sort, std::max(scan_a, scan_b));
  L->temp = take(L->temp_bytes);
  L->total = off;
  return NGT_OK;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_window_dup_workspace_bytes(int64_t n_nodes, size_t* bytes) {
  if (n_nodes < 0 || !bytes)
    return set_error(NGT_ERR_ARG, "ngt_window_dup_workspace_bytes: bad arguments");
  DupLayout L{};
  NGT_CHECK_OK(dup_layout(n_nodes, &L));
  *bytes = L.total;
  return NGT_OK;
}

extern "C" int ngt_window_dup_layout(const int64_t* nodes, int64_t n_nodes, const int64_t* win_ptr,
                                     int32_t n_windows, int32_t min_count, int64_t* reranged,
                                     int64_t* dup_ptr, int64_t* cache_ids, int64_t* dup_index,
                                     int64_t* info, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (n_nodes < 0 || n_windows < 0 || min_count < 1 || min_count > 65536)
    return set_error(NGT_ERR_ARG, "ngt_window_dup_layout: bad sizes (n_nodes=%lld n_windows=%d "
                     "min_count=%d)", static_cast<long long>(n_nodes), n_windows, min_count);
  if (n_nodes > 0x7ffffffe)
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_window_dup_layout: at most 2^31 - 2 node ids");
  if (!win_ptr || !dup_ptr || !info ||
      (n_nodes > 0 && (!nodes || !reranged || !cache_ids || !dup_index)))
    return set_error(NGT_ERR_ARG, "ngt_window_dup_layout: null pointer");
  DupLayout L{};
  NGT_CHECK_OK(dup_layout(n_nodes, &L));
  if (!workspace || workspace_bytes < L.total)
    return set_error(NGT_ERR_WORKSPACE, "ngt_window_dup_layout: workspace %zu < %zu",
                     workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int64_t T = n_nodes;
  int64_t* key_b = reinterpret_cast<int64_t*>(ws + L.key_b);
  int32_t* idx_a = reinterpret_cast<int32_t*>(ws + L.idx_a);
  int32_t* pos = reinterpret_cast<int32_t*>(ws + L.pos);
  int32_t* flag = reinterpret_cast<int32_t*>(ws + L.flag);
  int32_t* head = reinterpret_cast<int32_t*>(ws + L.head);
  int32_t* run = reinterpret_cast<int32_t*>(ws + L.run);
  int32_t* dscan = reinterpret_cast<int32_t*>(ws + L.dscan);
  int32_t* cidx = reinterpret_cast<int32_t*>(ws + L.cidx);
  void* temp = ws + L.temp;
  KernelTimer timer_("window_dup_layout", st);
  hipLaunchKernelGGL(k_dup_iota, dim3(grid_for(T)), dim3(kBlock), 0, st, idx_a, T, info, flag);
  NGT_HIP_CHECK(hipGetLastError());
  if (T > 0) {
    size_t tb = L.temp_bytes;
    // stable by id (elements of one id keep their original order)
    NGT_HIP_CHECK(rocprim::radix_sort_pairs(temp, tb, nodes, key_b, idx_a, pos, size_t(T), 0u,
                                            64u, st));
    hipLaunchKernelGGL(k_dup_mark, dim3(grid_for(T)), dim3(kBlock), 0, st, key_b, pos, T,
                       min_count, flag, head);
    NGT_HIP_CHECK(hipGetLastError());
    tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::inclusive_scan(temp, tb, head, run, size_t(T),
                                          rocprim::plus<int32_t>(), st));
    hipLaunchKernelGGL(k_dup_cache, dim3(grid_for(T)), dim3(kBlock), 0, st, key_b, pos, head, run,
                       flag, T, cache_ids, cidx, info);
    NGT_HIP_CHECK(hipGetLastError());
  }
  size_t tb = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::exclusive_scan(temp, tb, flag, dscan, 0, size_t(T + 1),
                                        rocprim::plus<int32_t>(), st));
  hipLaunchKernelGGL(k_dup_emit, dim3(grid_for(T)), dim3(kBlock), 0, st, nodes, win_ptr,
                     n_windows, T, flag, dscan, cidx, reranged, dup_index, info);
  NGT_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(k_dup_ptr, dim3(grid_for(int64_t(n_windows) + 1)), dim3(kBlock), 0, st,
                     win_ptr, n_windows, dscan, T, dup_ptr);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}
