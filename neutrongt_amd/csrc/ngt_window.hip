// Window preparation on the GPU: related-node selection and feature-row
// assembly.
//
// Related nodes (NeutronGT/core/metisPartition.py:397-425): the reference walks
// the partition in order, and for each adjacency entry (nb, w) with nb outside
// the partition adds w to a dict keyed by nb (insertion order = first
// appearance), then sorts the dict stably by weight descending and keeps the
// first len * pct // 100.  Here every adjacency entry of the partition gets a
// traversal index (prefix sum of partition degrees + offset); per external
// node the GPU keeps the integer weight sum (atomic add, exact) and the
// smallest traversal index (atomic min) -- its dict insertion position.  One
// radix sort by (weight desc, first appearance asc) reproduces the stable
// ranking exactly; membership flags + a scan emit the sorted union.
#include "ngt_common.h"

#include <limits.h>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr uint64_t kMaxWeight = (uint64_t(1) << 33) - 1;

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline int grid_for(int64_t n) {
  int64_t g = (n + kBlock - 1) / kBlock;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return static_cast<int>(g);
}

struct RelLayout {
  size_t in_part, first_seen, wsum, deg, base, nseg, seg_end, keys_a, keys_b, ids_a, ids_b, member,
      pos, temp, total, temp_bytes;
};

// A partition node's adjacency is walked in segments of kRelSeg entries, one
// wave each, so a hub node (hundreds of thousands of neighbours) is spread
// over many waves instead of serialising one.
constexpr int32_t kRelSeg = 2048;

int rel_layout(int32_t n_nodes, int32_t n_part, RelLayout* L) {
  const size_t n = size_t(n_nodes > 0 ? n_nodes : 1);
  const size_t np = size_t(n_part > 0 ? n_part : 1);
  size_t sort_bytes = 0, scan_bytes = 0, scan2 = 0;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, sort_bytes, (uint64_t*)nullptr,
                                          (uint64_t*)nullptr, (int32_t*)nullptr,
                                          (int32_t*)nullptr, n, 0u, 64u, hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan_bytes, (int32_t*)nullptr, (int32_t*)nullptr,
                                        int32_t(0), n, rocprim::plus<int32_t>(), hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan2, (int32_t*)nullptr, (int32_t*)nullptr,
                                        int32_t(0), np, rocprim::plus<int32_t>(), hipStream_t(0)));
  size_t scan3 = 0;
  NGT_HIP_CHECK(rocprim::inclusive_scan(nullptr, scan3, (int32_t*)nullptr, (int32_t*)nullptr, np,
                                        rocprim::plus<int32_t>(), hipStream_t(0)));
  if (scan3 > scan2) scan2 = scan3;
  size_t off = 0;
  auto take = [&](size_t b) {
    const size_t at = off;
    off += align256(b);
    return at;
  };
  L->in_part = take(n * 4);
  L->first_seen = take(n * 4);
  L->wsum = take(n * 8);
  L->deg = take(np * 4);
  L->base = take(np * 4);
  L->nseg = take(np * 4);
  L->seg_end = take(np * 4);
  L->keys_a = take(n * 8);
  L->keys_b = take(n * 8);
  L->ids_a = take(n * 4);
  L->ids_b = take(n * 4);
  L->member = take(n * 4);
  L->pos = take(n * 4);
  L->temp_bytes = sort_bytes;
  if (scan_bytes > L->temp_bytes) L->temp_bytes = scan_bytes;
  if (scan2 > L->temp_bytes) L->temp_bytes = scan2;
  L->temp = take(L->temp_bytes);
  L->total = off;
  return NGT_OK;
}

// status[0] = output length, status[1] = external neighbours, status[2] = errors
__global__ void k_rel_init(int32_t n_nodes, int32_t* in_part, int32_t* first_seen,
                           unsigned long long* wsum, int32_t* member, int32_t* status) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n_nodes;
       i += int64_t(gridDim.x) * blockDim.x) {
    in_part[i] = 0;
    first_seen[i] = INT_MAX;
    wsum[i] = 0ull;
    member[i] = 0;
  }
  if (blockIdx.x == 0 && threadIdx.x < 3) status[threadIdx.x] = 0;
}

__global__ void k_rel_mark(const int64_t* __restrict__ part, int32_t n_part,
                           const int32_t* __restrict__ xadj, int32_t n_nodes, int32_t* in_part,
                           int32_t* member, int32_t* deg, int32_t* status) {
  for (int64_t p = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; p < n_part;
       p += int64_t(gridDim.x) * blockDim.x) {
    const int64_t u = part[p];
    if (u < 0 || u >= n_nodes) {
      atomicAdd(status + 2, 1);
      deg[p] = 0;
      continue;
    }
    in_part[u] = 1;
    member[u] = 1;
    const int32_t d = xadj[u + 1] - xadj[u];
    if (d < 0) atomicAdd(status + 2, 1);  // a decreasing row pointer: rejected, row skipped
    deg[p] = d < 0 ? 0 : d;
  }
}

__global__ void k_rel_segs(const int32_t* __restrict__ deg, int32_t n_part, int32_t* nseg) {
  for (int64_t p = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; p < n_part;
       p += int64_t(gridDim.x) * blockDim.x)
    nseg[p] = (deg[p] + kRelSeg - 1) / kRelSeg;
}

// Waves stride over the segments (their count is read on the device, so every
// wave ends); a wave finds its partition position by binary search over the
// inclusive scan of the per-position segment counts.
__global__ void k_rel_accumulate(const int64_t* __restrict__ part, int32_t n_part,
                                 const int32_t* __restrict__ xadj,
                                 const int32_t* __restrict__ adjncy,
                                 const int32_t* __restrict__ eweights, int32_t n_nodes,
                                 const int32_t* __restrict__ in_part,
                                 const int32_t* __restrict__ base,
                                 const int32_t* __restrict__ nseg,
                                 const int32_t* __restrict__ seg_end, int32_t* first_seen,
                                 unsigned long long* wsum, int32_t* status) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t waves = int64_t(gridDim.x) * (blockDim.x / kWave);
  const int64_t n_segs = seg_end[n_part - 1];
  for (int64_t w = blockIdx.x * int64_t(blockDim.x / kWave) + (threadIdx.x / kWave); w < n_segs;
       w += waves) {
    int lo = 0, hi = n_part - 1;  // first p with seg_end[p] > w
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (seg_end[mid] > w)
        hi = mid;
      else
        lo = mid + 1;
    }
    const int64_t u = part[lo];  // in range: an invalid u has no segments
    const int32_t row_b = xadj[u], row_e = xadj[u + 1];
    const int32_t b = row_b + int32_t(w - (seg_end[lo] - nseg[lo])) * kRelSeg;
    const int32_t e = b + kRelSeg < row_e ? b + kRelSeg : row_e;
    for (int32_t a = b + lane; a < e; a += kWave) {
      const int32_t nb = adjncy[a];
      if (nb < 0 || nb >= n_nodes) {
        atomicAdd(status + 2, 1);
        continue;
      }
      if (in_part[nb]) continue;
      const int32_t wt = eweights[a];
      if (wt < 0) atomicAdd(status + 2, 1);
      atomicMin(first_seen + nb, base[lo] + (a - row_b));
      atomicAdd(wsum + nb, static_cast<unsigned long long>(wt < 0 ? 0 : wt));
    }
  }
}

__global__ void k_rel_keys(int32_t n_nodes, const int32_t* __restrict__ first_seen,
                           const unsigned long long* __restrict__ wsum, uint64_t* keys,
                           int32_t* ids, int32_t* status) {
  int32_t local = 0;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n_nodes;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int32_t fs = first_seen[i];
    uint64_t key = ~uint64_t(0);
    if (fs != INT_MAX) {
      uint64_t w = wsum[i];
      if (w > kMaxWeight) {
        atomicAdd(status + 2, 1);
        w = kMaxWeight;
      }
      key = ((kMaxWeight - w) << 31) | uint64_t(fs);
      ++local;
    }
    keys[i] = key;
    ids[i] = static_cast<int32_t>(i);
  }
  if (local) atomicAdd(status + 1, local);
}

__global__ void k_rel_select(const int32_t* __restrict__ ids_sorted, int32_t pct,
                             int32_t* member, const int32_t* __restrict__ status) {
  const int64_t n_ext = status[1];
  const int64_t n_select = pct > 0 ? (n_ext * pct) / 100 : 0;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < n_select;
       t += int64_t(gridDim.x) * blockDim.x)
    member[ids_sorted[t]] = 1;
}

__global__ void k_rel_emit(int32_t n_nodes, const int32_t* __restrict__ member,
                           const int32_t* __restrict__ pos, int64_t* __restrict__ out,
                           int32_t* status) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n_nodes;
       i += int64_t(gridDim.x) * blockDim.x) {
    if (member[i]) out[pos[i]] = i;
    if (i == n_nodes - 1) status[0] = pos[i] + member[i];
  }
}

__global__ void k_gather_rows(const uint32_t* __restrict__ src, int64_t n_src,
                              const int64_t* __restrict__ idx, int64_t n_rows, int64_t words,
                              uint32_t* __restrict__ dst, int32_t* bad) {
  const int64_t total = n_rows * words;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = t / words;
    const int64_t w = t - r * words;
    const int64_t s = idx[r];
    const bool ok = s >= 0 && s < n_src;
    dst[t] = ok ? src[s * words + w] : 0u;
    if (!ok && w == 0 && bad) atomicAdd(bad, 1);
  }
}

// out[s] = vals[seg[s]] + vals[seg[s]+1] + ... + vals[seg[s+1]-1], summed from
// 0.0f one element at a time in index order: the rounding of a sequential
// index_add_ over the same elements in the same order.
__global__ void k_segment_sum(const float* __restrict__ vals, int64_t n_vals,
                              const int64_t* __restrict__ seg, int64_t n_seg,
                              float* __restrict__ out, int32_t* bad) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n_seg) return;
  const int64_t b = seg[i], e = seg[i + 1];
  if (b < 0 || e < b || e > n_vals) {
    atomicAdd(bad, 1);
    out[i] = 0.f;
    return;
  }
  float acc = 0.f;
  for (int64_t p = b; p < e; ++p) acc += vals[p];
  out[i] = acc;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_related_workspace_bytes(int32_t n_nodes, int32_t n_part, size_t* bytes) {
  if (!bytes || n_nodes < 0 || n_part < 0)
    return set_error(NGT_ERR_ARG, "ngt_related_workspace_bytes: bad arguments");
  RelLayout L;
  const int rc = rel_layout(n_nodes, n_part, &L);
  if (rc != NGT_OK) return rc;
  *bytes = L.total;
  return NGT_OK;
}

extern "C" int ngt_merge_related_nodes(const int32_t* xadj, const int32_t* adjncy,
                                       const int32_t* eweights, int32_t n_nodes,
                                       const int64_t* partition, int32_t n_part,
                                       int32_t topk_percent, int64_t* out, int32_t* out_len,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  if (n_nodes < 0 || n_part < 0 || !out_len || (n_nodes > 0 && (!xadj || !out)) ||
      (n_part > 0 && !partition))
    return set_error(NGT_ERR_ARG, "ngt_merge_related_nodes: bad arguments");
  if (n_part > n_nodes)
    return set_error(NGT_ERR_ARG, "ngt_merge_related_nodes: partition larger than the graph");
  RelLayout L;
  int rc = rel_layout(n_nodes, n_part, &L);
  if (rc != NGT_OK) return rc;
  if (!workspace || workspace_bytes < L.total)
    return set_error(NGT_ERR_WORKSPACE, "ngt_merge_related_nodes: workspace %zu < %zu",
                     workspace_bytes, L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* in_part = reinterpret_cast<int32_t*>(ws + L.in_part);
  int32_t* first_seen = reinterpret_cast<int32_t*>(ws + L.first_seen);
  unsigned long long* wsum = reinterpret_cast<unsigned long long*>(ws + L.wsum);
  int32_t* deg = reinterpret_cast<int32_t*>(ws + L.deg);
  int32_t* base = reinterpret_cast<int32_t*>(ws + L.base);
  uint64_t* keys_a = reinterpret_cast<uint64_t*>(ws + L.keys_a);
  uint64_t* keys_b = reinterpret_cast<uint64_t*>(ws + L.keys_b);
  int32_t* ids_a = reinterpret_cast<int32_t*>(ws + L.ids_a);
  int32_t* ids_b = reinterpret_cast<int32_t*>(ws + L.ids_b);
  int32_t* member = reinterpret_cast<int32_t*>(ws + L.member);
  int32_t* pos = reinterpret_cast<int32_t*>(ws + L.pos);

  hipLaunchKernelGGL(k_rel_init, dim3(grid_for(n_nodes)), dim3(kBlock), 0, st, n_nodes, in_part,
                     first_seen, wsum, member, out_len);
  NGT_HIP_CHECK(hipGetLastError());
  if (n_nodes == 0) return NGT_OK;
  if (n_part > 0) {
    hipLaunchKernelGGL(k_rel_mark, dim3(grid_for(n_part)), dim3(kBlock), 0, st, partition, n_part,
                       xadj, n_nodes, in_part, member, deg, out_len);
    NGT_HIP_CHECK(hipGetLastError());
    size_t tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::exclusive_scan(ws + L.temp, tb, deg, base, int32_t(0), size_t(n_part),
                                          rocprim::plus<int32_t>(), st));
    int32_t* nseg = reinterpret_cast<int32_t*>(ws + L.nseg);
    int32_t* seg_end = reinterpret_cast<int32_t*>(ws + L.seg_end);
    hipLaunchKernelGGL(k_rel_segs, dim3(grid_for(n_part)), dim3(kBlock), 0, st, deg, n_part, nseg);
    tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::inclusive_scan(ws + L.temp, tb, nseg, seg_end, size_t(n_part),
                                          rocprim::plus<int32_t>(), st));
    hipLaunchKernelGGL(k_rel_accumulate, dim3(grid_for(int64_t(n_part) * kWave)), dim3(kBlock), 0,
                       st, partition, n_part, xadj, adjncy, eweights, n_nodes, in_part, base, nseg,
                       seg_end, first_seen, wsum, out_len);
    NGT_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(k_rel_keys, dim3(grid_for(n_nodes)), dim3(kBlock), 0, st, n_nodes,
                     first_seen, wsum, keys_a, ids_a, out_len);
  NGT_HIP_CHECK(hipGetLastError());
  size_t tb = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(ws + L.temp, tb, keys_a, keys_b, ids_a, ids_b,
                                          size_t(n_nodes), 0u, 64u, st));
  hipLaunchKernelGGL(k_rel_select, dim3(grid_for(n_nodes)), dim3(kBlock), 0, st, ids_b,
                     topk_percent, member, out_len);
  NGT_HIP_CHECK(hipGetLastError());
  tb = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::exclusive_scan(ws + L.temp, tb, member, pos, int32_t(0), size_t(n_nodes),
                                        rocprim::plus<int32_t>(), st));
  hipLaunchKernelGGL(k_rel_emit, dim3(grid_for(n_nodes)), dim3(kBlock), 0, st, n_nodes, member,
                     pos, out, out_len);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_gather_rows(const void* src, int64_t n_src, const int64_t* idx, int64_t n_rows,
                               int64_t row_bytes, void* dst, int32_t* bad, void* stream) {
  if (n_rows < 0 || n_src < 0 || row_bytes < 0 || row_bytes % 4)
    return set_error(NGT_ERR_ARG, "ngt_gather_rows: bad sizes (row_bytes must be a multiple of 4)");
  if (n_rows == 0 || row_bytes == 0) return NGT_OK;
  if (!src || !idx || !dst) return set_error(NGT_ERR_ARG, "ngt_gather_rows: null pointer");
  const int64_t words = row_bytes / 4;
  hipLaunchKernelGGL(k_gather_rows, dim3(grid_for(n_rows * words)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(src), n_src,
                     idx, n_rows, words, static_cast<uint32_t*>(dst), bad);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_segment_sum_f32(const float* vals, int64_t n_vals, const int64_t* seg,
                                   int64_t n_seg, float* out, int32_t* bad, void* stream) {
  if (n_vals < 0 || n_seg < 0 || (n_seg > 0 && (!seg || !out || !bad)) || (n_vals > 0 && !vals))
    return set_error(NGT_ERR_ARG, "ngt_segment_sum_f32: bad arguments");
  if (n_seg == 0) return NGT_OK;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  KernelTimer timer_("segment_sum", st);
  hipLaunchKernelGGL(k_segment_sum, dim3((n_seg + kBlock - 1) / kBlock),
                     dim3(kBlock), 0, st, vals, n_vals, seg, n_seg, out, bad);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}
