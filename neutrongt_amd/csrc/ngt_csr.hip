// Window adjacency construction: COO edge_index -> query-major CSR,
// key-major (transposed) CSR, the position map between them and the
// degree-binned work lists the attention kernels are scheduled from:
//   rows with more than `chunk` edges -> chunks of `chunk` edges (listed first),
//   rows with small < degree <= chunk -> one work item per row, longest first,
//   rows with degree <= small         -> packed list, longest first; the
//                                        kernels give each such row one edge
//                                        slot (several rows per wave);
// and, when asked for, the rows longest first (the tiled kernels' order): all
// query rows, and the key rows j < min(n_q, n_k) (the window's own nodes).
//
// The reference keeps the window mask as a COO edge_index
// (NeutronGT/core/node_level_pipeline/window_state.py:122-140) and consumes it
// with gathers and torch_scatter adds
// (NeutronGT/models/graphormer_dist_node_level.py:75-97).  Here the ordering is
// made canonical: query-major rows are sorted by (dst, src, edge id) and
// key-major rows by (src, dst, edge id), so the CSR is a pure function of the
// edge list (bit-exact, independent of launch shapes).  The sort is rocPRIM's
// LSD radix sort, which is stable, so duplicate edges keep edge-id order.
#include "ngt_common.h"

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

namespace ngt {
namespace {

constexpr int kBlock = 256;

struct Count3 {
  int32_t split_items;  // chunks of rows longer than `chunk`
  int32_t plain_items;  // rows that fit one item
  int32_t split_rows;
};

struct Count3Plus {
  __host__ __device__ Count3 operator()(const Count3& a, const Count3& b) const {
    return Count3{a.split_items + b.split_items, a.plain_items + b.plain_items,
                  a.split_rows + b.split_rows};
  }
};

inline unsigned bits_for(uint64_t v) {
  unsigned b = 0;
  while (b < 64 && (v >> b) != 0) ++b;
  return b == 0 ? 1 : b;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__global__ void k_make_keys(const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
                            int64_t E, int32_t n_q, int32_t n_k, uint64_t* __restrict__ key_q,
                            uint64_t* __restrict__ key_k, int32_t* __restrict__ eid,
                            int32_t* __restrict__ info) {
  const uint64_t sentinel = uint64_t(n_q) * uint64_t(n_k);
  for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < E;
       e += int64_t(gridDim.x) * blockDim.x) {
    const int64_t s = src[e];
    const int64_t d = dst[e];
    const bool ok = s >= 0 && s < n_k && d >= 0 && d < n_q;
    if (ok) {
      key_q[e] = uint64_t(d) * uint64_t(n_k) + uint64_t(s);
      key_k[e] = uint64_t(s) * uint64_t(n_q) + uint64_t(d);
    } else {
      key_q[e] = sentinel;
      key_k[e] = sentinel;
      atomicAdd(info + NGT_INFO_BAD_EDGES, 1);
    }
    eid[e] = static_cast<int32_t>(e);
  }
}

// rowptr[r] = first sorted position whose row >= r; col = key % n_cols.
// Sentinel keys (dropped edges) map to row n_rows and therefore sit past
// rowptr[n_rows].
__global__ void k_rowptr(const uint64_t* __restrict__ keys, int64_t E, uint64_t n_cols,
                         int32_t n_rows, int32_t* __restrict__ rowptr,
                         int32_t* __restrict__ col) {
  for (int64_t p = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; p <= E;
       p += int64_t(gridDim.x) * blockDim.x) {
    int64_t r_cur = n_rows;
    if (p < E) {
      const uint64_t r = keys[p] / n_cols;
      r_cur = r < uint64_t(n_rows) ? int64_t(r) : int64_t(n_rows);
      col[p] = r_cur < n_rows ? static_cast<int32_t>(keys[p] % n_cols) : 0;
    }
    int64_t r_prev = -1;
    if (p > 0) {
      const uint64_t r = keys[p - 1] / n_cols;
      r_prev = r < uint64_t(n_rows) ? int64_t(r) : int64_t(n_rows);
    }
    for (int64_t r = r_prev + 1; r <= r_cur; ++r) rowptr[r] = static_cast<int32_t>(p);
  }
}

__global__ void k_scatter_pos(const int32_t* __restrict__ perm, int64_t E,
                              int32_t* __restrict__ pos_of_eid) {
  for (int64_t p = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; p < E;
       p += int64_t(gridDim.x) * blockDim.x)
    pos_of_eid[perm[p]] = static_cast<int32_t>(p);
}

__global__ void k_compose(const int32_t* __restrict__ perm, const int32_t* __restrict__ tpos_of_eid,
                          int64_t E, int32_t* __restrict__ q2t) {
  for (int64_t p = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; p < E;
       p += int64_t(gridDim.x) * blockDim.x)
    q2t[p] = tpos_of_eid[perm[p]];
}

__device__ __forceinline__ Count3 row_counts(int32_t deg, int32_t chunk) {
  if (deg > chunk) return Count3{(deg + chunk - 1) / chunk, 0, 1};
  return Count3{0, 1, 0};
}

// Per row: chunk counts for the scan, and (degree, row) pairs for the sort.
__global__ void k_count(const int32_t* __restrict__ rowptr, int32_t n_rows, int32_t chunk,
                        Count3* __restrict__ cnt, uint32_t* __restrict__ deg_key,
                        int32_t* __restrict__ row_val, int32_t* __restrict__ info,
                        int max_deg_slot) {
  int32_t local_max = 0;
  for (int32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < n_rows; r += gridDim.x * blockDim.x) {
    const int32_t deg = rowptr[r + 1] - rowptr[r];
    cnt[r] = row_counts(deg, chunk);
    deg_key[r] = static_cast<uint32_t>(deg);
    row_val[r] = r;
    local_max = max(local_max, deg);
  }
  if (local_max > 0) atomicMax(info + max_deg_slot, local_max);
}

// Chunks of the rows longer than `chunk` (row order) and the split table.
__global__ void k_emit_split(const int32_t* __restrict__ rowptr, int32_t n_rows, int32_t chunk,
                             const Count3* __restrict__ scan, int4* __restrict__ items,
                             int4* __restrict__ splits) {
  for (int32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < n_rows; r += gridDim.x * blockDim.x) {
    const int32_t beg = rowptr[r];
    const int32_t end = rowptr[r + 1];
    if (end - beg <= chunk) continue;
    const Count3 pre = scan[r];
    const int32_t n = (end - beg + chunk - 1) / chunk;
    for (int32_t c = 0; c < n; ++c) {
      const int32_t b = beg + c * chunk;
      const int32_t slot = pre.split_items + c;
      items[slot] = make_int4(r, b, min(end, b + chunk), slot);
    }
    splits[pre.split_rows] = make_int4(r, pre.split_items, n, 0);
  }
}

// First index in sorted[0, n) whose value exceeds x.
__device__ __forceinline__ int32_t upper_bound_u32(const uint32_t* __restrict__ sorted, int32_t n,
                                                   uint32_t x) {
  int32_t lo = 0, hi = n;
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (sorted[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Packing threshold read from the degrees (small = NGT_SMALL_FROM_DEGREES):
// the first step that packs at least kPackSharePct % of the rows.
constexpr int32_t kPackSteps[4] = {8, 16, 24, 32};
constexpr int64_t kPackSharePct = 78;

__device__ __forceinline__ int32_t packing_threshold(const uint32_t* __restrict__ sdeg,
                                                     int32_t n_rows, int32_t chunk) {
  int32_t t = 0;
  for (int i = 0; i < 4; ++i) {
    t = min(kPackSteps[i], chunk - 1);
    const int32_t packed = upper_bound_u32(sdeg, n_rows, static_cast<uint32_t>(t));
    if (int64_t(packed) * 100 >= int64_t(n_rows) * kPackSharePct) break;
  }
  return t;
}

// From the rows sorted by ascending degree: the packed small rows and the
// single-item medium rows, both longest first.  info gets the totals and the
// packing threshold used.
__global__ void k_emit_sorted(const int32_t* __restrict__ rowptr, int32_t n_rows, int32_t chunk,
                              int32_t small_in, const uint32_t* __restrict__ sdeg,
                              const int32_t* __restrict__ srow, const Count3* __restrict__ scan,
                              int4* __restrict__ items, int32_t* __restrict__ packed,
                              int32_t* __restrict__ order, int32_t* __restrict__ info,
                              int info_base, int packed_slot, int small_slot) {
  const int32_t small = small_in < 0 ? packing_threshold(sdeg, n_rows, chunk) : small_in;
  const int32_t n_small = upper_bound_u32(sdeg, n_rows, static_cast<uint32_t>(small));
  const int32_t n_le_chunk = upper_bound_u32(sdeg, n_rows, static_cast<uint32_t>(chunk));
  const int32_t n_medium = n_le_chunk - n_small;
  Count3 tot{0, 0, 0};
  if (n_rows > 0) {
    const Count3 last = scan[n_rows - 1];
    const Count3 own = row_counts(rowptr[n_rows] - rowptr[n_rows - 1], chunk);
    tot = Count3{last.split_items + own.split_items, last.plain_items + own.plain_items,
                 last.split_rows + own.split_rows};
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    info[info_base + 0] = tot.split_items + n_medium;  // work items
    info[info_base + 1] = tot.split_items;             // partial slots
    info[info_base + 2] = tot.split_rows;              // split rows
    info[packed_slot] = n_small;                       // packed rows
    info[small_slot] = small;                          // their threshold
  }
  for (int32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < n_le_chunk;
       p += gridDim.x * blockDim.x) {
    const int32_t r = srow[p];
    if (p < n_small) {
      packed[n_small - 1 - p] = r;
    } else {
      items[tot.split_items + (n_le_chunk - 1 - p)] = make_int4(r, rowptr[r], rowptr[r + 1], -1);
    }
  }
  // every row, longest first (when the order covers all rows)
  if (order)
    for (int32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < n_rows;
         p += gridDim.x * blockDim.x)
      order[n_rows - 1 - p] = srow[p];
}

// order[n - 1 - p] = srow[p]: rows sorted by ascending degree, reversed.
__global__ void k_emit_order(const int32_t* __restrict__ srow, int32_t n,
                             int32_t* __restrict__ order) {
  for (int32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < n; p += gridDim.x * blockDim.x)
    order[n - 1 - p] = srow[p];
}

__global__ void k_ends(const uint64_t* __restrict__ key_q, const uint64_t* __restrict__ key_k,
                       const int32_t* __restrict__ rowptr, int32_t n_q, int32_t n_k,
                       int32_t* __restrict__ info) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const int32_t nv = rowptr[n_q];  // valid edges (dropped ones sort last)
    info[NGT_INFO_DST_END] = nv > 0 ? int32_t(key_q[nv - 1] / uint64_t(n_k)) + 1 : 0;
    info[NGT_INFO_SRC_END] = nv > 0 ? int32_t(key_k[nv - 1] / uint64_t(n_q)) + 1 : 0;
  }
}

__global__ void k_zero(int32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

inline int grid_for(int64_t n) {
  int64_t g = (n + kBlock - 1) / kBlock;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return static_cast<int>(g);
}

struct CsrLayout {
  size_t key_a, key_b, key_c, eid, tpos, cnt, cnt_scan, deg_a, deg_b, row_a, row_b, deg_c, row_c,
      temp, total;
  size_t temp_bytes;
};

int csr_layout(int64_t E, int32_t n_q, int32_t n_k, CsrLayout* L) {
  const int64_t n_rows = n_q > n_k ? n_q : n_k;
  size_t sort_bytes = 0, scan_bytes = 0;
  const size_t n = static_cast<size_t>(E > 0 ? E : 1);
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, sort_bytes, (uint64_t*)nullptr,
                                          (uint64_t*)nullptr, (int32_t*)nullptr,
                                          (int32_t*)nullptr, n, 0u, 64u, hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan_bytes, (Count3*)nullptr, (Count3*)nullptr,
                                        Count3{0, 0, 0}, size_t(n_rows > 0 ? n_rows : 1),
                                        Count3Plus(), hipStream_t(0)));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  };
  L->key_a = take(n * 8);
  L->key_b = take(n * 8);
  L->key_c = take(n * 8);
  L->eid = take(n * 4);
  L->tpos = take(n * 4);
  L->cnt = take(size_t(n_rows + 1) * sizeof(Count3));
  L->cnt_scan = take(size_t(n_rows + 1) * sizeof(Count3));
  L->deg_a = take(size_t(n_rows + 1) * 4);
  L->deg_b = take(size_t(n_rows + 1) * 4);
  L->row_a = take(size_t(n_rows + 1) * 4);
  L->row_b = take(size_t(n_rows + 1) * 4);
  L->deg_c = take(size_t(n_rows + 1) * 4);
  L->row_c = take(size_t(n_rows + 1) * 4);
  size_t deg_sort_bytes = 0;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, deg_sort_bytes, (uint32_t*)nullptr,
                                          (uint32_t*)nullptr, (int32_t*)nullptr,
                                          (int32_t*)nullptr, size_t(n_rows > 0 ? n_rows : 1),
                                          0u, 32u, hipStream_t(0)));
  L->temp_bytes = sort_bytes > scan_bytes ? sort_bytes : scan_bytes;
  if (deg_sort_bytes > L->temp_bytes) L->temp_bytes = deg_sort_bytes;
  L->temp = take(L->temp_bytes);
  L->total = off;
  return NGT_OK;
}

// order (optional): the first n_order rows (all rows when n_order == n_rows),
// longest first.
int build_worklist(const int32_t* rowptr, int32_t n_rows, int32_t chunk, int32_t small,
                   int4* items, int4* splits, int32_t* packed, int32_t* order, int32_t n_order,
                   int32_t* info, int info_base,
                   int packed_slot, int small_slot, int max_deg_slot, char* ws,
                   const CsrLayout& L, hipStream_t st) {
  Count3* cnt = reinterpret_cast<Count3*>(ws + L.cnt);
  Count3* scan = reinterpret_cast<Count3*>(ws + L.cnt_scan);
  uint32_t* deg_a = reinterpret_cast<uint32_t*>(ws + L.deg_a);
  uint32_t* deg_b = reinterpret_cast<uint32_t*>(ws + L.deg_b);
  int32_t* row_a = reinterpret_cast<int32_t*>(ws + L.row_a);
  int32_t* row_b = reinterpret_cast<int32_t*>(ws + L.row_b);
  if (n_rows == 0) {
    hipLaunchKernelGGL(k_emit_sorted, dim3(1), dim3(kBlock), 0, st, rowptr, n_rows, chunk, small,
                       deg_b, row_b, scan, items, packed, order, info, info_base, packed_slot,
                       small_slot);
    NGT_HIP_CHECK(hipGetLastError());
    return NGT_OK;
  }
  hipLaunchKernelGGL(k_count, dim3(grid_for(n_rows)), dim3(kBlock), 0, st, rowptr, n_rows, chunk,
                     cnt, deg_a, row_a, info, max_deg_slot);
  NGT_HIP_CHECK(hipGetLastError());
  size_t temp_bytes = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::exclusive_scan(ws + L.temp, temp_bytes, cnt, scan, Count3{0, 0, 0},
                                        size_t(n_rows), Count3Plus(), st));
  hipLaunchKernelGGL(k_emit_split, dim3(grid_for(n_rows)), dim3(kBlock), 0, st, rowptr, n_rows,
                     chunk, scan, items, splits);
  NGT_HIP_CHECK(hipGetLastError());
  temp_bytes = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(ws + L.temp, temp_bytes, deg_a, deg_b, row_a, row_b,
                                          size_t(n_rows), 0u, 32u, st));
  const bool full_order = order && n_order >= n_rows;
  hipLaunchKernelGGL(k_emit_sorted, dim3(grid_for(n_rows)), dim3(kBlock), 0, st, rowptr, n_rows,
                     chunk, small, deg_b, row_b, scan, items, packed,
                     full_order ? order : nullptr, info, info_base, packed_slot, small_slot);
  NGT_HIP_CHECK(hipGetLastError());
  if (order && !full_order && n_order > 0) {
    // the leading rows alone: (degree, row) of rows [0, n_order) are the
    // first n_order entries of deg_a / row_a (row order)
    uint32_t* deg_c = reinterpret_cast<uint32_t*>(ws + L.deg_c);
    int32_t* row_c = reinterpret_cast<int32_t*>(ws + L.row_c);
    temp_bytes = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::radix_sort_pairs(ws + L.temp, temp_bytes, deg_a, deg_c, row_a, row_c,
                                            size_t(n_order), 0u, 32u, st));
    hipLaunchKernelGGL(k_emit_order, dim3(grid_for(n_order)), dim3(kBlock), 0, st, row_c, n_order,
                       order);
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_csr_sizes(int64_t n_edges, int32_t n_q, int32_t n_k, int32_t chunk_q,
                             int32_t chunk_k, int32_t* max_items_q, int32_t* max_splits_q,
                             int32_t* max_items_k, int32_t* max_splits_k) {
  if (n_edges < 0 || n_q < 0 || n_k < 0 || chunk_q <= 0 || chunk_k <= 0)
    return set_error(NGT_ERR_ARG, "ngt_csr_sizes: negative size or non-positive chunk");
  if (n_edges >= (int64_t(1) << 31) - 1)
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_csr_sizes: %lld edges exceed int32 indexing",
                     (long long)n_edges);
  const int64_t cq = (n_edges + chunk_q - 1) / chunk_q;
  const int64_t ck = (n_edges + chunk_k - 1) / chunk_k;
  const int64_t iq = int64_t(n_q) + 2 * cq + 1;
  const int64_t ik = int64_t(n_k) + 2 * ck + 1;
  if (iq >= (int64_t(1) << 31) || ik >= (int64_t(1) << 31))
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_csr_sizes: work list exceeds int32");
  if (max_items_q) *max_items_q = int32_t(iq);
  if (max_items_k) *max_items_k = int32_t(ik);
  if (max_splits_q) *max_splits_q = int32_t((cq < n_q ? cq : n_q) + 1);
  if (max_splits_k) *max_splits_k = int32_t((ck < n_k ? ck : n_k) + 1);
  return NGT_OK;
}

extern "C" int ngt_csr_workspace_bytes(int64_t n_edges, int32_t n_q, int32_t n_k, size_t* bytes) {
  if (!bytes) return set_error(NGT_ERR_ARG, "ngt_csr_workspace_bytes: null output");
  CsrLayout L;
  const int rc = csr_layout(n_edges, n_q, n_k, &L);
  if (rc != NGT_OK) return rc;
  *bytes = L.total;
  return NGT_OK;
}

extern "C" int ngt_csr_build(const int64_t* edge_index, ngt_window_csr* csr, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (!csr) return set_error(NGT_ERR_ARG, "ngt_csr_build: null csr");
  const int64_t E = csr->n_edges;
  const int32_t n_q = csr->n_q, n_k = csr->n_k;
  if (E < 0 || n_q < 0 || n_k < 0 || csr->chunk_q <= 0 || csr->chunk_k <= 0 ||
      csr->small_q < NGT_SMALL_FROM_DEGREES || csr->small_k < NGT_SMALL_FROM_DEGREES ||
      csr->small_q >= csr->chunk_q || csr->small_k >= csr->chunk_k)
    return set_error(NGT_ERR_ARG,
                     "ngt_csr_build: bad sizes (need 0 <= small < chunk, or small = "
                     "NGT_SMALL_FROM_DEGREES)");
  if (E > 0 && (!edge_index || n_q == 0 || n_k == 0))
    return set_error(NGT_ERR_ARG, "ngt_csr_build: edges given for an empty window");
  if (!csr->rowptr || !csr->t_rowptr || !csr->info || !csr->items_q || !csr->items_k ||
      !csr->splits_q || !csr->splits_k || (n_q > 0 && !csr->packed_q) ||
      (n_k > 0 && !csr->packed_k) || (E > 0 && (!csr->col || !csr->perm || !csr->t_col ||
                                                     !csr->t_perm || !csr->q2t)))
    return set_error(NGT_ERR_ARG, "ngt_csr_build: null output array");
  int32_t miq, msq, mik, msk;
  int rc = ngt_csr_sizes(E, n_q, n_k, csr->chunk_q, csr->chunk_k, &miq, &msq, &mik, &msk);
  if (rc != NGT_OK) return rc;
  if (csr->max_items_q < miq || csr->max_items_k < mik || csr->max_splits_q < msq ||
      csr->max_splits_k < msk)
    return set_error(NGT_ERR_ARG, "ngt_csr_build: work-list arrays smaller than ngt_csr_sizes");
  CsrLayout L;
  rc = csr_layout(E, n_q, n_k, &L);
  if (rc != NGT_OK) return rc;
  if (!workspace || workspace_bytes < L.total)
    return set_error(NGT_ERR_WORKSPACE, "ngt_csr_build: workspace %zu < %zu bytes",
                     workspace_bytes, L.total);

  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  uint64_t* key_a = reinterpret_cast<uint64_t*>(ws + L.key_a);
  uint64_t* key_b = reinterpret_cast<uint64_t*>(ws + L.key_b);
  uint64_t* key_c = reinterpret_cast<uint64_t*>(ws + L.key_c);
  int32_t* eid = reinterpret_cast<int32_t*>(ws + L.eid);
  int32_t* tpos = reinterpret_cast<int32_t*>(ws + L.tpos);

  hipLaunchKernelGGL(k_zero, dim3(1), dim3(64), 0, st, csr->info, NGT_INFO_LEN);
  NGT_HIP_CHECK(hipGetLastError());
  const uint64_t sentinel = uint64_t(n_q) * uint64_t(n_k);
  const unsigned end_bit = bits_for(sentinel);
  if (E > 0) {
    // key_a <- query-major keys, key_c <- key-major keys.
    hipLaunchKernelGGL(k_make_keys, dim3(grid_for(E)), dim3(kBlock), 0, st, edge_index,
                       edge_index + E, E, n_q, n_k, key_a, key_c, eid, csr->info);
    NGT_HIP_CHECK(hipGetLastError());
    size_t tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::radix_sort_pairs(ws + L.temp, tb, key_a, key_b, eid, csr->perm,
                                            size_t(E), 0u, end_bit, st));
    tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::radix_sort_pairs(ws + L.temp, tb, key_c, key_a, eid, csr->t_perm,
                                            size_t(E), 0u, end_bit, st));
    // Sorted: key_b = query-major keys, key_a = key-major keys.
  }
  hipLaunchKernelGGL(k_rowptr, dim3(grid_for(E + 1)), dim3(kBlock), 0, st, key_b, E,
                     uint64_t(n_k > 0 ? n_k : 1), n_q, csr->rowptr, csr->col);
  NGT_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(k_rowptr, dim3(grid_for(E + 1)), dim3(kBlock), 0, st, key_a, E,
                     uint64_t(n_q > 0 ? n_q : 1), n_k, csr->t_rowptr, csr->t_col);
  NGT_HIP_CHECK(hipGetLastError());
  if (E > 0) {
    hipLaunchKernelGGL(k_scatter_pos, dim3(grid_for(E)), dim3(kBlock), 0, st, csr->t_perm, E,
                       tpos);
    NGT_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(k_compose, dim3(grid_for(E)), dim3(kBlock), 0, st, csr->perm, tpos, E,
                       csr->q2t);
    NGT_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(k_ends, dim3(1), dim3(64), 0, st, key_b, key_a, csr->rowptr, n_q, n_k,
                       csr->info);
    NGT_HIP_CHECK(hipGetLastError());
  }
  rc = build_worklist(csr->rowptr, n_q, csr->chunk_q, csr->small_q,
                      reinterpret_cast<int4*>(csr->items_q), reinterpret_cast<int4*>(csr->splits_q),
                      csr->packed_q, csr->order_q, n_q, csr->info, NGT_INFO_ITEMS_Q,
                      NGT_INFO_PACKED_Q,
                      NGT_INFO_SMALL_Q, NGT_INFO_MAX_DEG_Q, ws, L, st);
  if (rc != NGT_OK) return rc;
  rc = build_worklist(csr->t_rowptr, n_k, csr->chunk_k, csr->small_k,
                      reinterpret_cast<int4*>(csr->items_k), reinterpret_cast<int4*>(csr->splits_k),
                      csr->packed_k, csr->order_k, n_q < n_k ? n_q : n_k, csr->info,
                      NGT_INFO_ITEMS_K, NGT_INFO_PACKED_K,
                      NGT_INFO_SMALL_K, NGT_INFO_MAX_DEG_K, ws, L, st);
  return rc;
}
