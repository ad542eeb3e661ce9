// Induced window subgraphs on the GPU, in the two orders the reference uses.
//
//  * COO form: torch_geometric.utils.subgraph(subset, edge_index,
//    relabel_nodes=True, num_nodes) as called at
//    NeutronGT/core/node_level_pipeline/window_state.py:82,127 and
//    NeutronGT/core/metisPartition.py:280,290.  Edge e is kept iff both of its
//    endpoints are in the subset; kept edges stay in global edge order; every
//    node is relabelled to its position in the subset.
//  * CSR form: _subgraph_from_csr (window_state.py:92-119).  For each node of
//    the set, in set order, its CSR neighbours in CSR order that are in the
//    set; row 0 = the row node's position, row 1 = the neighbour's position.
//
// Positions come from a map pos[n_nodes] (-1 = outside) scattered from the
// set.  A duplicate or out-of-range set entry is an error here (the
// reference's relabel map would keep an arbitrary one of the duplicates), and
// so is an edge endpoint outside [0, n_nodes).
//
// Output is compacted in order: a count pass per tile (COO: 2,048 consecutive
// edges per block; CSR: one wave per set node), an inclusive scan of the
// counts, then an emit pass that recomputes the flags and writes each kept
// edge at its tile's start + its rank inside the tile (wave ballots, mbcnt,
// and the per-wave totals in LDS).  Reads are coalesced runs of the edge list
// or CSR rows plus random 4-byte reads of pos; the work is HBM-bound.
#include "ngt_common.h"

#include <rocprim/device/device_scan.hpp>

namespace ngt {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kRounds = 8;
constexpr int64_t kTile = int64_t(kBlock) * kRounds;

// result[1] error bits
constexpr unsigned long long kBadSetNode = 1, kDuplicateSetNode = 2, kBadEdge = 4, kBadRowptr = 8;

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct SubLayout {
  size_t pos, cnt, end, nseg, seg_end, temp, temp_bytes, total;
};

// n_items: scan length (COO tiles or CSR segment waves); n_set: set size
int sub_layout(int64_t n_nodes, int64_t n_items, int64_t n_set, SubLayout* L) {
  const size_t n = size_t(n_nodes > 0 ? n_nodes : 1);
  if (n_set > n_items) n_items = n_set;
  const size_t m = size_t(n_items > 0 ? n_items : 1);
  const size_t ns = size_t(n_set > 0 ? n_set : 1);
  size_t scan_bytes = 0;
  NGT_HIP_CHECK(rocprim::inclusive_scan(nullptr, scan_bytes, (int64_t*)nullptr, (int64_t*)nullptr,
                                        m, rocprim::plus<int64_t>(), hipStream_t(0)));
  size_t off = 0;
  auto take = [&](size_t b) {
    const size_t at = off;
    off += align256(b);
    return at;
  };
  L->pos = take(n * 4);
  L->cnt = take(m * 8);
  L->end = take(m * 8);
  L->nseg = take(ns * 8);
  L->seg_end = take(ns * 8);
  L->temp_bytes = scan_bytes;
  L->temp = take(scan_bytes);
  L->total = off;
  return NGT_OK;
}

__device__ __forceinline__ uint32_t lane_rank(unsigned long long mask) {
  return __builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0u));
}

__global__ void k_sub_init(int64_t n_nodes, int32_t* pos, unsigned long long* result) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n_nodes; i += stride)
    pos[i] = -1;
  if (blockIdx.x == 0 && threadIdx.x < 2) result[threadIdx.x] = 0;
}

__global__ void k_sub_mark(const int64_t* set, int32_t n_set, int64_t n_nodes, int32_t* pos,
                           unsigned long long* result) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n_set) return;
  const int64_t g = set[i];
  if (g < 0 || g >= n_nodes) {
    atomicOr(&result[1], kBadSetNode);
    return;
  }
  if (atomicCAS(&pos[g], -1, int32_t(i)) != -1) atomicOr(&result[1], kDuplicateSetNode);
}

// ------------------------------------------------------------------ COO form
__device__ __forceinline__ bool coo_flag(const int64_t* src, const int64_t* dst, int64_t e,
                                         int64_t n_nodes, const int32_t* pos, int32_t& ps,
                                         int32_t& pd, bool& bad) {
  const int64_t s = src[e], d = dst[e];
  if (s < 0 || s >= n_nodes || d < 0 || d >= n_nodes) {
    bad = true;
    return false;
  }
  ps = pos[s];
  if (ps < 0) return false;  // most edges leave here: no random read of pos[d]
  pd = pos[d];
  return pd >= 0;
}

__global__ __launch_bounds__(kBlock) void k_coo_count(const int64_t* ei, int64_t n_edges,
                                                      int64_t n_nodes, const int32_t* pos,
                                                      int64_t* cnt, unsigned long long* result) {
  __shared__ int wave_cnt[kWaves];
  const int64_t base = blockIdx.x * kTile;
  int c = 0;
  bool bad = false;
  for (int r = 0; r < kRounds; ++r) {
    const int64_t e = base + int64_t(r) * kBlock + threadIdx.x;
    int32_t ps, pd;
    if (e < n_edges && coo_flag(ei, ei + n_edges, e, n_nodes, pos, ps, pd, bad)) ++c;
  }
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
  if ((threadIdx.x & 63) == 0) wave_cnt[threadIdx.x >> 6] = c;
  if (bad) atomicOr(&result[1], kBadEdge);
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < kWaves; ++w) t += wave_cnt[w];
    cnt[blockIdx.x] = t;
  }
}

__global__ __launch_bounds__(kBlock) void k_coo_emit(const int64_t* ei, int64_t n_edges,
                                                     int64_t n_nodes, const int32_t* pos,
                                                     const int64_t* cnt, const int64_t* end,
                                                     int64_t* out, int64_t cap) {
  __shared__ int wave_tot[2][kWaves];
  const int wave = threadIdx.x >> 6;
  const int64_t base = blockIdx.x * kTile;
  int64_t at = end[blockIdx.x] - cnt[blockIdx.x];
  for (int r = 0; r < kRounds; ++r) {
    const int64_t e = base + int64_t(r) * kBlock + threadIdx.x;
    int32_t ps = 0, pd = 0;
    bool bad = false;
    const bool keep = e < n_edges && coo_flag(ei, ei + n_edges, e, n_nodes, pos, ps, pd, bad);
    const unsigned long long m = __ballot(keep);
    if ((threadIdx.x & 63) == 0) wave_tot[r & 1][wave] = __popcll(m);
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < kWaves; ++w) {
      const int t = wave_tot[r & 1][w];
      before += w < wave ? t : 0;
      total += t;
    }
    if (keep) {
      const int64_t k = at + before + lane_rank(m);
      if (k < cap) {
        out[k] = ps;
        out[cap + k] = pd;
      }
    }
    at += total;
  }
}

// ------------------------------------------------------------------ CSR form
// A set node's CSR row is cut into segments of kSeg entries, one wave each, so
// a hub row (hundreds of thousands of neighbours) is spread over many waves.
// Segments are numbered in (set order, position in row) order, which is the
// output order; a wave finds its segment by binary search over the inclusive
// scan of the per-node segment counts.
constexpr int64_t kSeg = 2048;

__global__ void k_csr_segs(const int64_t* rowptr, int64_t n_col, int64_t n_nodes,
                           const int64_t* set, int32_t n_set, int64_t* nseg,
                           unsigned long long* result) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n_set) return;
  const int64_t g = set[i];
  int64_t ns = 0;
  if (g >= 0 && g < n_nodes) {  // a bad set node is flagged by k_sub_mark
    const int64_t b = rowptr[g], e = rowptr[g + 1];
    if (b < 0 || e < b || e > n_col)
      atomicOr(&result[1], kBadRowptr);
    else
      ns = (e - b + kSeg - 1) / kSeg;
  }
  nseg[i] = ns;
}

struct Segment {
  int64_t row, b, e;  // set position; CSR range [b, e)
};

__device__ __forceinline__ bool find_segment(int64_t w, const int64_t* seg_end, const int64_t* nseg,
                                             int32_t n_set, const int64_t* rowptr,
                                             const int64_t* set, Segment& sg) {
  if (n_set == 0 || w >= seg_end[n_set - 1]) return false;
  int lo = 0, hi = n_set - 1;  // first i with seg_end[i] > w
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (seg_end[mid] > w)
      hi = mid;
    else
      lo = mid + 1;
  }
  const int64_t k = w - (seg_end[lo] - nseg[lo]);
  const int64_t g = set[lo];
  const int64_t e0 = rowptr[g + 1];
  sg.row = lo;
  sg.b = rowptr[g] + k * kSeg;
  sg.e = sg.b + kSeg < e0 ? sg.b + kSeg : e0;
  return true;
}

__global__ __launch_bounds__(kBlock) void k_csr_count(const int64_t* rowptr, const int64_t* col,
                                                      int64_t n_nodes, const int64_t* set,
                                                      int32_t n_set, const int64_t* nseg,
                                                      const int64_t* seg_end, int64_t n_waves,
                                                      const int32_t* pos, int64_t* cnt,
                                                      unsigned long long* result) {
  const int64_t w = blockIdx.x * int64_t(kWaves) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w >= n_waves) return;
  // rows that overlap (a non-monotone rowptr) could need more segments than
  // the launch covers: refuse rather than drop edges
  if (w == 0 && lane == 0 && n_set > 0 && seg_end[n_set - 1] > n_waves)
    atomicOr(&result[1], kBadRowptr);
  Segment sg;
  if (!find_segment(w, seg_end, nseg, n_set, rowptr, set, sg)) {
    if (lane == 0) cnt[w] = 0;
    return;
  }
  int64_t c = 0;
  bool bad = false;
  for (int64_t p0 = sg.b; p0 < sg.e; p0 += 64) {
    const int64_t p = p0 + lane;
    bool keep = false;
    if (p < sg.e) {
      const int64_t nb = col[p];
      if (nb < 0 || nb >= n_nodes)
        bad = true;
      else
        keep = pos[nb] >= 0;
    }
    c += __popcll(__ballot(keep));
  }
  if (bad) atomicOr(&result[1], kBadEdge);
  if (lane == 0) cnt[w] = c;
}

__global__ __launch_bounds__(kBlock) void k_csr_emit(const int64_t* rowptr, const int64_t* col,
                                                     int64_t n_nodes, const int64_t* set,
                                                     int32_t n_set, const int64_t* nseg,
                                                     const int64_t* seg_end, int64_t n_waves,
                                                     const int32_t* pos, const int64_t* cnt,
                                                     const int64_t* end, int64_t* out,
                                                     int64_t cap) {
  const int64_t w = blockIdx.x * int64_t(kWaves) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w >= n_waves) return;
  Segment sg;
  if (!find_segment(w, seg_end, nseg, n_set, rowptr, set, sg)) return;
  int64_t at = end[w] - cnt[w];
  for (int64_t p0 = sg.b; p0 < sg.e; p0 += 64) {
    const int64_t p = p0 + lane;
    int32_t pn = -1;
    if (p < sg.e) {
      const int64_t nb = col[p];
      if (nb >= 0 && nb < n_nodes) pn = pos[nb];
    }
    const bool keep = pn >= 0;
    const unsigned long long m = __ballot(keep);
    if (keep) {
      const int64_t k = at + lane_rank(m);
      if (k < cap) {
        out[k] = sg.row;
        out[cap + k] = pn;
      }
    }
    at += __popcll(m);
  }
}

__global__ void k_sub_total(const int64_t* end, int64_t n_items, unsigned long long* result) {
  if (threadIdx.x == 0 && blockIdx.x == 0)
    result[0] = n_items > 0 ? (unsigned long long)end[n_items - 1] : 0ull;
}

inline int grid_for(int64_t n) {
  int64_t g = (n + kBlock - 1) / kBlock;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return int(g);
}

int sub_prepare(int64_t n_nodes, int64_t n_items, const int64_t* set, int32_t n_set, void* ws,
                size_t ws_bytes, hipStream_t s, int64_t* result, SubLayout* L, const char* who) {
  NGT_CHECK_OK(sub_layout(n_nodes, n_items, n_set, L));
  if (!ws || ws_bytes < L->total)
    return set_error(NGT_ERR_ARG, "%s: workspace too small (%zu < %zu)", who, ws_bytes, L->total);
  char* base = static_cast<char*>(ws);
  int32_t* pos = reinterpret_cast<int32_t*>(base + L->pos);
  auto* res = reinterpret_cast<unsigned long long*>(result);
  hipLaunchKernelGGL(k_sub_init, dim3(grid_for(n_nodes)), dim3(kBlock), 0, s, n_nodes, pos, res);
  if (n_set > 0)
    hipLaunchKernelGGL(k_sub_mark, dim3((n_set + kBlock - 1) / kBlock), dim3(kBlock), 0, s, set,
                       n_set, n_nodes, pos, res);
  return NGT_OK;
}

int sub_scan(const SubLayout& L, char* base, int64_t n_items, int64_t* result, hipStream_t s) {
  if (n_items <= 0) return NGT_OK;
  size_t temp_bytes = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::inclusive_scan(base + L.temp, temp_bytes,
                                        reinterpret_cast<int64_t*>(base + L.cnt),
                                        reinterpret_cast<int64_t*>(base + L.end), size_t(n_items),
                                        rocprim::plus<int64_t>(), s));
  hipLaunchKernelGGL(k_sub_total, dim3(1), dim3(64), 0, s,
                     reinterpret_cast<const int64_t*>(base + L.end), n_items,
                     reinterpret_cast<unsigned long long*>(result));
  return NGT_OK;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_subgraph_workspace_bytes(int64_t n_nodes, int64_t n_edges, int32_t n_set,
                                            size_t* bytes) {
  if (!bytes || n_nodes < 0 || n_edges < 0 || n_set < 0)
    return set_error(NGT_ERR_ARG, "ngt_subgraph_workspace_bytes: bad arguments");
  // COO form: n_edges edges in 2,048-edge tiles; CSR form: n_edges = entries of
  // col, at most n_set + n_edges / kSeg segment waves
  const int64_t tiles = (n_edges + kTile - 1) / kTile;
  const int64_t segs = int64_t(n_set) + (n_edges + kSeg - 1) / kSeg;
  SubLayout L;
  NGT_CHECK_OK(sub_layout(n_nodes, tiles > segs ? tiles : segs, n_set, &L));
  *bytes = L.total;
  return NGT_OK;
}

extern "C" int ngt_subgraph_coo(const int64_t* edge_index, int64_t n_edges, int64_t n_nodes,
                                const int64_t* subset, int32_t n_subset, int64_t* out, int64_t cap,
                                int64_t* result, void* ws, size_t ws_bytes, void* stream) {
  if (n_edges < 0 || n_nodes < 0 || n_subset < 0 || cap < 0 || !result ||
      (n_edges > 0 && !edge_index) || (n_subset > 0 && !subset))
    return set_error(NGT_ERR_ARG, "ngt_subgraph_coo: bad arguments");
  if (n_subset > n_nodes)
    return set_error(NGT_ERR_ARG, "ngt_subgraph_coo: subset longer than the node count");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tiles = (n_edges + kTile - 1) / kTile;
  SubLayout L;
  NGT_CHECK_OK(sub_prepare(n_nodes, tiles > n_subset ? tiles : n_subset, subset, n_subset, ws,
                           ws_bytes, s, result, &L, "ngt_subgraph_coo"));
  if (tiles == 0) return NGT_OK;
  char* base = static_cast<char*>(ws);
  const int32_t* pos = reinterpret_cast<const int32_t*>(base + L.pos);
  int64_t* cnt = reinterpret_cast<int64_t*>(base + L.cnt);
  const int64_t* end = reinterpret_cast<const int64_t*>(base + L.end);
  auto* res = reinterpret_cast<unsigned long long*>(result);
  KernelTimer timer_("subgraph_coo", s);
  hipLaunchKernelGGL(k_coo_count, dim3(tiles), dim3(kBlock), 0, s, edge_index, n_edges, n_nodes,
                     pos, cnt, res);
  NGT_CHECK_OK(sub_scan(L, base, tiles, result, s));
  if (out && cap > 0)
    hipLaunchKernelGGL(k_coo_emit, dim3(tiles), dim3(kBlock), 0, s, edge_index, n_edges, n_nodes,
                       pos, cnt, end, out, cap);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

extern "C" int ngt_subgraph_csr(const int64_t* rowptr, const int64_t* col, int64_t n_col,
                                int64_t n_nodes, const int64_t* node_set, int32_t n_set,
                                int64_t* out, int64_t cap, int64_t* result, void* ws,
                                size_t ws_bytes, void* stream) {
  if (n_nodes < 0 || n_col < 0 || n_set < 0 || cap < 0 || !result || (n_nodes > 0 && !rowptr) ||
      (n_col > 0 && !col) || (n_set > 0 && !node_set))
    return set_error(NGT_ERR_ARG, "ngt_subgraph_csr: bad arguments");
  if (n_set > n_nodes)
    return set_error(NGT_ERR_ARG, "ngt_subgraph_csr: node set longer than the node count");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_waves = int64_t(n_set) + (n_col + kSeg - 1) / kSeg;
  SubLayout L;
  NGT_CHECK_OK(sub_prepare(n_nodes, n_waves, node_set, n_set, ws, ws_bytes, s, result, &L,
                           "ngt_subgraph_csr"));
  if (n_set == 0) return NGT_OK;
  char* base = static_cast<char*>(ws);
  const int32_t* pos = reinterpret_cast<const int32_t*>(base + L.pos);
  int64_t* cnt = reinterpret_cast<int64_t*>(base + L.cnt);
  const int64_t* end = reinterpret_cast<const int64_t*>(base + L.end);
  int64_t* nseg = reinterpret_cast<int64_t*>(base + L.nseg);
  int64_t* seg_end = reinterpret_cast<int64_t*>(base + L.seg_end);
  auto* res = reinterpret_cast<unsigned long long*>(result);
  KernelTimer timer_("subgraph_csr", s);
  hipLaunchKernelGGL(k_csr_segs, dim3((n_set + kBlock - 1) / kBlock), dim3(kBlock), 0, s, rowptr,
                     n_col, n_nodes, node_set, n_set, nseg, res);
  size_t temp_bytes = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::inclusive_scan(base + L.temp, temp_bytes, nseg, seg_end, size_t(n_set),
                                        rocprim::plus<int64_t>(), s));
  const int64_t grid = (n_waves + kWaves - 1) / kWaves;
  hipLaunchKernelGGL(k_csr_count, dim3(grid), dim3(kBlock), 0, s, rowptr, col, n_nodes, node_set,
                     n_set, nseg, seg_end, n_waves, pos, cnt, res);
  NGT_CHECK_OK(sub_scan(L, base, n_waves, result, s));
  if (out && cap > 0)
    hipLaunchKernelGGL(k_csr_emit, dim3(grid), dim3(kBlock), 0, s, rowptr, col, n_nodes, node_set,
                       n_set, nseg, seg_end, n_waves, pos, cnt, end, out, cap);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}
