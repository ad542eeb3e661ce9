// METIS adjacency with PPR weights on the GPU (build_adj_fromat,
// NeutronGT/core/ppr_preprocess.py:30-71): every PPR entry (src, dst, val) is
// an undirected key (min, max); the values of one key are summed in fp32, the
// weight is int32(clamp_min(sum * 1000, 1)), and both directions of every key
// form a symmetric CSR.
//
// Fixed order: a stable radix sort by key keeps each key's entries in their
// input order, and one lane adds them in that order from 0.0f -- the rounding
// of the reference's scatter_add_ when it runs sequentially (CPU), not an
// atomic order.  Rows are ascending node ids; inside row u the entries of keys
// (u, v > u) come first in ascending v, then those of keys (v < u, u) in
// ascending v (a stable sort of [uu, vv] by node; the reference's argsort is
// unstable there, so its order inside a row is implementation-defined).
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

inline unsigned bits_for(uint64_t v) {
  unsigned b = 1;
  while (b < 64 && (v >> b) != 0) ++b;
  return b;
}

// info[0] = unique keys U, info[1] = bad entries (ids outside [0, n)),
// info[2] = weights that do not fit int32 (sum * 1000 >= 2^31).
__global__ void k_adj_keys(const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
                           int64_t E, int64_t n, uint64_t* __restrict__ key,
                           int32_t* __restrict__ idx, int64_t* __restrict__ info) {
  const int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (e >= E) return;
  const int64_t a = src[e], b = dst[e];
  idx[e] = static_cast<int32_t>(e);
  if (a < 0 || a >= n || b < 0 || b >= n) {
    key[e] = uint64_t(n) * uint64_t(n);  // sorts after every valid key; dropped
    atomicAdd(reinterpret_cast<unsigned long long*>(info + 1), 1ull);
    return;
  }
  const uint64_t u = a < b ? a : b, v = a < b ? b : a;
  key[e] = u * uint64_t(n) + v;
}

// head[s] = 1 where a new valid key starts in the sorted order.
__global__ void k_adj_heads(const uint64_t* __restrict__ key, int64_t E, uint64_t sentinel,
                            int32_t* __restrict__ head) {
  const int64_t s = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (s >= E) return;
  head[s] = key[s] < sentinel && (s == 0 || key[s] != key[s - 1]) ? 1 : 0;
}

// Segment starts of the unique keys, their endpoints, and U (info[0]).
__global__ void k_adj_starts(const uint64_t* __restrict__ key, const int32_t* __restrict__ head,
                             const int32_t* __restrict__ pos, int64_t E, uint64_t sentinel,
                             int64_t n, int32_t* __restrict__ start, int32_t* __restrict__ uu,
                             int32_t* __restrict__ vv, int64_t* __restrict__ info) {
  const int64_t s = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (s >= E) return;
  const bool valid = key[s] < sentinel;
  if (valid && head[s]) {
    const int32_t p = pos[s];
    start[p] = static_cast<int32_t>(s);
    uu[p] = static_cast<int32_t>(key[s] / uint64_t(n));
    vv[p] = static_cast<int32_t>(key[s] % uint64_t(n));
  }
  // the last valid entry closes the last segment
  if (valid && (s + 1 == E || key[s + 1] >= sentinel)) {
    const int32_t u_count = pos[s] + head[s];
    start[u_count] = static_cast<int32_t>(s + 1);
    info[0] = u_count;
  }
}

// One lane per unique key: the values of its entries in input order, from 0.
__global__ void k_adj_weights(const float* __restrict__ val, const int32_t* __restrict__ perm,
                              const int32_t* __restrict__ start, int64_t* info,
                              int32_t* __restrict__ w, int32_t* __restrict__ deg,
                              const int32_t* __restrict__ uu, const int32_t* __restrict__ vv) {
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= info[0]) return;
  float sum = 0.f;
  for (int32_t s = start[t]; s < start[t + 1]; ++s) sum += val[perm[s]];
  float m = sum * 1000.0f;
  m = m < 1.0f ? 1.0f : m;
  int32_t wi = 0;
  if (m < 2147483648.0f) {
    wi = static_cast<int32_t>(m);  // truncation toward zero, as .to(torch.int32)
  } else {
    atomicAdd(reinterpret_cast<unsigned long long*>(info + 2), 1ull);
  }
  w[t] = wi;
  atomicAdd(deg + uu[t], 1);  // integer counts: the order of the adds does not matter
  atomicAdd(deg + vv[t], 1);
}

// Both directions: entry t < U is (uu[t] -> vv[t]), entry U + t is (vv[t] -> uu[t]).
// The sort that follows runs over the 2E bound, so the slots [2U, 2E) get node
// id n (past every real node): they sort after all real entries.
__global__ void k_adj_dir_keys(const int32_t* __restrict__ uu, const int32_t* __restrict__ vv,
                               const int64_t* __restrict__ info, int64_t slots, uint32_t n,
                               uint32_t* __restrict__ node, int32_t* __restrict__ ent) {
  const int64_t U = info[0];
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= slots) return;
  node[t] = t < U ? static_cast<uint32_t>(uu[t]) : t < 2 * U ? static_cast<uint32_t>(vv[t - U]) : n;
  ent[t] = static_cast<int32_t>(t);
}

__global__ void k_adj_emit(const int32_t* __restrict__ ent, const int32_t* __restrict__ uu,
                           const int32_t* __restrict__ vv, const int32_t* __restrict__ w,
                           const int64_t* __restrict__ info, int32_t* __restrict__ adjncy,
                           int32_t* __restrict__ eweights) {
  const int64_t U = info[0];
  const int64_t p = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (p >= 2 * U) return;
  const int32_t t = ent[p];
  const bool fwd = t < U;
  const int32_t k = fwd ? t : static_cast<int32_t>(t - U);
  adjncy[p] = fwd ? vv[k] : uu[k];
  eweights[p] = w[k];
}

__global__ void k_adj_zero(int32_t* __restrict__ p, int64_t n, int64_t* __restrict__ info) {
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i < n) p[i] = 0;
  if (i < 3) info[i] = 0;
}

struct AdjLayout {
  size_t key_a, key_b, idx_a, perm, head, pos, start, uu, vv, w, node_a, node_b, ent_a, ent_b,
      deg, temp, total, temp_bytes;
};

int adj_layout(int64_t E, int64_t n, AdjLayout* L) {
  const size_t e = size_t(E > 0 ? E : 1);
  size_t sort64 = 0, sort32 = 0, scan = 0, scan_n = 0;
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, sort64, (uint64_t*)nullptr, (uint64_t*)nullptr,
                                          (int32_t*)nullptr, (int32_t*)nullptr, e, 0u, 64u,
                                          hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, sort32, (uint32_t*)nullptr, (uint32_t*)nullptr,
                                          (int32_t*)nullptr, (int32_t*)nullptr, 2 * e, 0u, 32u,
                                          hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan, (int32_t*)nullptr, (int32_t*)nullptr, 0, e,
                                        rocprim::plus<int32_t>(), hipStream_t(0)));
  NGT_HIP_CHECK(rocprim::exclusive_scan(nullptr, scan_n, (int32_t*)nullptr, (int32_t*)nullptr, 0,
                                        size_t(n + 1), rocprim::plus<int32_t>(), hipStream_t(0)));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  };
  L->key_a = take(e * 8);
  L->key_b = take(e * 8);
  L->idx_a = take(e * 4);
  L->perm = take(e * 4);
  L->head = take(e * 4);
  L->pos = take(e * 4);
  L->start = take((e + 1) * 4);
  L->uu = take(e * 4);
  L->vv = take(e * 4);
  L->w = take(e * 4);
  L->node_a = take(2 * e * 4);
  L->node_b = take(2 * e * 4);
  L->ent_a = take(2 * e * 4);
  L->ent_b = take(2 * e * 4);
  L->deg = take(size_t(n + 1) * 4);
  L->temp_bytes = std::max(std::max(sort64, sort32), std::max(scan, scan_n));
  L->temp = take(L->temp_bytes);
  L->total = off;
  return NGT_OK;
}

}  // namespace
}  // namespace ngt

using namespace ngt;

extern "C" int ngt_adj_weights_workspace_bytes(int64_t n_entries, int64_t n_nodes, size_t* bytes) {
  if (n_entries < 0 || n_nodes < 0 || !bytes)
    return set_error(NGT_ERR_ARG, "ngt_adj_weights_workspace_bytes: bad arguments");
  AdjLayout L{};
  NGT_CHECK_OK(adj_layout(n_entries, n_nodes, &L));
  *bytes = L.total;
  return NGT_OK;
}

extern "C" int ngt_adj_weights(const int64_t* edge_index, const float* ppr_val, int64_t n_entries,
                               int64_t n_nodes, int32_t* xadj, int32_t* adjncy,
                               int32_t* eweights, int64_t* info, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (n_entries < 0 || n_nodes < 0)
    return set_error(NGT_ERR_ARG, "ngt_adj_weights: negative size");
  if (n_entries > 0x3fffffff)
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_adj_weights: at most 2^30 entries");
  if (n_nodes > 0x7fffffff || uint64_t(n_nodes) * uint64_t(n_nodes) >= (uint64_t(1) << 63))
    return set_error(NGT_ERR_UNSUPPORTED, "ngt_adj_weights: too many nodes");
  if (!xadj || !info || (n_entries > 0 && (!edge_index || !ppr_val || !adjncy || !eweights)))
    return set_error(NGT_ERR_ARG, "ngt_adj_weights: null pointer");
  AdjLayout L{};
  NGT_CHECK_OK(adj_layout(n_entries, n_nodes, &L));
  if (!workspace || workspace_bytes < L.total)
    return set_error(NGT_ERR_WORKSPACE, "ngt_adj_weights: workspace %zu < %zu", workspace_bytes,
                     L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* deg = reinterpret_cast<int32_t*>(ws + L.deg);
  KernelTimer timer_("adj_weights", st);
  hipLaunchKernelGGL(k_adj_zero, dim3(grid_for(n_nodes + 1)), dim3(kBlock), 0, st, deg,
                     n_nodes + 1, info);
  NGT_HIP_CHECK(hipGetLastError());
  const int64_t E = n_entries;
  if (E > 0) {
    uint64_t* key_a = reinterpret_cast<uint64_t*>(ws + L.key_a);
    uint64_t* key_b = reinterpret_cast<uint64_t*>(ws + L.key_b);
    int32_t* idx_a = reinterpret_cast<int32_t*>(ws + L.idx_a);
    int32_t* perm = reinterpret_cast<int32_t*>(ws + L.perm);
    int32_t* head = reinterpret_cast<int32_t*>(ws + L.head);
    int32_t* pos = reinterpret_cast<int32_t*>(ws + L.pos);
    int32_t* start = reinterpret_cast<int32_t*>(ws + L.start);
    int32_t* uu = reinterpret_cast<int32_t*>(ws + L.uu);
    int32_t* vv = reinterpret_cast<int32_t*>(ws + L.vv);
    int32_t* w = reinterpret_cast<int32_t*>(ws + L.w);
    uint32_t* node_a = reinterpret_cast<uint32_t*>(ws + L.node_a);
    uint32_t* node_b = reinterpret_cast<uint32_t*>(ws + L.node_b);
    int32_t* ent_a = reinterpret_cast<int32_t*>(ws + L.ent_a);
    int32_t* ent_b = reinterpret_cast<int32_t*>(ws + L.ent_b);
    void* temp = ws + L.temp;
    const uint64_t sentinel = uint64_t(n_nodes) * uint64_t(n_nodes);
    hipLaunchKernelGGL(k_adj_keys, dim3(grid_for(E)), dim3(kBlock), 0, st, edge_index,
                       edge_index + E, E, n_nodes, key_a, idx_a, info);
    NGT_HIP_CHECK(hipGetLastError());
    size_t tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::radix_sort_pairs(temp, tb, key_a, key_b, idx_a, perm, size_t(E), 0u,
                                            bits_for(sentinel), st));
    hipLaunchKernelGGL(k_adj_heads, dim3(grid_for(E)), dim3(kBlock), 0, st, key_b, E, sentinel,
                       head);
    NGT_HIP_CHECK(hipGetLastError());
    tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::exclusive_scan(temp, tb, head, pos, 0, size_t(E),
                                          rocprim::plus<int32_t>(), st));
    hipLaunchKernelGGL(k_adj_starts, dim3(grid_for(E)), dim3(kBlock), 0, st, key_b, head, pos,
                       E, sentinel, n_nodes, start, uu, vv, info);
    NGT_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(k_adj_weights, dim3(grid_for(E)), dim3(kBlock), 0, st, ppr_val, perm, start,
                       info, w, deg, uu, vv);
    NGT_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(k_adj_dir_keys, dim3(grid_for(2 * E)), dim3(kBlock), 0, st, uu, vv, info,
                       int64_t(2 * E), uint32_t(n_nodes), node_a, ent_a);
    NGT_HIP_CHECK(hipGetLastError());
    // stable by node: within a row the (u, v > u) entries, then the (v < u, u)
    // ones, each in key order
    tb = L.temp_bytes;
    NGT_HIP_CHECK(rocprim::radix_sort_pairs(temp, tb, node_a, node_b, ent_a, ent_b, size_t(2 * E),
                                            0u, bits_for(uint64_t(n_nodes)), st));
    hipLaunchKernelGGL(k_adj_emit, dim3(grid_for(2 * E)), dim3(kBlock), 0, st, ent_b, uu, vv, w,
                       info, adjncy, eweights);
    NGT_HIP_CHECK(hipGetLastError());
  }
  size_t tb = L.temp_bytes;
  NGT_HIP_CHECK(rocprim::exclusive_scan(ws + L.temp, tb, deg, xadj, 0, size_t(n_nodes + 1),
                                        rocprim::plus<int32_t>(), st));
  return NGT_OK;
}
