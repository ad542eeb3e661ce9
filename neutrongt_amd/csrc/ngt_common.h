// Shared device helpers for the window attention kernels (gfx950, wave64).
//
// Element types: the kernels read q/k/v and write outputs in either fp32 or
// bf16 (stored as raw uint16).  All arithmetic is fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/ngt_attn.h"

namespace ngt {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 <-> f32
struct bf16_t {
  uint16_t x;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even (the rule torch uses for float -> bfloat16); NaN stays
// a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Two floats -> packed bf16 pair with the hardware round-to-nearest-even
// conversion (v_cvt_pk_bf16_f32); low half = a.
typedef float ngt_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 ngt_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  const ngt_f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ngt_bf16x2));
}

template <typename T>
struct elem;
template <>
struct elem<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <>
struct elem<bf16_t> {
  static __device__ __forceinline__ float load(const bf16_t* p) { return bf16_to_f32(p->x); }
  static __device__ __forceinline__ void store(bf16_t* p, float v) { p->x = f32_to_bf16(v); }
};

// ------------------------------------------------------- vector row load/store
// Load DH consecutive elements starting at p into fp32 registers.  The widest
// access that divides the row is used (16 B when the row is a multiple of 16 B;
// callers guarantee 16-byte aligned base pointers and row strides).
template <typename T, int DH>
__device__ __forceinline__ void load_row(const T* __restrict__ p, float (&out)[DH]) {
  constexpr int bytes = DH * static_cast<int>(sizeof(T));
  if constexpr (bytes % 16 == 0) {
    const uint4* v = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < bytes / 16; ++i) {
      const uint4 w = v[i];
      if constexpr (sizeof(T) == 4) {
        out[4 * i + 0] = __uint_as_float(w.x);
        out[4 * i + 1] = __uint_as_float(w.y);
        out[4 * i + 2] = __uint_as_float(w.z);
        out[4 * i + 3] = __uint_as_float(w.w);
      } else {
        out[8 * i + 0] = __uint_as_float(w.x << 16);
        out[8 * i + 1] = __uint_as_float(w.x & 0xffff0000u);
        out[8 * i + 2] = __uint_as_float(w.y << 16);
        out[8 * i + 3] = __uint_as_float(w.y & 0xffff0000u);
        out[8 * i + 4] = __uint_as_float(w.z << 16);
        out[8 * i + 5] = __uint_as_float(w.z & 0xffff0000u);
        out[8 * i + 6] = __uint_as_float(w.w << 16);
        out[8 * i + 7] = __uint_as_float(w.w & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) out[c] = elem<T>::load(p + c);
  }
}

template <typename T, int DH>
__device__ __forceinline__ void store_row(T* __restrict__ p, const float (&in)[DH]) {
  constexpr int bytes = DH * static_cast<int>(sizeof(T));
  if constexpr (bytes % 16 == 0) {
    uint4* v = reinterpret_cast<uint4*>(p);
#pragma unroll
    for (int i = 0; i < bytes / 16; ++i) {
      uint4 w;
      if constexpr (sizeof(T) == 4) {
        w.x = __float_as_uint(in[4 * i + 0]);
        w.y = __float_as_uint(in[4 * i + 1]);
        w.z = __float_as_uint(in[4 * i + 2]);
        w.w = __float_as_uint(in[4 * i + 3]);
      } else {
        w.x = pack2_bf16(in[8 * i + 0], in[8 * i + 1]);
        w.y = pack2_bf16(in[8 * i + 2], in[8 * i + 3]);
        w.z = pack2_bf16(in[8 * i + 4], in[8 * i + 5]);
        w.w = pack2_bf16(in[8 * i + 6], in[8 * i + 7]);
      }
      v[i] = w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) elem<T>::store(p + c, in[c]);
  }
}

// Raw 16-byte row chunks: a row slice of DH elements of T is NV = DH*sizeof(T)/16
// uint4 words (every supported head size is a multiple of 16 bytes).  Loading raw
// words first and converting at use keeps bf16 rows packed in registers while
// the loads of several edges are in flight.
template <typename T, int DH>
struct RowWords {
  static_assert((DH * sizeof(T)) % 16 == 0, "row slice must be a multiple of 16 bytes");
  static constexpr int NV = DH * static_cast<int>(sizeof(T)) / 16;
  uint4 w[NV];
};

template <typename T, int DH>
__device__ __forceinline__ void load_words(const T* __restrict__ p, RowWords<T, DH>& r) {
  const uint4* v = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < RowWords<T, DH>::NV; ++i) r.w[i] = v[i];
}

template <typename T, int DH>
__device__ __forceinline__ void zero_words(RowWords<T, DH>& r) {
#pragma unroll
  for (int i = 0; i < RowWords<T, DH>::NV; ++i) r.w[i] = make_uint4(0u, 0u, 0u, 0u);
}

template <typename T, int DH>
__device__ __forceinline__ float word_elem(const RowWords<T, DH>& r, int c) {
  if constexpr (sizeof(T) == 4) {
    const uint4 w = r.w[c / 4];
    const uint32_t x = (c % 4 == 0) ? w.x : (c % 4 == 1) ? w.y : (c % 4 == 2) ? w.z : w.w;
    return __uint_as_float(x);
  } else {
    const uint4 w = r.w[c / 8];
    const int k = (c % 8) / 2;
    const uint32_t x = (k == 0) ? w.x : (k == 1) ? w.y : (k == 2) ? w.z : w.w;
    return (c % 2 == 0) ? __uint_as_float(x << 16) : __uint_as_float(x & 0xffff0000u);
  }
}

template <typename T, int DH>
__device__ __forceinline__ void words_to_f32(const RowWords<T, DH>& r, float (&out)[DH]) {
#pragma unroll
  for (int c = 0; c < DH; ++c) out[c] = word_elem<T, DH>(r, c);
}

template <typename T, int DH>
__device__ __forceinline__ uint32_t row_word(const RowWords<T, DH>& r, int p) {
  const uint4 w = r.w[p / 4];
  return (p % 4 == 0) ? w.x : (p % 4 == 1) ? w.y : (p % 4 == 2) ? w.z : w.w;
}

// Dot product of two head slices held as raw words.  Every score of the sparse
// path goes through this one function (operands in the same order), so the
// backward recomputes bit-identical scores.  bf16: v_dot2c_f32_bf16 over
// element pairs (products exact in fp32); fp32: fma chains.  Two interleaved
// accumulators either way.
typedef __bf16 ngt_bf16x2v __attribute__((ext_vector_type(2)));
template <typename T, int DH>
__device__ __forceinline__ float edge_dot(const RowWords<T, DH>& a, const RowWords<T, DH>& b) {
  float s0 = 0.f, s1 = 0.f;
  if constexpr (sizeof(T) == 2) {
    constexpr int NW = DH / 2;
#pragma unroll
    for (int p = 0; p < NW; p += 2) {
      s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ngt_bf16x2v, row_word<T, DH>(a, p)),
                                           __builtin_bit_cast(ngt_bf16x2v, row_word<T, DH>(b, p)),
                                           s0, false);
      if (p + 1 < NW)
        s1 = __builtin_amdgcn_fdot2_f32_bf16(
            __builtin_bit_cast(ngt_bf16x2v, row_word<T, DH>(a, p + 1)),
            __builtin_bit_cast(ngt_bf16x2v, row_word<T, DH>(b, p + 1)), s1, false);
    }
  } else {
#pragma unroll
    for (int c = 0; c < DH; c += 2) {
      s0 = fmaf(word_elem<T, DH>(a, c), word_elem<T, DH>(b, c), s0);
      if (c + 1 < DH) s1 = fmaf(word_elem<T, DH>(a, c + 1), word_elem<T, DH>(b, c + 1), s1);
    }
  }
  return s0 + s1;
}

// fp32 rows (partials, statistics) with 16-byte accesses when DH % 4 == 0.
template <int DH>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&out)[DH]) {
  if constexpr (DH % 4 == 0) {
    const float4* v = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < DH / 4; ++i) {
      float4 w = v[i];
      out[4 * i + 0] = w.x;
      out[4 * i + 1] = w.y;
      out[4 * i + 2] = w.z;
      out[4 * i + 3] = w.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) out[c] = p[c];
  }
}

template <int DH>
__device__ __forceinline__ void store_f32(float* __restrict__ p, const float (&in)[DH]) {
  if constexpr (DH % 4 == 0) {
    float4* v = reinterpret_cast<float4*>(p);
#pragma unroll
    for (int i = 0; i < DH / 4; ++i) v[i] = make_float4(in[4 * i], in[4 * i + 1], in[4 * i + 2], in[4 * i + 3]);
  } else {
#pragma unroll
    for (int c = 0; c < DH; ++c) p[c] = in[c];
  }
}

// ------------------------------------------------------------ wave reductions
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// Sum over the lanes that share (lane % L) -- i.e. across the 64/L edge slots
// of a wave whose lanes are laid out as (slot, head).
template <int DH>
__device__ __forceinline__ void reduce_slots(float (&acc)[DH], float& z, int L) {
  for (int off = L; off < kWave; off <<= 1) {
    z += shfl_xor(z, off);
#pragma unroll
    for (int c = 0; c < DH; ++c) acc[c] += shfl_xor(acc[c], off);
  }
}

template <int DH>
__device__ __forceinline__ void reduce_slots2(float (&a)[DH], float (&b)[DH], int L) {
  for (int off = L; off < kWave; off <<= 1) {
#pragma unroll
    for (int c = 0; c < DH; ++c) {
      a[c] += shfl_xor(a[c], off);
      b[c] += shfl_xor(b[c], off);
    }
  }
}

template <int DH>
__device__ __forceinline__ void reduce_slots1(float (&a)[DH], int L) {
  for (int off = L; off < kWave; off <<= 1) {
#pragma unroll
    for (int c = 0; c < DH; ++c) a[c] += shfl_xor(a[c], off);
  }
}

// Sum over the low log2(L) lane bits (the heads of one slot).
__device__ __forceinline__ float reduce_heads(float v, int L) {
  for (int off = 1; off < L; off <<= 1) v += shfl_xor(v, off);
  return v;
}

// ------------------------------------------------------------ dropout masks
// Dropout of attention probabilities (dense attention in training mode).
// One 32-bit word serves two adjacent keys of a (head, query) row:
//   word(h, i, j) = mix32((i * ceil(n_k / 2) + j / 2) ^ head_key(seed, h))
//   keep(h, i, j) = (j odd ? word >> 16 : word & 0xffff) >= thr
// with thr = round(p * 65536), so the keep probability is 1 - thr / 65536
// (exactly 1 - p for p a multiple of 2^-16, e.g. 0.5).  Every kernel derives
// the same bit for an element from its coordinates alone, so the backward
// reproduces the forward's mask without storing it.  Kept probabilities are
// scaled by 1 / (1 - p); p = 1 drops everything (scale 0).  mix32 is the
// "lowbias32" integer hash (C. Wellons, hash-prospector, public domain).
// The seed is either a value fixed at launch or, with seed_dev set, read from
// device memory when the kernel starts: a captured HIP graph whose replays
// refresh that word (e.g. from torch's graph-safe generator) then draws a new
// mask per replay instead of replaying the captured one.
struct DropoutMask {
  uint64_t seed;
  const uint64_t* seed_dev;  // null: use seed
  uint32_t head_key;  // drop_head_key(seed, h): set by the kernel for its head
  uint32_t n_kp;      // ceil(n_k / 2): words per query row
  uint32_t thr;       // keep iff the 16-bit half >= thr
  float scale;        // 1 / (1 - p), 0 for p = 1
};

__host__ __device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

__host__ __device__ __forceinline__ uint32_t drop_head_key(uint64_t seed, uint32_t h) {
  return mix32(static_cast<uint32_t>(seed) ^
               mix32(static_cast<uint32_t>(seed >> 32) + 0x9e3779b9U * (h + 1U)));
}

__device__ __forceinline__ uint64_t drop_seed(const DropoutMask& dm) {
  return dm.seed_dev ? *dm.seed_dev : dm.seed;
}

__device__ __forceinline__ DropoutMask drop_for_head(DropoutMask dm, int h) {
  dm.seed = drop_seed(dm);
  dm.head_key = drop_head_key(dm.seed, static_cast<uint32_t>(h));
  return dm;
}

__device__ __forceinline__ uint32_t drop_word(const DropoutMask& dm, uint32_t i, uint32_t j) {
  return mix32((i * dm.n_kp + (j >> 1)) ^ dm.head_key);
}

// Scale applied to element (.., j) given its pair's word: 1/(1-p) or 0.
__device__ __forceinline__ float drop_scale(const DropoutMask& dm, uint32_t word, uint32_t j) {
  const uint32_t half = (j & 1U) ? (word >> 16) : (word & 0xffffU);
  return half >= dm.thr ? dm.scale : 0.f;
}


template <typename T>
struct dtype_of;
template <>
struct dtype_of<float> {
  static constexpr int value = NGT_F32;
};
template <>
struct dtype_of<bf16_t> {
  static constexpr int value = NGT_BF16;
};

// Key split of a dense matrix-core pass: n_split blocks along grid z, each
// over split_keys consecutive keys (a multiple of the 128-key stage).
struct MfSplit {
  int n_split;
  int split_keys;
};

// Records a message for ngt_last_error() (thread-local) and returns the code.
int set_error(int code, const char* fmt, ...);

// Optional per-kernel timing (ngt_timing_enable): when on, a KernelTimer
// placed around a launch records a start/stop hipEvent pair on the launch
// stream; ngt_timing_summary() aggregates them per kernel name.
bool timing_enabled();
void timing_record(const char* name, hipStream_t st, bool start);

struct KernelTimer {
  const char* name;
  hipStream_t st;
  bool on;
  KernelTimer(const char* n, hipStream_t s) : name(n), st(s), on(timing_enabled()) {
    if (on) timing_record(name, st, true);
  }
  ~KernelTimer() {
    if (on) timing_record(name, st, false);
  }
};

// Host: the DropoutMask of keep probability 1 - p for an n_q x n_k score
// matrix (one word per query and key pair); *on is false for p = 0.
inline int make_dropout(const char* fn, float p, uint64_t seed, const uint64_t* seed_dev, int n_q,
                 int n_k, DropoutMask* dm, bool* on) {
  *on = false;
  if (!(p >= 0.f && p <= 1.f))
    return set_error(NGT_ERR_ARG, "%s: dropout_p=%g outside [0, 1]", fn, double(p));
  if (p == 0.f) return NGT_OK;
  const uint64_t words = uint64_t(n_q) * ((uint64_t(n_k) + 1) / 2);
  if (words > (uint64_t(1) << 32))
    return set_error(NGT_ERR_UNSUPPORTED,
                     "%s: dropout needs n_q * ceil(n_k / 2) <= 2^32 (n_q=%d n_k=%d)", fn, n_q, n_k);
  dm->seed = seed;
  dm->seed_dev = seed_dev;
  dm->head_key = 0;
  dm->n_kp = static_cast<uint32_t>((uint64_t(n_k) + 1) / 2);
  if (p >= 1.f) {  // everything dropped: keep-all mask with scale 0
    dm->thr = 0;
    dm->scale = 0.f;
  } else {
    dm->thr = static_cast<uint32_t>(lrint(double(p) * 65536.0));
    dm->scale = static_cast<float>(1.0 / (1.0 - double(p)));
  }
  *on = true;
  return NGT_OK;
}

}  // namespace ngt

#define NGT_CHECK_OK(expr)                                                               \
  do {                                                                                   \
    const int _rc = (expr);                                                              \
    if (_rc != NGT_OK) return _rc;                                                       \
  } while (0)

#define NGT_HIP_CHECK(expr)                                                              \
  do {                                                                                   \
    hipError_t _e = (expr);                                                              \
    if (_e != hipSuccess)                                                                \
      return ::ngt::set_error(NGT_ERR_HIP, "%s:%d %s: %s", __FILE__, __LINE__, #expr,    \
                              hipGetErrorString(_e));                                    \
  } while (0)
