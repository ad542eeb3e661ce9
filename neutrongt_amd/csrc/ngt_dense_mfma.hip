// Dense full-window attention on the matrix cores (bf16 inputs, fp32
// accumulation), head_dim d in {8, 16, 24, 32}.
//
// Products run on v_mfma_f32_32x32x8_bf16 and, two K steps at a time, on
// v_mfma_f32_32x32x16_bf16 (mfma2): K = 8 equals the smallest head dim, so the
// QK^T and dP = G V^T contractions over d have no padding, and the PV-class
// contractions over keys/queries take 16-row K steps.  Lane layouts of the
// 32x32x8 instruction (checked on gfx950):
//   A (32 x 8):  lane l holds A[l % 32][4*(l/32) + i], i < 4
//   B (8 x 32):  lane l holds B[4*(l/32) + i][l % 32], i < 4
//   D (32 x 32): lane l holds D[8*(i/4) + 4*(l/32) + i%4][l % 32], i < 16
// The D rows a lane holds for i = 4j..4j+3 are exactly the B rows it must
// supply for K step j, so a score tile computed with the contraction index in
// its rows feeds the next MFMA as B without any data movement.
//
// Forward, per (head, 32 queries): S^T = K Q^T (rows = keys, cols = queries),
// online softmax per query column (in-lane over 16 keys; the column maximum
// over both wave halves only when the base moves), O^T += V^T P^T with V^T
// staged in LDS.  Column scores sum_i |S| come from key-major blocks in the
// same launch (S tiles again on MFMA).  Backward, in this order: query-major
// dQ (dQ += dS K with K staged in LDS; it also forms each query's D = G . o)
// and key-major dK/dV (S and dP recomputed as D[q][key], dV += P^T G and
// dK += dS^T Q with Q/G tiles staged in LDS; extra blocks merge the dQ key
// splits).
// Per-score arithmetic rides in the MFMAs: the softmax scale as a hi/lo bf16
// pair of the per-lane operand (split_scaled), the per-query -lse, -D and the
// forward's running maximum as accumulator inputs or as one more K step of
// three bf16 pieces (split3), so a score costs an exponential and a pack.
// Dropout (DROP = true): the PV-class products take P o M, M = keep/(1-p)
// from DropoutMask; the forward's row sums still come from the unmasked P
// (an extra MFMA per K step against a constant ones row), and the backward
// forms dS = P o (M dP - D) on the VALU.
#include "ngt_common.h"

#include <math.h>
#include <stdlib.h>

#include <algorithm>

namespace ngt {
namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Work-item and work-group ids as register reads.  The kernels of this file
// are built with the IEEE mode bit off, which the device library's functions
// behind threadIdx / blockIdx / gridDim are not, and the compiler does not
// inline across that difference: each use would be a call whose result it
// treats as a per-lane value, so loop bounds derived from a block index would
// be compared on the VALU in every tile.
__device__ __forceinline__ int tid_x() { return static_cast<int>(__builtin_amdgcn_workitem_id_x()); }
__device__ __forceinline__ int wg_x() { return static_cast<int>(__builtin_amdgcn_workgroup_id_x()); }
__device__ __forceinline__ int wg_y() { return static_cast<int>(__builtin_amdgcn_workgroup_id_y()); }
__device__ __forceinline__ int wg_z() { return static_cast<int>(__builtin_amdgcn_workgroup_id_z()); }

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kT = 32;                  // tile edge (rows/cols of one MFMA)
constexpr int kRowsPerBlock = kWaves * kT;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRebase = 8.f;  // forward: P entries stay below 2^8 (fp32 sums, bf16 operands)

__device__ __forceinline__ f32x16 mfma(s16x4 a, s16x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(a, b, c, 0, 0, 0);
}

// Two K = 8 steps as one v_mfma_f32_32x32x16_bf16 (which the chip runs at
// twice the rate of the K = 8 form): the lane's A operand is a0 ++ a1 and its
// B operand b0 ++ b1.  Element r of a lane's A and of its B carry the same
// contraction index, so pairing a0 with b0 and a1 with b1 slot by slot gives
// exactly mfma(a1, b1, mfma(a0, b0, c)) up to the fp32 accumulation order,
// whatever order the instruction assigns to the 16 indices.
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x16 mfma2(s16x4 a0, s16x4 a1, s16x4 b0, s16x4 b1, f32x16 c) {
  const s16x8 a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
  const s16x8 b = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// 4 consecutive bf16 of a row (8-byte aligned: d is a multiple of 8).
__device__ __forceinline__ s16x4 load4(const bf16_t* p) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  s16x4 r;
  r[0] = static_cast<short>(w.x & 0xffffu);
  r[1] = static_cast<short>(w.x >> 16);
  r[2] = static_cast<short>(w.y & 0xffffu);
  r[3] = static_cast<short>(w.y >> 16);
  return r;
}

// Operands loaded from global memory before a stage loop go through an empty
// asm that reads and rewrites their registers: the wait for those loads is
// then placed before the loop.  Without it the wait lands on the first MFMA
// inside the loop as vmcnt(0), which also waits for the next stage's prefetch
// and serialises it with the compute.
__device__ __forceinline__ s16x4 settle(s16x4 x) {
  uint2 w = __builtin_bit_cast(uint2, x);
  asm volatile("" : "+v"(w.x), "+v"(w.y));
  return __builtin_bit_cast(s16x4, w);
}

__device__ __forceinline__ s16x4 zero4() {
  s16x4 r;
  r[0] = r[1] = r[2] = r[3] = 0;
  return r;
}

// Four floats -> MFMA operand of packed bf16 (hardware RNE conversion).
__device__ __forceinline__ s16x4 pack4(float a, float b, float c, float d) {
  const uint2 w = make_uint2(pack2_bf16(a, b), pack2_bf16(c, d));
  return __builtin_bit_cast(s16x4, w);
}

// x * s as two bf16 operands hi = RNE(x s), lo = RNE(x s - hi) (the
// difference is exact in fp32): contracting a bf16 row r against hi ++ lo
// gives r . (x s) with products exact and a relative error of at most 2^-18
// per term, so the softmax scale rides inside the MFMA instead of costing a
// VALU multiply per score.
__device__ __forceinline__ void split_scaled(s16x4 x, float s, s16x4& hi, s16x4& lo) {
  float f[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) f[i] = bf16_to_f32(static_cast<uint16_t>(x[i])) * s;
  hi = pack4(f[0], f[1], f[2], f[3]);
  lo = pack4(f[0] - bf16_to_f32(static_cast<uint16_t>(hi[0])),
             f[1] - bf16_to_f32(static_cast<uint16_t>(hi[1])),
             f[2] - bf16_to_f32(static_cast<uint16_t>(hi[2])),
             f[3] - bf16_to_f32(static_cast<uint16_t>(hi[3])));
}

// x as three bf16 pieces {hi, mid, lo, 0} (each the RNE of the exact fp32
// remainder), so that hi + mid + lo carries x to fp32 precision: a per-row
// term folded into a tile as one more MFMA K step costs no accuracy.
__device__ __forceinline__ uint2 split3(float x) {
  const uint16_t hi = f32_to_bf16(x);
  const float r1 = x - bf16_to_f32(hi);
  const uint16_t mid = f32_to_bf16(r1);
  const float r2 = r1 - bf16_to_f32(mid);
  return make_uint2(uint32_t(hi) | (uint32_t(mid) << 16), uint32_t(f32_to_bf16(r2)));
}

// Constant MFMA operand with ones in slots 0-2 of the lanes of half `which`:
// against split3 pieces held by those lanes it adds hi + mid + lo.
__device__ __forceinline__ s16x4 ones3(int half, int which) {
  s16x4 r = zero4();
  if (half == which) r[0] = r[1] = r[2] = static_cast<short>(0x3f80);
  return r;
}

__device__ __forceinline__ f32x16 fill16(float v) {
  f32x16 r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = v;
  return r;
}

__device__ __forceinline__ float sum4(s16x4 x) {
  return (bf16_to_f32(static_cast<uint16_t>(x[0])) + bf16_to_f32(static_cast<uint16_t>(x[1]))) +
         (bf16_to_f32(static_cast<uint16_t>(x[2])) + bf16_to_f32(static_cast<uint16_t>(x[3])));
}


// ------------------------------------------------------------- LDS staging
// A block stages kSB rows (keys or queries) of one head at a time: each thread
// prefetches its 16-byte pieces of the next stage into registers while the
// block computes on the current one, then writes them to LDS either row-major
// ([row][c], read as A operands) or transposed ([c][row], read as B operands).
constexpr int kSB = 128;

// LDS row padding (shorts) of the row-major stages [kSB][DH + kRowPad] and the
// transposed ones [kT][kSB + kColPad].  Operands are read 8 bytes per lane
// from 32 consecutive rows; with row strides of DH + 4 and kSB + 4 shorts
// (odd multiples of 8 bytes) 16 lanes fall on 16 distinct
// bank pairs for every supported d, where + 8 left 2-4 lanes per bank
// (SQ_LDS_BANK_CONFLICT 4x the LDS busy cycles in the forward; 16,000-node
// window fwd+bwd 1.51 -> 1.47 ms).
#ifndef NGT_DENSE_ROW_PAD
#define NGT_DENSE_ROW_PAD 4
#endif
#ifndef NGT_DENSE_COL_PAD
#define NGT_DENSE_COL_PAD 4
#endif
constexpr int kRowPad = NGT_DENSE_ROW_PAD;
constexpr int kColPad = NGT_DENSE_COL_PAD;
static_assert(kRowPad % 4 == 0 && kColPad % 4 == 0, "8-byte aligned operand reads");

template <int DH>
struct Stage {
  static constexpr int VPR = DH / 8;                          // 16-byte pieces per row
  static constexpr int NV = (kSB * VPR + kBlock - 1) / kBlock;  // pieces per thread
  uint4 w[NV];

  __device__ __forceinline__ void load(const bf16_t* __restrict__ base, int64_t row0, int n_rows,
                                       int H, int h) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid_x() + i * kBlock;
      const int r = e / VPR, cv = e - r * VPR;
      w[i] = make_uint4(0u, 0u, 0u, 0u);
      if (e < kSB * VPR && row0 + r < n_rows)
        w[i] = *reinterpret_cast<const uint4*>(base + ((row0 + r) * H + h) * DH + 8 * cv);
    }
  }
  __device__ __forceinline__ void store_rows(short (*lds)[DH + kRowPad]) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid_x() + i * kBlock;
      if (e < kSB * VPR) {
        const int r = e / VPR, cv = e - r * VPR;
        if constexpr ((DH + kRowPad) % 8 == 0) {
          *reinterpret_cast<uint4*>(&lds[r][8 * cv]) = w[i];
        } else {  // rows only 8-byte aligned
          *reinterpret_cast<uint2*>(&lds[r][8 * cv]) = make_uint2(w[i].x, w[i].y);
          *reinterpret_cast<uint2*>(&lds[r][8 * cv + 4]) = make_uint2(w[i].z, w[i].w);
        }
      }
    }
  }
  __device__ __forceinline__ void store_trans(short (*lds)[kSB + kColPad]) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid_x() + i * kBlock;
      if (e < kSB * VPR) {
        const int r = e / VPR, cv = e - r * VPR;
        const uint32_t u[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          lds[8 * cv + 2 * t][r] = static_cast<short>(u[t] & 0xffffu);
          lds[8 * cv + 2 * t + 1][r] = static_cast<short>(u[t] >> 16);
        }
      }
    }
  }
};

__device__ __forceinline__ s16x4 lds4(const short* p) {
  return __builtin_bit_cast(s16x4, *reinterpret_cast<const uint2*>(p));
}

// Transposed stages are kT rows tall: rows DH .. kT-1 hold constants written
// once (zeros, and for the forward with DH < 32 a row of ones at DH), so every
// lane reads its B operand unconditionally -- no exec-masked LDS reads, whose
// waits would serialise the K steps.
template <int DH>
__device__ __forceinline__ void fill_pad_rows(short (*t)[kSB + kColPad], bool ones_row) {
  constexpr int kPadRows = kT - DH;
  for (int e = tid_x(); e < kPadRows * (kSB + kColPad); e += kBlock) {
    const int r = DH + e / (kSB + kColPad), c = e % (kSB + kColPad);
    t[r][c] = (ones_row && r == DH) ? static_cast<short>(0x3f80) : static_cast<short>(0);
  }
}

// max(x, x of lane ^ 32): v_permlane32_swap exchanges the two wave halves.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ------------------------------------------------------------------ forward
// One block: queries bx*128 .. +127 of head h, keys of split z; wave w owns
// queries q0 .. q0+31.
template <int DH, bool DROP>
__device__ __forceinline__ void mf_fwd_block(int bx, int h, int z, const bf16_t* __restrict__ q,
                                             const bf16_t* __restrict__ k,
                                             const bf16_t* __restrict__ v, int32_t n_q,
                                             int32_t n_k, int32_t H, float scale, DropoutMask dm,
                                             bf16_t* __restrict__ out, float* __restrict__ out32,
                                             float* __restrict__ lse, int32_t split_keys,
                                             float* __restrict__ part_ml,
                                             float* __restrict__ part_acc) {
  constexpr int NC = DH / 8;  // K chunks of the QK^T contraction
  __shared__ __align__(16) short ks[kSB][DH + kRowPad];  // K rows
  __shared__ __align__(16) short vt[kT][kSB + kColPad];  // V^T: [c][key], rows >= DH constant
  const int lane = tid_x() & (kWave - 1);
  const int wave = tid_x() >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int64_t qi = int64_t(bx) * kRowsPerBlock + wave * kT + l32;
  const bool q_ok = qi < n_q;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  // With dropout the ones row moves out of V^T into this constant A operand
  // (row DH of A), multiplied with the unmasked P.
  s16x4 ones_a = zero4();
  if constexpr (DROP && DH < 32) {
    if (l32 == DH) ones_a[0] = ones_a[1] = ones_a[2] = ones_a[3] = static_cast<short>(0x3f80);
  }

  // Q^T as the B operand of S^T = K Q^T: lane holds Q[qi][8j + 4*half .. +4].
  s16x4 qb[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j)
    qb[j] = settle(q_ok ? load4(q + (qi * H + h) * DH + 8 * j + 4 * half) : zero4());

  const float s2 = scale * kLog2e;  // scores in log2 units
  // Q^T s2 as hi ++ lo operands: the MFMA yields scores already scaled, and
  // with the accumulator input -m (m the running maximum, once one is set) it
  // yields S s2 - m, so a tile that does not raise any column's maximum -- all
  // but the first few -- goes straight to exp2.
  s16x4 qhi[NC], qlo[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) split_scaled(qb[j], s2, qhi[j], qlo[j]);
  float m = -INFINITY, l = 0.f;
  float thr = -INFINITY;   // rebase threshold on S s2 - m
  f32x16 base = zero16();  // -m once m is finite
  f32x16 acc = zero16();  // O^T[c][q]: c = 8*(i/4) + 4*half + i%4

  // keys [k_begin, k_end) of this block's split (z; split_keys a
  // multiple of kSB); one split covers all keys
  const int k_begin = z * split_keys;
  const int k_end = min(n_k, k_begin + split_keys);
  fill_pad_rows<DH>(vt, !DROP);
  Stage<DH> pk, pv;
  pk.load(k, k_begin, k_end, H, h);
  pv.load(v, k_begin, k_end, H, h);
  for (int kb = k_begin; kb < k_end; kb += kSB) {
    __syncthreads();
    pk.store_rows(ks);
    pv.store_trans(vt);
    __syncthreads();
    if (kb + kSB < k_end) {
      pk.load(k, kb + kSB, k_end, H, h);
      pv.load(v, kb + kSB, k_end, H, h);
    }
    for (int sub = 0; sub < kSB / kT && kb + sub * kT < k_end; ++sub) {
      const int r0 = sub * kT;
      // S^T s2 - m tile (S^T s2 before the first maximum): rows = keys
      // kb + r0 + (8*(i/4) + 4*half + i%4), col = this lane's query.
      f32x16 st = base;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const s16x4 ka = lds4(&ks[r0 + l32][8 * j + 4 * half]);
        st = mfma2(ka, ka, qhi[j], qlo[j], st);
      }
      float mx = -INFINITY;
      if (kb + r0 + kT <= k_end) {
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[i]);
      } else {  // tail tile: keys past the split's end drop out
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (kb + r0 + 8 * (i / 4) + 4 * half + (i % 4) >= k_end) st[i] = -INFINITY;
          mx = fmaxf(mx, st[i]);
        }
      }
      // The base m moves only when a column's maximum exceeds it by more
      // than kRebase (log2 units), so scores up to 2^kRebase times the base
      // enter P and the row sum as they are -- exact, since both share the
      // base -- and after the first tile (m unset, base 0) a wave rebases
      // only on a rare large jump instead of whenever any of its 32 columns
      // finds a new maximum (most tiles).  The test needs no column maximum:
      // some lane's own 16 scores exceed thr (-inf before the first tile,
      // kRebase after it) exactly when some column's maximum does.
      if (__any(mx > thr)) {
        mx = max_halves(mx);  // the column's maximum; finite: the tile holds a key
        const bool first = m == -INFINITY;
        const float up = first ? mx : fmaxf(mx, 0.f);
        const float m_new = first ? mx : m + up;
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 0 for the first tile
        l *= alpha;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          acc[i] *= alpha;
          st[i] -= up;
        }
        m = m_new;
        base = fill16(-m);
        thr = kRebase;
      }
      s16x4 pb[4], pm[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p0 = __builtin_amdgcn_exp2f(st[4 * j]);
        const float p1 = __builtin_amdgcn_exp2f(st[4 * j + 1]);
        const float p2 = __builtin_amdgcn_exp2f(st[4 * j + 2]);
        const float p3 = __builtin_amdgcn_exp2f(st[4 * j + 3]);
        pb[j] = pack4(p0, p1, p2, p3);
        if constexpr (DROP) {
          // keys kb + r0 + 8j + 4*half + (0..3): two key pairs, one word each
          const uint32_t key = uint32_t(kb + r0 + 8 * j + 4 * half);
          const uint32_t w0 = drop_word(dm, uint32_t(qi), key);
          const uint32_t w1 = drop_word(dm, uint32_t(qi), key + 2);
          pm[j] = pack4(p0 * drop_scale(dm, w0, key), p1 * drop_scale(dm, w0, key + 1),
                        p2 * drop_scale(dm, w1, key + 2), p3 * drop_scale(dm, w1, key + 3));
        }
      }
      if constexpr (DH == 32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) l += sum4(pb[j]);
      }
      // O^T += V^T P^T, K steps of 8 keys.  For d < 32 row c = d of V^T is all
      // ones, so O^T row d accumulates the row sum of the (rounded) P; with
      // dropout that row comes from ones_a and the unmasked P instead.
      s16x4 va[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) va[j] = lds4(&vt[l32][r0 + 8 * j + 4 * half]);
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        if constexpr (DROP) {
          acc = mfma2(va[j], va[j + 1], pm[j], pm[j + 1], acc);
          if constexpr (DH < 32) acc = mfma2(ones_a, ones_a, pb[j], pb[j + 1], acc);
        } else {
          acc = mfma2(va[j], va[j + 1], pb[j], pb[j + 1], acc);
        }
      }
    }
  }
  if constexpr (DH < 32) {
    // O^T row d sits in acc[d/2] of the half-0 lanes (d is a multiple of 8).
    l = __shfl(acc[DH / 2], l32, kWave);
  } else {
    l = sum_halves(l);
  }
  if (!q_ok) return;
  if (part_ml) {
    // this split's softmax state in natural-log units (m ln 2, l) and its
    // unnormalised O, merged in split order by k_dense_combine
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = 8 * (i / 4) + 4 * half + (i % 4);
      if (c < DH) part_acc[((z * n_q + qi) * H + h) * DH + c] = acc[i];
    }
    if (half == 0) {
      part_ml[2 * ((z * H + h) * n_q + qi)] = m * kLn2;
      part_ml[2 * ((z * H + h) * n_q + qi) + 1] = l;
    }
    return;
  }
  const float inv = n_k > 0 ? 1.0f / l : 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = 8 * (i / 4) + 4 * half + (i % 4);
    if (c < DH) {
      out[(qi * H + h) * DH + c].x = f32_to_bf16(acc[i] * inv);
      if (out32) out32[(qi * H + h) * DH + c] = acc[i] * inv;
    }
  }
  if (half == 0) lse[int64_t(h) * n_q + qi] = n_k > 0 ? (m + __log2f(l)) * kLn2 : -INFINITY;
}

// Column scores: part[h][j] = sum_i |S[h, i, j]|.  One block: keys
// bx*128 .. +127 of head h; wave w owns keys k0 .. k0+31; S = Q K^T tiles
// with rows = queries, Q staged 128 rows at a time in LDS (prefetched while
// the previous stage computes).
template <int DH>
__device__ __forceinline__ void mf_scores_block(int bx, int h, const bf16_t* __restrict__ q,
                                                const bf16_t* __restrict__ k, int32_t n_q,
                                                int32_t n_k, int32_t H, float scale,
                                                float* __restrict__ part) {
  constexpr int NC = DH / 8;
  __shared__ __align__(16) short qs[kSB][DH + kRowPad];
  const int lane = tid_x() & (kWave - 1);
  const int wave = tid_x() >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int64_t kj = int64_t(bx) * kRowsPerBlock + wave * kT + l32;
  const bool k_ok = kj < n_k;
  s16x4 kbv[NC];  // K^T as B: lane holds K[kj][8j + 4*half .. +4]
#pragma unroll
  for (int j = 0; j < NC; ++j)
    kbv[j] = settle(k_ok ? load4(k + (kj * H + h) * DH + 8 * j + 4 * half) : zero4());
  float s = 0.f;
  Stage<DH> pq;
  pq.load(q, 0, n_q, H, h);
  for (int qb = 0; qb < n_q; qb += kSB) {
    __syncthreads();
    pq.store_rows(qs);
    __syncthreads();
    if (qb + kSB < n_q) pq.load(q, qb + kSB, n_q, H, h);
    for (int sub = 0; sub < kSB / kT && qb + sub * kT < n_q; ++sub) {
      f32x16 st = zero16();
#pragma unroll
      for (int j = 0; j + 1 < NC; j += 2)
        st = mfma2(lds4(&qs[sub * kT + l32][8 * j + 4 * half]),
                   lds4(&qs[sub * kT + l32][8 * j + 8 + 4 * half]), kbv[j], kbv[j + 1], st);
      if constexpr (NC % 2)
        st = mfma(lds4(&qs[sub * kT + l32][8 * (NC - 1) + 4 * half]), kbv[NC - 1], st);
#pragma unroll
      for (int i = 0; i < 16; ++i) s += fabsf(st[i]);  // padded query rows are zero
    }
  }
  s = sum_halves(s);
  if (k_ok && half == 0) part[int64_t(h) * n_k + kj] = s * scale;
}

// The forward and the column scores in one launch.  grid = (max(fwd_bx,
// score_bx), H, n_split + (part ? 1 : 0)): slices z < n_split are forward
// blocks (fwd_bx = ceil(n_q / 128)); the last slice, dispatched last, holds
// the score blocks (score_bx = ceil(n_k / 128)).  The scores need neither the
// softmax nor the output, so their blocks fill the CUs that the forward's
// last, partial round of blocks leaves idle, instead of running as a launch
// of their own after it.
template <int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_mf_fwd(const bf16_t* __restrict__ q,
                                                   const bf16_t* __restrict__ k,
                                                   const bf16_t* __restrict__ v, int32_t n_q,
                                                   int32_t n_k, int32_t H, float scale,
                                                   DropoutMask dm, bf16_t* __restrict__ out,
                                                   float* __restrict__ out32,
                                                   float* __restrict__ lse, int32_t split_keys,
                                                   float* __restrict__ part_ml,
                                                   float* __restrict__ part_acc,
                                                   int32_t n_split, int32_t fwd_bx,
                                                   int32_t score_bx, float* __restrict__ part) {
  const int bx = wg_x(), h = wg_y();
  const int z = wg_z();
  if (z == n_split) {  // block-uniform
    if (bx < score_bx) mf_scores_block<DH>(bx, h, q, k, n_q, n_k, H, scale, part);
    return;
  }
  if (bx < fwd_bx)
    mf_fwd_block<DH, DROP>(bx, h, z, q, k, v, n_q, n_k, H, scale, dm, out, out32, lse,
                           split_keys, part_ml, part_acc);
}

// grad_q = scale * sum of the key splits' partial dQ, added in split order;
// block b of nb takes elements b * kBlock + tid_x(), stepping nb * kBlock.
__device__ __forceinline__ void dq_combine(const float* __restrict__ part, int n_split, int64_t n,
                                           float scale, bf16_t* __restrict__ grad_q, int64_t b,
                                           int64_t nb) {
  for (int64_t t = b * kBlock + tid_x(); t < n; t += nb * kBlock) {
    float a = part[t];
    for (int s = 1; s < n_split; ++s) a += part[int64_t(s) * n + t];
    grad_q[t].x = f32_to_bf16(a * scale);
  }
}

// ----------------------------------------------------------------- backward
// Key-major: dK, dV for keys k0 .. k0+31 of one head.  S, dP recomputed as
// D[q][key]; Q and G stages of 128 queries in LDS, row-major (A operands of S
// and dP) and transposed (B operands of dV += P^T G and dK += dS^T Q).
//
// Blocks at grid x >= kv_bx do not take keys: with a split dQ pass
// (part_dq set) they add its partial dQ in split order into grad_q, so that
// merge rides in this launch instead of a launch of its own.
template <int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_mf_bwd_kv(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ g, const float* __restrict__ lse, const float* __restrict__ dsum,
    int32_t n_q, int32_t n_k, int32_t H, float scale, DropoutMask dm,
    bf16_t* __restrict__ grad_k, bf16_t* __restrict__ grad_v, int32_t kv_bx, int32_t comb_bx,
    const float* __restrict__ part_dq, int32_t n_split_q, bf16_t* __restrict__ grad_q) {
  if (wg_x() >= kv_bx) {  // block-uniform: a merge block (grid.y = H)
    dq_combine(part_dq, n_split_q, int64_t(n_q) * H * DH, scale, grad_q,
               int64_t(wg_x() - kv_bx) * H + wg_y(), int64_t(comb_bx) * H);
    return;
  }
  constexpr int NC = DH / 8;
  __shared__ __align__(16) short qs[kSB][DH + kRowPad];
  __shared__ __align__(16) short gs[kSB][DH + kRowPad];
  __shared__ __align__(16) short qt[kT][kSB + kColPad];  // rows >= DH zero
  __shared__ __align__(16) short gt[kT][kSB + kColPad];
  // per query row: the split3 pieces of -L (log2 units) in xr[0], of -D in
  // xr[1] (half-major: a half-wave reads 32 consecutive records)
  __shared__ __align__(16) uint2 xr[2][kSB];
  __shared__ __align__(16) float dd[kSB];  // -D, with dropout only
  const int lane = tid_x() & (kWave - 1);
  const int wave = tid_x() >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int h = wg_y();
  const int64_t kj = int64_t(wg_x()) * kRowsPerBlock + wave * kT + l32;
  const bool k_ok = kj < n_k;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  s16x4 kbv[NC], vbv[NC];  // K^T, V^T as B operands
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    kbv[j] = settle(k_ok ? load4(k + (kj * H + h) * DH + 8 * j + 4 * half) : zero4());
    vbv[j] = settle(k_ok ? load4(v + (kj * H + h) * DH + 8 * j + 4 * half) : zero4());
  }
  const float s2 = scale * kLog2e;
  // S s2 - L and dP - D come straight out of the MFMAs: K^T s2 as hi ++ lo
  // operands (each Q row read once, fed twice), and the query's -L and -D
  // pieces from its LDS record as one more K step each: -L held by the lower
  // lanes, -D by the upper ones, against constant ones on the matching half.
  s16x4 khi[NC], klo[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) split_scaled(kbv[j], s2, khi[j], klo[j]);
  const s16x4 ones_l = ones3(half, 0), ones_d = ones3(half, 1);
  f32x16 dk = zero16(), dv = zero16();  // D[key][c]: key = 8*(i/4)+4*half+i%4, c = l32
  Stage<DH> pq, pg;
  float pl = 0.f, pd = 0.f;
  auto prefetch = [&](int qb) {
    pq.load(q, qb, n_q, H, h);
    pg.load(g, qb, n_q, H, h);
    if (tid_x() < kSB) {
      const bool ok = qb + int(tid_x()) < n_q;
      // raw values here: scaling now would wait on this load (and on the
      // stage's prefetch before it) at once
      pl = ok ? lse[int64_t(h) * n_q + qb + tid_x()] : INFINITY;
      pd = ok ? dsum[int64_t(h) * n_q + qb + tid_x()] : 0.f;
    }
  };
  fill_pad_rows<DH>(qt, false);
  fill_pad_rows<DH>(gt, false);
  prefetch(0);
  for (int qb = 0; qb < n_q; qb += kSB) {
    __syncthreads();
    pq.store_rows(qs);
    pg.store_rows(gs);
    pq.store_trans(qt);
    pg.store_trans(gt);
    if (tid_x() < kSB) {
      // padded rows: -L = -1e30 (finite, so the zero slots of the D step
      // stay 0; exp2 of the score is 0), D = 0 with zero G rows
      const float nl = pl == INFINITY ? -1e30f : -pl * kLog2e;
      xr[0][tid_x()] = split3(nl);
      xr[1][tid_x()] = split3(-pd);
      if constexpr (DROP) dd[tid_x()] = -pd;
    }
    __syncthreads();
    if (qb + kSB < n_q) prefetch(qb + kSB);
    for (int sub = 0; sub < kSB / kT && qb + sub * kT < n_q; ++sub) {
      const int r0 = sub * kT;
      // S s2 - L and dP - D tiles (dP alone with dropout), rows = queries
      // qb + r0 + 8*(i/4) + 4*half + i%4, col = this lane's key.
      const s16x4 xa = __builtin_bit_cast(s16x4, xr[half][r0 + l32]);
      f32x16 st = zero16(), dp = zero16();
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const s16x4 qa = lds4(&qs[r0 + l32][8 * j + 4 * half]);
        st = mfma2(qa, qa, khi[j], klo[j], st);
      }
      st = mfma(xa, ones_l, st);
#pragma unroll
      for (int j = 0; j + 1 < NC; j += 2)
        dp = mfma2(lds4(&gs[r0 + l32][8 * j + 4 * half]), lds4(&gs[r0 + l32][8 * j + 8 + 4 * half]),
                   vbv[j], vbv[j + 1], dp);
      if constexpr (DROP) {
        if constexpr (NC % 2) dp = mfma(lds4(&gs[r0 + l32][8 * (NC - 1) + 4 * half]), vbv[NC - 1], dp);
      } else if constexpr (NC % 2) {
        dp = mfma2(lds4(&gs[r0 + l32][8 * (NC - 1) + 4 * half]), xa, vbv[NC - 1], ones_d, dp);
      } else {
        dp = mfma(xa, ones_d, dp);
      }
      s16x4 pa[4], dsa[4];  // P^T and dS^T as A operands: A[key][query step row]
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = r0 + 8 * j + 4 * half;  // rows r .. r+3 of this K step
        const float p0 = __builtin_amdgcn_exp2f(st[4 * j]);
        const float p1 = __builtin_amdgcn_exp2f(st[4 * j + 1]);
        const float p2 = __builtin_amdgcn_exp2f(st[4 * j + 2]);
        const float p3 = __builtin_amdgcn_exp2f(st[4 * j + 3]);
        if constexpr (DROP) {
          // this lane's key with queries qb + r .. +3: one word per element
          const float4 dv4 = *reinterpret_cast<const float4*>(&dd[r]);  // -D
          const uint32_t qr = uint32_t(qb + r), kk = uint32_t(kj);
          const float m0 = drop_scale(dm, drop_word(dm, qr, kk), kk);
          const float m1 = drop_scale(dm, drop_word(dm, qr + 1, kk), kk);
          const float m2 = drop_scale(dm, drop_word(dm, qr + 2, kk), kk);
          const float m3 = drop_scale(dm, drop_word(dm, qr + 3, kk), kk);
          pa[j] = pack4(p0 * m0, p1 * m1, p2 * m2, p3 * m3);
          dsa[j] = pack4(p0 * fmaf(m0, dp[4 * j], dv4.x), p1 * fmaf(m1, dp[4 * j + 1], dv4.y),
                         p2 * fmaf(m2, dp[4 * j + 2], dv4.z), p3 * fmaf(m3, dp[4 * j + 3], dv4.w));
        } else {
          pa[j] = pack4(p0, p1, p2, p3);
          dsa[j] = pack4(p0 * dp[4 * j], p1 * dp[4 * j + 1], p2 * dp[4 * j + 2], p3 * dp[4 * j + 3]);
        }
      }
      s16x4 gb[4], qbq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c0 = r0 + 8 * j + 4 * half;
        gb[j] = lds4(&gt[l32][c0]);
        qbq[j] = lds4(&qt[l32][c0]);
      }
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        dv = mfma2(pa[j], pa[j + 1], gb[j], gb[j + 1], dv);
        dk = mfma2(dsa[j], dsa[j + 1], qbq[j], qbq[j + 1], dk);
      }
    }
  }
  // D[key][c] -> grad rows; lane holds column c = l32 of 16 key rows.
  if (l32 >= DH) return;
  const int64_t k0 = int64_t(wg_x()) * kRowsPerBlock + wave * kT;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t key = k0 + 8 * (i / 4) + 4 * half + (i % 4);
    if (key < n_k) {
      grad_k[(key * H + h) * DH + l32].x = f32_to_bf16(dk[i] * scale);
      grad_v[(key * H + h) * DH + l32].x = f32_to_bf16(dv[i]);
    }
  }
}

// D[h][q] = sum_c G[q][h][c] o[q][h][c] (o the forward's fp32 output when
// it kept one, else the bf16 output), one thread per (query, head), with
// k_mf_bwd_q's arithmetic: each half's 4-column groups j = 0 .. NC-1 as one
// fmaf chain, then the two halves' sums added.  The single-pass backward
// reads it as k_mf_bwd_kv does.
template <int DH>
__global__ __launch_bounds__(kBlock) void k_mf_dsum(const bf16_t* __restrict__ g,
                                                    const bf16_t* __restrict__ out,
                                                    const float* __restrict__ out32, int32_t n_q,
                                                    int32_t H, float* __restrict__ dsum) {
  constexpr int NC = DH / 8;
  const int64_t t = int64_t(wg_x()) * kBlock + tid_x();
  if (t >= int64_t(n_q) * H) return;
  const int64_t qi = t / H;
  const int h = int(t - qi * H);
  const int64_t row = (qi * H + h) * DH;
  float part[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t o = row + 8 * j + 4 * half;
      const s16x4 gb = load4(g + o);
      float ov[4];
      if (out32) {
        const float4 f = *reinterpret_cast<const float4*>(out32 + o);
        ov[0] = f.x, ov[1] = f.y, ov[2] = f.z, ov[3] = f.w;
      } else {
        const s16x4 ob = load4(out + o);
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = bf16_to_f32(static_cast<uint16_t>(ob[i]));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) a = fmaf(bf16_to_f32(static_cast<uint16_t>(gb[i])), ov[i], a);
    }
    part[half] = a;
  }
  dsum[int64_t(h) * n_q + qi] = part[0] + part[1];
}

// Single-pass backward, key-major: dK and dV as k_mf_bwd_kv, and each score
// tile's dS, already packed to bf16 for dK, is also contracted with the
// wave's own K rows into a partial dQ, so the exponentials are computed once
// instead of once per pass.  dS crosses lanes through a wave-private LDS tile
// (written one key per lane, read one query per lane as the MFMA's A
// operand).  Within a block the 4 waves' partials of a query sub-tile are
// added in a fixed order: in step t of a stage, wave w takes sub-tile
// (w + t) mod 4, so each step's waves touch distinct sub-tiles, and sub-tile
// s collects waves s, s-1, s-2, s-3 (mod 4) in that order as the accumulator
// input of their MFMAs, a block barrier between steps.  At the end of a stage
// the block's partial dQ over its 128 keys goes to part_dq[block][q][h][c];
// k_mf_dq_combine adds the blocks' partials in block order.
constexpr int kTrPad = 4;  // shorts: rows of 72 bytes
template <int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_mf_bwd_fused(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ g, const float* __restrict__ lse, const float* __restrict__ dsum,
    int32_t n_q, int32_t n_k, int32_t H, float scale, DropoutMask dm,
    bf16_t* __restrict__ grad_k, bf16_t* __restrict__ grad_v, float* __restrict__ part_dq) {
  constexpr int NC = DH / 8;
  constexpr int kSubs = kSB / kT;  // query sub-tiles per stage (= waves per block)
  static_assert(kSubs == kWaves, "one sub-tile per wave and step");
  __shared__ __align__(16) short qs[kSB][DH + kRowPad];
  __shared__ __align__(16) short gs[kSB][DH + kRowPad];
  __shared__ __align__(16) short qt[kT][kSB + kColPad];  // rows >= DH zero
  __shared__ __align__(16) short gt[kT][kSB + kColPad];
  __shared__ __align__(16) uint2 xr[2][kSB];
  __shared__ __align__(16) float dd[kSB];               // -D, with dropout only
  __shared__ __align__(16) short tr[kWaves][kT][kT + kTrPad];  // a wave's dS tile, [q][key]
  // the stage's partial dQ per sub-tile in the MFMA's D layout:
  // [sub][row group u][half][c][4 rows], so a lane's 16-byte accesses of one u
  // are 16 bytes apart.  Lanes of columns c >= DH (zeros, never stored) all
  // use the spare column DH, so every lane takes the same path.
  __shared__ __align__(16) float red[kSubs][4][2][DH + 1][4];
  const int lane = tid_x() & (kWave - 1);
  const int wave = tid_x() >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int h = wg_y();
  const int64_t k0 = int64_t(wg_x()) * kRowsPerBlock + wave * kT;
  const int64_t kj = k0 + l32;
  const bool k_ok = kj < n_k;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  s16x4 kbv[NC], vbv[NC];  // K^T, V^T as B operands
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    kbv[j] = settle(k_ok ? load4(k + (kj * H + h) * DH + 8 * j + 4 * half) : zero4());
    vbv[j] = settle(k_ok ? load4(v + (kj * H + h) * DH + 8 * j + 4 * half) : zero4());
  }
  // this wave's K rows as the B operand of dQ += dS K: lane (c = l32, half)
  // holds K[k0 + 8j + 4 half + i][c] (zero for c >= DH and keys past n_k)
  s16x4 kq[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t key = k0 + 8 * j + 4 * half + i;
      kq[j][i] = (l32 < DH && key < n_k) ? static_cast<short>(k[(key * H + h) * DH + l32].x)
                                         : static_cast<short>(0);
    }
    kq[j] = settle(kq[j]);
  }
  const float s2 = scale * kLog2e;
  s16x4 khi[NC], klo[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) split_scaled(kbv[j], s2, khi[j], klo[j]);
  const s16x4 ones_l = ones3(half, 0), ones_d = ones3(half, 1);
  f32x16 dk = zero16(), dv = zero16();
  Stage<DH> pq, pg;
  float pl = 0.f, pd = 0.f;
  auto prefetch = [&](int qb) {
    pq.load(q, qb, n_q, H, h);
    pg.load(g, qb, n_q, H, h);
    if (tid_x() < kSB) {
      const bool ok = qb + int(tid_x()) < n_q;
      pl = ok ? lse[int64_t(h) * n_q + qb + tid_x()] : INFINITY;
      pd = ok ? dsum[int64_t(h) * n_q + qb + tid_x()] : 0.f;
    }
  };
  fill_pad_rows<DH>(qt, false);
  fill_pad_rows<DH>(gt, false);
  short (*T)[kT + kTrPad] = tr[wave];
  const int rc = l32 < DH ? l32 : DH;  // this lane's column of red
  prefetch(0);
  for (int qb = 0; qb < n_q; qb += kSB) {
    __syncthreads();
    pq.store_rows(qs);
    pg.store_rows(gs);
    pq.store_trans(qt);
    pg.store_trans(gt);
    if (tid_x() < kSB) {
      const float nl = pl == INFINITY ? -1e30f : -pl * kLog2e;
      xr[0][tid_x()] = split3(nl);
      xr[1][tid_x()] = split3(-pd);
      if constexpr (DROP) dd[tid_x()] = -pd;
    }
    __syncthreads();
    if (qb + kSB < n_q) prefetch(qb + kSB);
    // not unrolled: unrolled, the steps' operands stay live across them (162 -> 180 VGPRs)
#pragma unroll 1
    for (int step = 0; step < kSubs; ++step) {
      const int sub = (wave + step) & (kSubs - 1);
      if (qb + sub * kT < n_q) {  // uniform per wave; every wave meets the barrier below
        const int r0 = sub * kT;
        const s16x4 xa = __builtin_bit_cast(s16x4, xr[half][r0 + l32]);
        f32x16 st = zero16(), dp = zero16();
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          const s16x4 qa = lds4(&qs[r0 + l32][8 * j + 4 * half]);
          st = mfma2(qa, qa, khi[j], klo[j], st);
        }
        st = mfma(xa, ones_l, st);
#pragma unroll
        for (int j = 0; j + 1 < NC; j += 2)
          dp = mfma2(lds4(&gs[r0 + l32][8 * j + 4 * half]),
                     lds4(&gs[r0 + l32][8 * j + 8 + 4 * half]), vbv[j], vbv[j + 1], dp);
        if constexpr (DROP) {
          if constexpr (NC % 2)
            dp = mfma(lds4(&gs[r0 + l32][8 * (NC - 1) + 4 * half]), vbv[NC - 1], dp);
        } else if constexpr (NC % 2) {
          dp = mfma2(lds4(&gs[r0 + l32][8 * (NC - 1) + 4 * half]), xa, vbv[NC - 1], ones_d, dp);
        } else {
          dp = mfma(xa, ones_d, dp);
        }
        s16x4 pa[4], dsa[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = r0 + 8 * j + 4 * half;
          const float p0 = __builtin_amdgcn_exp2f(st[4 * j]);
          const float p1 = __builtin_amdgcn_exp2f(st[4 * j + 1]);
          const float p2 = __builtin_amdgcn_exp2f(st[4 * j + 2]);
          const float p3 = __builtin_amdgcn_exp2f(st[4 * j + 3]);
          if constexpr (DROP) {
            const float4 dv4 = *reinterpret_cast<const float4*>(&dd[r]);  // -D
            const uint32_t qr = uint32_t(qb + r), kk = uint32_t(kj);
            const float m0 = drop_scale(dm, drop_word(dm, qr, kk), kk);
            const float m1 = drop_scale(dm, drop_word(dm, qr + 1, kk), kk);
            const float m2 = drop_scale(dm, drop_word(dm, qr + 2, kk), kk);
            const float m3 = drop_scale(dm, drop_word(dm, qr + 3, kk), kk);
            pa[j] = pack4(p0 * m0, p1 * m1, p2 * m2, p3 * m3);
            dsa[j] = pack4(p0 * fmaf(m0, dp[4 * j], dv4.x), p1 * fmaf(m1, dp[4 * j + 1], dv4.y),
                           p2 * fmaf(m2, dp[4 * j + 2], dv4.z), p3 * fmaf(m3, dp[4 * j + 3], dv4.w));
          } else {
            pa[j] = pack4(p0, p1, p2, p3);
            dsa[j] = pack4(p0 * dp[4 * j], p1 * dp[4 * j + 1], p2 * dp[4 * j + 2],
                           p3 * dp[4 * j + 3]);
          }
        }
        // dS (queries r0 + 8j + 4 half + i, this lane's key) -> T[query][key]
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) T[8 * j + 4 * half + i][l32] = dsa[j][i];
        s16x4 gb[4], qbq[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c0 = r0 + 8 * j + 4 * half;
          gb[j] = lds4(&gt[l32][c0]);
          qbq[j] = lds4(&qt[l32][c0]);
        }
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
          dv = mfma2(pa[j], pa[j + 1], gb[j], gb[j + 1], dv);
          dk = mfma2(dsa[j], dsa[j + 1], qbq[j], qbq[j + 1], dk);
        }
        // partial dQ of this sub-tile over the wave's keys, on top of the
        // waves before it: A = dS[query][key] read back from T (a wave's own
        // LDS writes and reads complete in order), B = kq
        s16x4 ta[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ta[j] = lds4(&T[l32][8 * j + 4 * half]);
        f32x16 acc;
        if (step == 0) {  // uniform: the first wave of this sub-tile starts the sum
          acc = mfma2(ta[0], ta[1], kq[0], kq[1], zero16());
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float4 f = *reinterpret_cast<const float4*>(&red[sub][u][half][rc][0]);
            acc[4 * u] = f.x, acc[4 * u + 1] = f.y, acc[4 * u + 2] = f.z, acc[4 * u + 3] = f.w;
          }
          acc = mfma2(ta[0], ta[1], kq[0], kq[1], acc);
        }
        acc = mfma2(ta[2], ta[3], kq[2], kq[3], acc);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          *reinterpret_cast<float4*>(&red[sub][u][half][rc][0]) =
              make_float4(acc[4 * u], acc[4 * u + 1], acc[4 * u + 2], acc[4 * u + 3]);
      }
      __syncthreads();
    }
    // the block's partial dQ over its keys for this stage's queries
    const int nvalid = min(kSB, n_q - qb);
    float* pz = part_dq + int64_t(wg_x()) * n_q * H * DH;
    for (int e = tid_x(); e < nvalid * DH; e += kBlock) {
      const int r = e / DH, c = e - (e / DH) * DH;
      const int sb = r / kT, rr = r - sb * kT;  // D row rr = 8 u + 4 half + i, i < 4
      pz[(int64_t(qb + r) * H + h) * DH + c] = red[sb][rr >> 3][(rr >> 2) & 1][c][rr & 3];
    }
  }
  if (l32 >= DH) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t key = k0 + 8 * (i / 4) + 4 * half + (i % 4);
    if (key < n_k) {
      grad_k[(key * H + h) * DH + l32].x = f32_to_bf16(dk[i] * scale);
      grad_v[(key * H + h) * DH + l32].x = f32_to_bf16(dv[i]);
    }
  }
}

// Query-major: dQ for queries q0 .. q0+31.  S^T, dP^T as D[key][q]; K and V
// stages of 128 keys in LDS (row-major for the A operands, K^T for dQ += dS K).
// This pass runs first in the backward and forms each query's
// D = sum_c G o itself (o the forward's fp32 output when it kept one, else the
// bf16 output: D enters dS = P (dP - D) where the two terms nearly cancel for
// peaked rows, and the rounded output alone moves dQ by a few percent there);
// the blocks of key split 0 store it in dsum for the key-major pass.
template <int DH, bool DROP>
__global__ __launch_bounds__(kBlock) void k_mf_bwd_q(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ g, const bf16_t* __restrict__ out, const float* __restrict__ out32,
    const float* __restrict__ lse, float* __restrict__ dsum, int32_t n_q, int32_t n_k, int32_t H,
    float scale, DropoutMask dm, bf16_t* __restrict__ grad_q, int32_t split_keys,
    float* __restrict__ part_dq) {
  constexpr int NC = DH / 8;
  __shared__ __align__(16) short ks[kSB][DH + kRowPad];
  __shared__ __align__(16) short vs[kSB][DH + kRowPad];
  __shared__ __align__(16) short kt[kT][kSB + kColPad];  // rows >= DH zero
  const int lane = tid_x() & (kWave - 1);
  const int wave = tid_x() >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int h = wg_y();
  const int64_t qi = int64_t(wg_x()) * kRowsPerBlock + wave * kT + l32;
  const bool q_ok = qi < n_q;
  if constexpr (DROP) dm = drop_for_head(dm, h);
  s16x4 qbv[NC], gbv[NC];  // Q^T, G^T as B operands
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    qbv[j] = settle(q_ok ? load4(q + (qi * H + h) * DH + 8 * j + 4 * half) : zero4());
    gbv[j] = settle(q_ok ? load4(g + (qi * H + h) * DH + 8 * j + 4 * half) : zero4());
  }
  const float L2 = q_ok ? lse[int64_t(h) * n_q + qi] * kLog2e : INFINITY;
  // D: this lane's 4 * NC columns in order, then the other half's
  float dpart = 0.f;
  if (q_ok) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t o = (qi * H + h) * DH + 8 * j + 4 * half;
      float ov[4];
      if (out32) {
        const float4 f = *reinterpret_cast<const float4*>(out32 + o);
        ov[0] = f.x, ov[1] = f.y, ov[2] = f.z, ov[3] = f.w;
      } else {
        const s16x4 ob = load4(out + o);
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = bf16_to_f32(static_cast<uint16_t>(ob[i]));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dpart = fmaf(bf16_to_f32(static_cast<uint16_t>(gbv[j][i])), ov[i], dpart);
    }
  }
  const float Dq = sum_halves(dpart);
  if (wg_z() == 0 && half == 0 && q_ok) dsum[int64_t(h) * n_q + qi] = Dq;
  const float s2 = scale * kLog2e;
  // S^T s2 - L and dP^T - D come straight out of the MFMAs: Q^T s2 as hi ++ lo
  // operands (the K rows read once, fed twice), the lane's -L as the
  // accumulator input of every S tile, and its -D pieces as one more K step
  // of dP against constant ones.  Padded queries: -L = -inf (p = 0) and D = 0
  // with zero G rows (dP = 0).
  s16x4 qhi[NC], qlo[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) split_scaled(qbv[j], s2, qhi[j], qlo[j]);
  const f32x16 st0 = fill16(-L2);
  const s16x4 ones_a = ones3(half, 0);
  const s16x4 db = half == 0 ? __builtin_bit_cast(s16x4, split3(-Dq)) : zero4();
  f32x16 dq = zero16();  // D[q][c]: q = 8*(i/4)+4*half+i%4 (tile row), c = l32
  const int k_begin = wg_z() * split_keys;  // this block's key split
  const int k_end = min(n_k, k_begin + split_keys);
  fill_pad_rows<DH>(kt, false);
  Stage<DH> pk, pv;
  pk.load(k, k_begin, k_end, H, h);
  pv.load(v, k_begin, k_end, H, h);
  for (int kb = k_begin; kb < k_end; kb += kSB) {
    __syncthreads();
    pk.store_rows(ks);
    pv.store_rows(vs);
    pk.store_trans(kt);
    __syncthreads();
    if (kb + kSB < k_end) {
      pk.load(k, kb + kSB, k_end, H, h);
      pv.load(v, kb + kSB, k_end, H, h);
    }
    for (int sub = 0; sub < kSB / kT && kb + sub * kT < k_end; ++sub) {
      const int r0 = sub * kT;
      f32x16 st = st0, dp = zero16();  // -> S^T s2 - L, dP^T - D (dP^T with dropout)
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const s16x4 ka = lds4(&ks[r0 + l32][8 * j + 4 * half]);
        st = mfma2(ka, ka, qhi[j], qlo[j], st);
      }
#pragma unroll
      for (int j = 0; j + 1 < NC; j += 2)
        dp = mfma2(lds4(&vs[r0 + l32][8 * j + 4 * half]), lds4(&vs[r0 + l32][8 * j + 8 + 4 * half]),
                   gbv[j], gbv[j + 1], dp);
      if constexpr (DROP) {
        if constexpr (NC % 2) dp = mfma(lds4(&vs[r0 + l32][8 * (NC - 1) + 4 * half]), gbv[NC - 1], dp);
      } else if constexpr (NC % 2) {
        dp = mfma2(lds4(&vs[r0 + l32][8 * (NC - 1) + 4 * half]), ones_a, gbv[NC - 1], db, dp);
      } else {
        dp = mfma(ones_a, db, dp);
      }
      if constexpr (DROP) {  // dP o M - D: keys kb + r0 + 8*(i/4) + 4*half + i%4
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const uint32_t key = uint32_t(kb + r0 + 8 * (i / 4) + 4 * half + (i % 4));
          const uint32_t w = drop_word(dm, uint32_t(qi), key);
          dp[i] = fmaf(dp[i], drop_scale(dm, w, key), -Dq);
          dp[i + 1] = fmaf(dp[i + 1], drop_scale(dm, w, key + 1), -Dq);
        }
      }
      float ds[16];
      if (kb + r0 + kT <= k_end) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ds[i] = __builtin_amdgcn_exp2f(st[i]) * dp[i];
      } else {  // tail tile: keys past the split's end drop out
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb + r0 + 8 * (i / 4) + 4 * half + (i % 4);
          ds[i] = key < k_end ? __builtin_amdgcn_exp2f(st[i]) * dp[i] : 0.f;
        }
      }
      s16x4 dsa[4];  // dS as A operand: A[q][key step row] from the D[key][q] layout
#pragma unroll
      for (int j = 0; j < 4; ++j) dsa[j] = pack4(ds[4 * j], ds[4 * j + 1], ds[4 * j + 2], ds[4 * j + 3]);
      s16x4 kbk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) kbk[j] = lds4(&kt[l32][r0 + 8 * j + 4 * half]);
#pragma unroll
      for (int j = 0; j < 4; j += 2) dq = mfma2(dsa[j], dsa[j + 1], kbk[j], kbk[j + 1], dq);
    }
  }
  if (l32 >= DH) return;
  const int64_t q0 = int64_t(wg_x()) * kRowsPerBlock + wave * kT;
  if (part_dq) {  // this split's dQ, unscaled fp32; the splits are added in order afterwards
    float* pz = part_dq + int64_t(wg_z()) * n_q * H * DH;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t qq = q0 + 8 * (i / 4) + 4 * half + (i % 4);
      if (qq < n_q) pz[(qq * H + h) * DH + l32] = dq[i];
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t qq = q0 + 8 * (i / 4) + 4 * half + (i % 4);
    if (qq < n_q) grad_q[(qq * H + h) * DH + l32].x = f32_to_bf16(dq[i] * scale);
  }
}

// grad_q = scale * sum of the key splits' partial dQ, added in split order
// (kernel: a grid of its own, used when no dK/dV launch follows).
__global__ __launch_bounds__(kBlock) void k_mf_dq_combine(const float* __restrict__ part,
                                                          int32_t n_split, int64_t n,
                                                          float scale,
                                                          bf16_t* __restrict__ grad_q,
                                                          int32_t n_blocks) {
  dq_combine(part, n_split, n, scale, grad_q, wg_x(), n_blocks);
}

}  // namespace

// Launchers used by ngt_dense.hip for bf16 and d in {8, 16, 24, 32}.
bool mfma_dense_supported(int d) { return d == 8 || d == 16 || d == 24 || d == 32; }

// Key splits: the forward (one wave per 32 queries and head, all keys) and
// the dQ pass have grids of ceil(n_q / 32) * H waves, about 4 per SIMD at
// 16,000 queries and 8 heads, while their registers leave room for more.
// Splitting the keys over the grid's z dimension raises the waves per SIMD; each split's
// state is merged afterwards in split order.  Measured at 16,000 nodes, 8
// heads, d = 8 with the per-score arithmetic in the MFMAs (us per launch):
// forward alone 331 / 325 / 324 / 329 / 334 at 2 / 3 / 4 / 6 / 8 splits plus a
// 7-13 us combine; dQ 348 / 337 / 334 / 332 / 335 at 1 / 2 / 3 / 4 / 6.  When
// the column-score blocks share the forward's launch they bring as many waves
// again, and one split is best: 384 us for forward and scores against 392 us
// plus the combine at 2 splits.  `shared_waves` counts such other waves.
// What bounds these kernels is the per-score VALU work (an exponential, a
// pack and, in the backward, a product per score) at 4-5 waves per SIMD;
// issuing the next tile's products ahead of the current tile's softmax work
// costs registers (one wave less per SIMD) and measured slower: forward
// 406 -> 432 us, dK/dV 479 -> 585 us.
// NGT_MF_FWD_SPLIT / NGT_MF_DQ_SPLIT override the count.
static MfSplit plan_split(int n_q, int n_k, int H, int target_waves, int64_t shared_waves,
                          const char* env) {
  const int64_t base = int64_t((n_q + kRowsPerBlock - 1) / kRowsPerBlock) * H * kWaves;
  const int64_t room = std::max<int64_t>(target_waves - shared_waves, 0);
  int want = base > 0 ? int((room + base / 2) / base) : 1;
  if (const char* e = getenv(env)) want = atoi(e);
  want = std::max(1, std::min({want, 8, std::max(1, n_k / 512)}));
  if (want <= 1 || n_k <= 0) return {1, std::max(n_k, 1)};
  int keys = (n_k + want - 1) / want;
  keys = (keys + kSB - 1) / kSB * kSB;
  return {(n_k + keys - 1) / keys, keys};
}
MfSplit mfma_fwd_split(int n_q, int n_k, int H, bool node_scores) {
  const int64_t score_waves =
      node_scores ? int64_t((n_k + kRowsPerBlock - 1) / kRowsPerBlock) * H * kWaves : 0;
  return plan_split(n_q, n_k, H, 6144, score_waves, "NGT_MF_FWD_SPLIT");
}
MfSplit mfma_dq_split(int n_q, int n_k, int H) {
  return plan_split(n_q, n_k, H, 12288, 0, "NGT_MF_DQ_SPLIT");
}

// The single-pass backward (k_mf_bwd_fused) or the two passes: the number of
// 128-key blocks whose partial dQ the backward workspace holds, 0 for the two
// passes.  Two passes by default: at 16,000 nodes, 8 heads, d = 8 the single
// pass measured 991 us plus a 136 us combine of its 512 MB of partials
// against 470 + 324 us (162 VGPRs, 3 waves per SIMD, against 114 and 4;
// forced to 4 waves per SIMD, 30 VGPRs spilled, 923 us: the block's
// lockstep steps and each step's LDS round trips lengthen a tile's chain).
// NGT_DENSE_FUSED=1 turns it on.
int mfma_fused_blocks(int n_q, int n_k, int H, int d) {
  (void)H;
  (void)d;
  if (n_q <= 0 || n_k < kSB) return 0;
  bool on = false;
  if (const char* e = getenv("NGT_DENSE_FUSED")) on = atoi(e) != 0;
  return on ? (n_k + kRowsPerBlock - 1) / kRowsPerBlock : 0;
}

template <int DH>
static int mf_fwd(const void* q, const void* k, const void* v, int n_q, int n_k, int H,
                  float scale, const DropoutMask* dm, void* out, float* out32, float* lse,
                  float* part, MfSplit sp, float* part_ml, float* part_acc, hipStream_t st) {
  const int fwd_bx = (n_q + kRowsPerBlock - 1) / kRowsPerBlock;
  const int score_bx = part && n_k > 0 ? (n_k + kRowsPerBlock - 1) / kRowsPerBlock : 0;
  const dim3 grid(std::max(fwd_bx, score_bx), H, sp.n_split + (score_bx > 0 ? 1 : 0));
  float* pml = sp.n_split > 1 ? part_ml : nullptr;
  float* pacc = sp.n_split > 1 ? part_acc : nullptr;
  // one launch: the forward and, when wanted, the column scores
  KernelTimer timer_("dense_fwd", st);
  const DropoutMask m = dm ? *dm : DropoutMask{};
  if (dm)
    hipLaunchKernelGGL((k_mf_fwd<DH, true>), grid, dim3(kBlock), 0, st,
                       static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                       static_cast<const bf16_t*>(v), n_q, n_k, H, scale, m,
                       static_cast<bf16_t*>(out), out32, lse, sp.split_keys, pml, pacc,
                       sp.n_split, fwd_bx, score_bx, part);
  else
    hipLaunchKernelGGL((k_mf_fwd<DH, false>), grid, dim3(kBlock), 0, st,
                       static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                       static_cast<const bf16_t*>(v), n_q, n_k, H, scale, m,
                       static_cast<bf16_t*>(out), out32, lse, sp.split_keys, pml, pacc,
                       sp.n_split, fwd_bx, score_bx, part);
  NGT_HIP_CHECK(hipGetLastError());
  return NGT_OK;
}

// The single-pass backward: D, then dK/dV with the blocks' partial dQ, then
// dQ as the partials' sum in block order.
template <int DH>
static int mf_bwd_fused(const void* q, const void* k, const void* v, const void* g,
                        const void* out, const float* out32, const float* lse, float* dsum,
                        int n_q, int n_k, int H, float scale, const DropoutMask* dm, void* gq,
                        void* gk, void* gv, int kv_bx, float* part, hipStream_t st) {
  {
    KernelTimer timer_("dense_dsum", st);
    const int64_t nrh = int64_t(n_q) * H;
    hipLaunchKernelGGL((k_mf_dsum<DH>), dim3(unsigned((nrh + kBlock - 1) / kBlock)), dim3(kBlock),
                       0, st, static_cast<const bf16_t*>(g), static_cast<const bf16_t*>(out), out32,
                       n_q, H, dsum);
    NGT_HIP_CHECK(hipGetLastError());
  }
  {
    KernelTimer timer_("dense_bwd_fused", st);
    const DropoutMask m = dm ? *dm : DropoutMask{};
    const dim3 grid(kv_bx, H);
    if (dm)
      hipLaunchKernelGGL((k_mf_bwd_fused<DH, true>), grid, dim3(kBlock), 0, st,
                         static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                         static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g), lse, dsum,
                         n_q, n_k, H, scale, m, static_cast<bf16_t*>(gk), static_cast<bf16_t*>(gv),
                         part);
    else
      hipLaunchKernelGGL((k_mf_bwd_fused<DH, false>), grid, dim3(kBlock), 0, st,
                         static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                         static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g), lse, dsum,
                         n_q, n_k, H, scale, m, static_cast<bf16_t*>(gk), static_cast<bf16_t*>(gv),
                         part);
    NGT_HIP_CHECK(hipGetLastError());
  }
  {
    KernelTimer timer_("dense_dq_combine", st);
    const int64_t n_dq = int64_t(n_q) * H * DH;
    const unsigned blocks = unsigned(std::min<int64_t>((n_dq + kBlock - 1) / kBlock, 65536));
    hipLaunchKernelGGL(k_mf_dq_combine, dim3(blocks), dim3(kBlock), 0, st, part, kv_bx, n_dq,
                       scale, static_cast<bf16_t*>(gq), int32_t(blocks));
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

// The backward in two launches: the dQ pass (which also stores D), then the
// dK/dV pass (which reads it), carrying the dQ splits' merge in extra blocks.
template <int DH>
static int mf_bwd(const void* q, const void* k, const void* v, const void* g, const void* out,
                  const float* out32, const float* lse, float* dsum, int n_q, int n_k, int H,
                  float scale, const DropoutMask* dm, void* gq, void* gk, void* gv, MfSplit sq,
                  float* part_dq, hipStream_t st) {
  const DropoutMask m = dm ? *dm : DropoutMask{};
  float* pdq = n_q > 0 && sq.n_split > 1 ? part_dq : nullptr;
  if (n_q > 0) {
    KernelTimer timer_("dense_bwd_q", st);
    const dim3 grid((n_q + kRowsPerBlock - 1) / kRowsPerBlock, H, sq.n_split);
    if (dm)
      hipLaunchKernelGGL((k_mf_bwd_q<DH, true>), grid, dim3(kBlock), 0, st,
                         static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                         static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g),
                         static_cast<const bf16_t*>(out), out32, lse, dsum, n_q, n_k, H, scale, m,
                         static_cast<bf16_t*>(gq), sq.split_keys, pdq);
    else
      hipLaunchKernelGGL((k_mf_bwd_q<DH, false>), grid, dim3(kBlock), 0, st,
                         static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                         static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g),
                         static_cast<const bf16_t*>(out), out32, lse, dsum, n_q, n_k, H, scale, m,
                         static_cast<bf16_t*>(gq), sq.split_keys, pdq);
    NGT_HIP_CHECK(hipGetLastError());
  }
  const int64_t n_dq = int64_t(n_q) * H * DH;
  if (n_k > 0) {
    KernelTimer timer_("dense_bwd_kv", st);
    const int kv_bx = (n_k + kRowsPerBlock - 1) / kRowsPerBlock;
    // merge blocks per head: about 4 elements per thread
    const int cbx = pdq ? int((n_dq + int64_t(4) * kBlock * H - 1) / (int64_t(4) * kBlock * H)) : 0;
    const dim3 grid(kv_bx + cbx, H);
    if (dm)
      hipLaunchKernelGGL((k_mf_bwd_kv<DH, true>), grid, dim3(kBlock), 0, st,
                         static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                         static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g), lse, dsum,
                         n_q, n_k, H, scale, m, static_cast<bf16_t*>(gk), static_cast<bf16_t*>(gv),
                         kv_bx, cbx, pdq, sq.n_split, static_cast<bf16_t*>(gq));
    else
      hipLaunchKernelGGL((k_mf_bwd_kv<DH, false>), grid, dim3(kBlock), 0, st,
                         static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
                         static_cast<const bf16_t*>(v), static_cast<const bf16_t*>(g), lse, dsum,
                         n_q, n_k, H, scale, m, static_cast<bf16_t*>(gk), static_cast<bf16_t*>(gv),
                         kv_bx, cbx, pdq, sq.n_split, static_cast<bf16_t*>(gq));
    NGT_HIP_CHECK(hipGetLastError());
  } else if (pdq) {  // no dK/dV launch to carry the merge
    KernelTimer timer_("dense_dq_combine", st);
    const unsigned blocks = unsigned(std::min<int64_t>((n_dq + kBlock - 1) / kBlock, 65536));
    hipLaunchKernelGGL(k_mf_dq_combine, dim3(blocks), dim3(kBlock), 0, st, pdq, sq.n_split, n_dq,
                       scale, static_cast<bf16_t*>(gq), int32_t(blocks));
    NGT_HIP_CHECK(hipGetLastError());
  }
  return NGT_OK;
}

int mfma_dense_fwd(int d, const void* q, const void* k, const void* v, int n_q, int n_k, int H,
                   float scale, const DropoutMask* dm, void* out, float* out32, float* lse,
                   float* part, MfSplit sp, float* part_ml, float* part_acc, hipStream_t st) {
  switch (d) {
    case 8: return mf_fwd<8>(q, k, v, n_q, n_k, H, scale, dm, out, out32, lse, part, sp, part_ml, part_acc, st);
    case 16: return mf_fwd<16>(q, k, v, n_q, n_k, H, scale, dm, out, out32, lse, part, sp, part_ml, part_acc, st);
    case 24: return mf_fwd<24>(q, k, v, n_q, n_k, H, scale, dm, out, out32, lse, part, sp, part_ml, part_acc, st);
    case 32: return mf_fwd<32>(q, k, v, n_q, n_k, H, scale, dm, out, out32, lse, part, sp, part_ml, part_acc, st);
    default: return set_error(NGT_ERR_UNSUPPORTED, "mfma dense: head_dim %d", d);
  }
}

int mfma_dense_bwd(int d, const void* q, const void* k, const void* v, const void* g,
                   const void* out, const float* out32, const float* lse, float* dsum, int n_q,
                   int n_k, int H, float scale, const DropoutMask* dm, void* gq, void* gk, void* gv,
                   MfSplit sq, float* part_dq, int fused_blocks, hipStream_t st) {
#define NGT_MF_BWD(DH)                                                                      \
  case DH:                                                                                  \
    if (fused_blocks > 0)                                                                   \
      return mf_bwd_fused<DH>(q, k, v, g, out, out32, lse, dsum, n_q, n_k, H, scale, dm, gq, \
                              gk, gv, fused_blocks, part_dq, st);                           \
    return mf_bwd<DH>(q, k, v, g, out, out32, lse, dsum, n_q, n_k, H, scale, dm, gq, gk, gv, \
                      sq, part_dq, st);
  switch (d) {
    NGT_MF_BWD(8)
    NGT_MF_BWD(16)
    NGT_MF_BWD(24)
    NGT_MF_BWD(32)
    default: return set_error(NGT_ERR_UNSUPPORTED, "mfma dense: head_dim %d", d);
  }
#undef NGT_MF_BWD
}

}  // namespace ngt
