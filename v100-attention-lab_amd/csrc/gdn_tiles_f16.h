// fp16 operand helpers for the v_mfma_f32_16x16x32_f16 products of the
// 64-row forward scan and of the backward recurrences.
//
// Lane (r, kq) (r = lane % 16, kq = lane / 16) supplies row r of A and row r
// of B^T, 8 consecutive contraction indices 8 kq .. from each 32-block; the
// accumulator holds rows 4 kq + i, column r.  Inputs q, k, v, dO are exact
// in fp16 (bf16 values within the fp16 range); an fp32 operand is an fp16
// pair hi + lo, and a product of two fp32 values is hi*hi + hi*lo + lo*hi
// (to about 2^-22 relative).
#pragma once

#include "gdn_tiles_f32.h"

namespace gdn {
namespace tiles16 {

using namespace tiles;

constexpr int HP = 8;  // LDS row padding in halves (rows stay 16-byte aligned)

__device__ __forceinline__ f16x8 frag8(const f16* p) { return *reinterpret_cast<const f16x8*>(p); }
// the same 8 halves by two 8-byte reads (rows only 8-byte aligned)
__device__ __forceinline__ f16x8 frag8_2(const f16* p) {
  const f16x4 a = *reinterpret_cast<const f16x4*>(p), b = *reinterpret_cast<const f16x4*>(p + 4);
  return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// x as an fp16 pair hi + lo.
__device__ __forceinline__ void split_f16(float x, f16& hi, f16& lo) {
  x = pin(x);
  hi = (f16)x;
  lo = (f16)(x - (float)hi);
}

// 4 consecutive values as fp16 pairs: hi[0..3] and lo[0..3].
__device__ __forceinline__ void store_pair4(f16* hi, f16* lo, const float (&x)[4]) {
  f16 h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split_f16(x[i], h[i], l[i]);
  *reinterpret_cast<f16x4*>(hi) = f16x4{h[0], h[1], h[2], h[3]};
  *reinterpret_cast<f16x4*>(lo) = f16x4{l[0], l[1], l[2], l[3]};
}

// Row m0 + r of X^T, contraction indices t0 + 8 kq .. t0 + 8 kq + 7, from
// row-major X in LDS by two ds_read_b64_tr_b16: in each group of 16 lanes,
// lane i receives as element j halfword i % 4 of the 8 bytes addressed by
// lane 4 j + i / 4 of the group.  Lane (r, kq) addresses
// x[t0 + 8 kq + 4 h + r / 4][m0 + 4 (r % 4)] and so receives
// X[t0 + 8 kq + 4 h + j][m0 + r], j = 0..3, for h = 0, 1.
template <int LD>
__device__ __forceinline__ f16x8 frag8_t(const f16 (*x)[LD], int t0, int m0, int r, int kq) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const f16* const a0 = &x[t0 + 8 * kq + (r >> 2)][m0 + 4 * (r & 3)];
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a0);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a0 + 4 * LD));
  union {
    s16x4 h[2];
    f16x8 f;
  } u;
  u.h[0] = lo;
  u.h[1] = hi;
  return u.f;
}

// The same with 4 contraction indices t0 + 4 kq .. t0 + 4 kq + 3 (one
// ds_read_b64_tr_b16): lane (r, kq) receives X[t0 + 4 kq + j][m0 + r].
template <int LD>
__device__ __forceinline__ f16x4 frag4_t(const f16 (*x)[LD], int t0, int m0, int r, int kq) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const f16* const a0 = &x[t0 + 4 * kq + (r >> 2)][m0 + 4 * (r & 3)];
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a0));
}

// The loaders below load unconditionally, guarded at most by a wave-uniform
// test (none when the vectors fill every lane): a lane-masked load, a zero
// written into a register a load may still target, or a load that a later
// path may leave unconsumed, makes the wave wait for every load in flight.

// ROWS x COLS halves, rows `ld` halves apart in global memory -> LDS rows of
// LD halves, 16 bytes per lane (NT threads).
template <int ROWS, int COLS, int NT>
struct HalfRows {
  static constexpr int RV = COLS / 8, NV = ROWS * RV, N = (NV + NT - 1) / NT;
  static_assert(NV % 64 == 0, "whole waves");
  u32x4 r[N];
  __device__ __forceinline__ void load(int tid, const f16* src, int64_t ld) {
    const int w0 = __builtin_amdgcn_readfirstlane(tid & ~63);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      if (NV % NT == 0 || w0 + i * NT < NV) r[i] = *reinterpret_cast<const u32x4*>(src + (e / RV) * ld + (e % RV) * 8);
    }
  }
  template <int LD>
  __device__ __forceinline__ void store(int tid, f16 (*dst)[LD]) const {
    const int w0 = __builtin_amdgcn_readfirstlane(tid & ~63);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      if (NV % NT == 0 || w0 + i * NT < NV) *reinterpret_cast<u32x4*>(&dst[e / RV][(e % RV) * 8]) = r[i];
    }
  }
};

// ROWS x COLS block of a 16-bit input, row-major, in 8-element vectors
// (vector e: row e / RV), stored as fp16.  Rows >= nvalid (>= 1) load row
// nvalid - 1 and are stored as zero.
template <typename TIn, int ROWS, int COLS, int NT>
struct InRows {
  static constexpr int RV = COLS / 8, NV = ROWS * RV, N = (NV + NT - 1) / NT;
  static_assert(NV % 64 == 0, "whole waves");
  uint4 r[N];
  int nv;
  __device__ __forceinline__ void load(int tid, const TIn* src, int64_t ld, int nvalid) {
    const int w0 = __builtin_amdgcn_readfirstlane(tid & ~63);
    nv = nvalid;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      if (NV % NT == 0 || w0 + i * NT < NV)
        r[i] = *reinterpret_cast<const uint4*>(src + min(e / RV, nvalid - 1) * ld + 8 * (e % RV));
    }
  }
  template <int LD>
  __device__ __forceinline__ void store(int tid, f16 (*dst)[LD]) const {
    const int w0 = __builtin_amdgcn_readfirstlane(tid & ~63);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      if (NV % NT == 0 || w0 + i * NT < NV) {
        const bool ok = e / RV < nv;
        const uint4 v = {ok ? r[i].x : 0u, ok ? r[i].y : 0u, ok ? r[i].z : 0u, ok ? r[i].w : 0u};
        f16 x[8];
        InTraits<TIn>::to_op(v, x);
        *reinterpret_cast<f16x8*>(&dst[e / RV][8 * (e % RV)]) = f16x8{x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
      }
    }
  }
};

// A ROWS x COLS slice of a 16-bit input (a V or dO column slice), one pair
// of elements per lane (row lane / (COLS / 2)), stored transposed as fp16
// (dst[column][row]).  Rows >= nvalid (>= 1) load row nvalid - 1 and are
// stored as zero.
template <typename TIn, int ROWS, int COLS, int NT>
struct SlicePairs {
  static_assert(ROWS * COLS / 2 == NT, "one pair per lane");
  uint32_t r;
  int nv;
  __device__ __forceinline__ void load(int tid, const TIn* src, int64_t ld, int nvalid) {
    nv = nvalid;
    r = *reinterpret_cast<const uint32_t*>(src + min(tid / (COLS / 2), nvalid - 1) * ld + 2 * (tid % (COLS / 2)));
  }
  // bf16 values are multiplied by sc (a power of two: exact) before the
  // conversion; fp16 values are stored as they are.
  template <int LD>
  __device__ __forceinline__ void store(int tid, f16 (*dst)[LD], float sc = 1.f) const {
    const int t = tid / (COLS / 2), c = tid % (COLS / 2);
    const uint32_t v = t < nv ? r : 0u;
    const uint16_t l16 = (uint16_t)(v & 0xffffu), h16 = (uint16_t)(v >> 16);
    if constexpr (std::is_same<TIn, f16>::value) {
      dst[2 * c][t] = __builtin_bit_cast(f16, l16);
      dst[2 * c + 1][t] = __builtin_bit_cast(f16, h16);
    } else {
      dst[2 * c][t] = (f16)(bf16_bits_to_float(l16) * sc);
      dst[2 * c + 1][t] = (f16)(bf16_bits_to_float(h16) * sc);
    }
  }
};

}  // namespace tiles16
}  // namespace gdn
