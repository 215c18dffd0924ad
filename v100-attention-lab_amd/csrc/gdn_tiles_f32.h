// fp32 matrix-core tiles over LDS operands, shared by the backward and the
// two-launch forward: 16-byte row loads into LDS, products on
// v_mfma_f32_16x16x4_f32 with operands read through accessors, DPP row
// reductions, and the chunk-slot numbering of packed sequences.

#pragma once

#include "gdn_fwd_kernel.h"

namespace gdn {
namespace tiles {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes of TIn -> 16 / sizeof(TIn) floats.
template <typename TIn>
__device__ __forceinline__ void unpack16(const u32x4& r, float* x) {
  if constexpr (std::is_same<TIn, float>::value) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(r[e]);
  } else if constexpr (std::is_same<TIn, f16>::value) {
    const f16x8 h = __builtin_bit_cast(f16x8, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)h[e];
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __uint_as_float(r[e] << 16);
      x[2 * e + 1] = __uint_as_float(r[e] & 0xffff0000u);
    }
  }
}

template <typename TIn>
__device__ __forceinline__ void stx(void* base, int64_t off, float x) {
  if constexpr (std::is_same<TIn, float>::value) static_cast<float*>(base)[off] = x;
  else if constexpr (std::is_same<TIn, f16>::value) static_cast<f16*>(base)[off] = (f16)x;
  else static_cast<uint16_t*>(base)[off] = float_to_bf16_bits(x);
}

// One element's raw bits (fp32 bits, or the 16-bit value zero-extended);
// bits_to_float converts where the value is used.  A load whose result is
// converted right away makes the wave wait for it and for every load issued
// before it, which would drain loads meant to run ahead.
__device__ __forceinline__ uint32_t load_bits(const void* base, int64_t off, int dtype) {
  return dtype == GDN_DTYPE_F32 ? static_cast<const uint32_t*>(base)[off]
                                : (uint32_t) static_cast<const uint16_t*>(base)[off];
}
__device__ __forceinline__ float bits_to_float(uint32_t x, int dtype) {
  if (dtype == GDN_DTYPE_F32) return __uint_as_float(x);
  if (dtype == GDN_DTYPE_F16) return (float)__builtin_bit_cast(f16, (uint16_t)x);
  return __uint_as_float(x << 16);
}

// ROWS x COLS block of a row-major TIn array (row stride `rs` elements,
// 16-byte aligned rows) -> LDS as fp32, in two steps so that all global loads
// of a phase are issued before the first LDS store.  Rows >= nvalid read as
// zero.
template <typename TIn, int ROWS, int COLS, int NT>
struct RowLoad {
  static constexpr int VEC = 16 / (int)sizeof(TIn), RV = COLS / VEC, N = (ROWS * RV + NT - 1) / NT;
  static_assert(COLS % VEC == 0, "row width");
  u32x4 r[N];
  __device__ __forceinline__ void load(int tid, const TIn* base, int64_t rs, int nvalid) {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT, t = e / RV, col = (e % RV) * VEC;
      r[i] = (e < ROWS * RV && t < nvalid) ? *reinterpret_cast<const u32x4*>(base + t * rs + col) : z;
    }
  }
  // Every lane loads (rows >= nvalid >= 1 read row nvalid - 1 again), so
  // that no load is lane-masked: a masked load makes the compiler wait for
  // every load in flight before the values are used.  store_masked zeroes
  // those rows.
  __device__ __forceinline__ void load_clamped(int tid, const TIn* base, int64_t rs, int nvalid) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT, t = e / RV, col = (e % RV) * VEC;
      if (ROWS * RV % NT == 0 || e < ROWS * RV)
        r[i] = *reinterpret_cast<const u32x4*>(base + min(t, nvalid - 1) * rs + col);
    }
  }
  template <int LD>
  __device__ __forceinline__ void store_masked(int tid, float (*dst)[LD], int nvalid) const {
    static_assert(LD % 4 == 0, "16-byte rows");
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT, t = e / RV, col = (e % RV) * VEC;
      if (ROWS * RV % NT == 0 || e < ROWS * RV) {
        float x[VEC];
        unpack16<TIn>(r[i], x);
        const bool ok = t < nvalid;
#pragma unroll
        for (int j = 0; j < VEC; ++j) x[j] = ok ? x[j] : 0.f;
#pragma unroll
        for (int j = 0; j < VEC; j += 4)
          *reinterpret_cast<f32x4*>(&dst[t][col + j]) = f32x4{x[j], x[j + 1], x[j + 2], x[j + 3]};
      }
    }
  }
  template <int LD>
  __device__ __forceinline__ void store(int tid, float (*dst)[LD]) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT, t = e / RV, col = (e % RV) * VEC;
      if (e < ROWS * RV) {
        if constexpr (std::is_same<TIn, float>::value && LD % 4 == 0) {
          *reinterpret_cast<u32x4*>(&dst[t][col]) = r[i];
        } else if constexpr (LD % 4 == 0) {
          float x[VEC];
          unpack16<TIn>(r[i], x);
#pragma unroll
          for (int j = 0; j < VEC; j += 4)
            *reinterpret_cast<f32x4*>(&dst[t][col + j]) = f32x4{x[j], x[j + 1], x[j + 2], x[j + 3]};
        } else {
          float x[VEC];
          unpack16<TIn>(r[i], x);
#pragma unroll
          for (int j = 0; j < VEC; ++j) dst[t][col + j] = x[j];
        }
      }
    }
  }
  // 16-bit rows kept 16-bit: the raw 16-byte pieces (rows >= nvalid zeroed)
  template <typename TD, int LD>
  __device__ __forceinline__ void store_raw(int tid, TD (*dst)[LD], int nvalid = ROWS) const {
    static_assert(sizeof(TD) == sizeof(TIn) && LD * sizeof(TD) % 16 == 0, "16-byte rows of the same width");
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT, t = e / RV, col = (e % RV) * VEC;
      if (ROWS * RV % NT == 0 || e < ROWS * RV) {
        const bool ok = t < nvalid;
        *reinterpret_cast<u32x4*>(&dst[t][col]) =
            u32x4{ok ? r[i][0] : 0u, ok ? r[i][1] : 0u, ok ? r[i][2] : 0u, ok ? r[i][3] : 0u};
      }
    }
  }
  // fp32 rows as fp16 pairs hi + lo (x - hi rounded), two 8-byte stores
  template <int LD>
  __device__ __forceinline__ void store_pairs(int tid, _Float16 (*hi)[LD], _Float16 (*lo)[LD]) const {
    static_assert(std::is_same<TIn, float>::value && LD % 4 == 0, "fp32 rows, 8-byte pieces");
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT, t = e / RV, col = (e % RV) * VEC;
      if (ROWS * RV % NT == 0 || e < ROWS * RV) {
        h4 h, l;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = pin(__uint_as_float(r[i][j]));
          h[j] = (_Float16)x;
          l[j] = (_Float16)(x - (float)h[j]);
        }
        *reinterpret_cast<h4*>(&hi[t][col]) = h;
        *reinterpret_cast<h4*>(&lo[t][col]) = l;
      }
    }
  }
  // 16-bit rows as floats, columns [0, 16) times sc0 and [16, 32) times sc1
  // (powers of two: exact)
  template <int LD>
  __device__ __forceinline__ void store_scaled(int tid, float (*dst)[LD], float sc0, float sc1) const {
    static_assert(sizeof(TIn) == 2 && LD % 4 == 0 && COLS <= 32, "16-bit rows of at most 32 columns");
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT, t = e / RV, col = (e % RV) * VEC;
      if (e < ROWS * RV) {
        float x[VEC];
        unpack16<TIn>(r[i], x);
        const float sc = col < 16 ? sc0 : sc1;
#pragma unroll
        for (int j = 0; j < VEC; j += 4)
          *reinterpret_cast<f32x4*>(&dst[t][col + j]) = f32x4{x[j], x[j + 1], x[j + 2], x[j + 3]} * sc;
      }
    }
  }
};

// One term sum_{kk < KD} a(m, kk) b(kk, n) of a product.
template <int KD, typename FA, typename FB>
struct Seg {
  FA a;
  FB b;
};
template <int KD, typename FA, typename FB>
__device__ __forceinline__ Seg<KD, FA, FB> seg(FA a, FB b) {
  return Seg<KD, FA, FB>{a, b};
}

// acc[g] += one segment over the 16 x 16 tiles at (m0[g], n0[g]), g < ng, on
// v_mfma_f32_16x16x4_f32 (full fp32), the G tiles in flight together.
// Lane l supplies a(m0 + l % 16, k0 + l / 16) and b(k0 + l / 16, n0 + l % 16)
// and holds rows m0 + 4 (l / 16) + i, column n0 + l % 16 of a tile.
// UNR0: contraction steps unrolled (0: all of a contraction of up to 32,
// else 2, which keeps register use low where two waves share a SIMD).
template <int G, int UNR0 = 0, int KD, typename FA, typename FB>
__device__ __forceinline__ void seg_mfma(f32x4 (&acc)[G], const int (&m0)[G], const int (&n0)[G],
                                         int ng, int r, int kq, const Seg<KD, FA, FB>& s) {
  static_assert(KD % 4 == 0, "contraction length");
  constexpr int UNR = UNR0 > 0 ? (UNR0 < KD / 4 ? UNR0 : KD / 4) : (KD <= 32 ? KD / 4 : 2);
#pragma unroll UNR
  for (int k0 = 0; k0 < KD; k0 += 4) {
    float av[G], bv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      av[g] = g < ng ? s.a(m0[g] + r, k0 + kq) : 0.f;
      bv[g] = g < ng ? s.b(k0 + kq, n0[g] + r) : 0.f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[g], bv[g], acc[g], 0, 0, 0);
  }
}

// out(m, n, sum over the segments) for an M x N result: 16 x 16 tiles dealt
// round-robin to the NT / 64 waves, up to 4 of them in flight per wave.
template <int NT, int M, int N, int UNR = 0, typename FO, typename... Segs>
__device__ __forceinline__ void mmx(int tid, FO&& out, const Segs&... segs) {
  static_assert(M % 16 == 0 && N % 16 == 0, "16 x 16 tiles");
  constexpr int TNt = N / 16, NTILE = (M / 16) * TNt, NW = NT / 64;
  constexpr int G = NTILE >= 4 * NW ? 4 : (NTILE >= 2 * NW ? 2 : 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r = lane & 15, kq = lane >> 4;
  for (int base = wave; base < NTILE; base += NW * G) {
    int m0[G], n0[G], ng = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int tile = base + g * NW;
      m0[g] = tile < NTILE ? (tile / TNt) * 16 : 0;
      n0[g] = tile < NTILE ? (tile % TNt) * 16 : 0;
      if (tile < NTILE) ng = g + 1;
    }
    f32x4 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
    (seg_mfma<G, UNR>(acc, m0, n0, ng, r, kq, segs), ...);
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (g < ng) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out(m0[g] + 4 * kq + i, n0[g] + r, acc[g][i]);
      }
  }
}

// sum_{i < LEN} f(r, i) for row r = tid / (NT / ROWS), computed by the
// NT / ROWS lanes of the row (a power of two inside one wave) and returned to
// all of them.
template <int NT, int ROWS, int LEN, typename F>
__device__ __forceinline__ float row_sum(int tid, F&& f) {
  constexpr int RL = NT / ROWS;
  static_assert(RL >= 1 && RL <= 64 && (RL & (RL - 1)) == 0, "row lanes");
  const int r = tid / RL, part = tid % RL;
  float acc = 0.f;
  for (int i = part; i < LEN; i += RL) acc += f(r, i);
#pragma unroll
  for (int o = RL / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  return acc;
}

// Sum over the 16 lanes of a lane's row (lanes 16 j .. 16 j + 15), returned
// to all of them: rotate-and-add within the row on DPP (row_ror 8, 4, 2, 1).
template <int CTRL>
__device__ __forceinline__ float dpp_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float sum16(float x) {
  x += dpp_ror<0x128>(x);
  x += dpp_ror<0x124>(x);
  x += dpp_ror<0x122>(x);
  x += dpp_ror<0x121>(x);
  return x;
}

// Inclusive prefix sum over lanes 0..31 (and separately 32..63): DPP
// row_shr 1, 2, 4, 8 within each row of 16 lanes (lanes shifted in from
// outside the row read 0), then row_bcast:15 adds the totals of rows 0 / 2
// to rows 1 / 3.  All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_shr0(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float scan32(float x) {
  x += dpp_shr0<0x111>(x);
  x += dpp_shr0<0x112>(x);
  x += dpp_shr0<0x114>(x);
  x += dpp_shr0<0x118>(x);
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xa, 0xf, false));
  return x;
}

// 16 bytes of LDS as four floats.
template <int LD>
__device__ __forceinline__ f32x4 ld4(const float (*x)[LD], int row, int col) {
  static_assert(LD % 4 == 0, "16-byte rows");
  return *reinterpret_cast<const f32x4*>(&x[row][col]);
}

// Chunk slot -> (sequence, its rows, chunk).  False for a slot that holds
// no chunk (the gaps between packed sequences).
// p: B (sequences when cu is set), T, nchmax = ceil(T / C), cu.
template <int C, typename Args>
__device__ __forceinline__ bool slot_chunk(const Args& p, int64_t slot, RowSpan& rs, int& c, int& seq) {
  if (p.cu == nullptr) {
    seq = (int)(slot / p.nchmax);
    c = (int)(slot % p.nchmax);
    rs = row_span(nullptr, p.T, seq);
    return seq < p.B && (int64_t)c * C < rs.T;
  }
  // the last sequence whose first slot floor(t0 / C) + i is <= slot
  int lo = 0, hi = p.B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (row_span(p.cu, p.T, mid).t0 / C + mid <= slot) lo = mid;
    else hi = mid - 1;
  }
  rs = row_span(p.cu, p.T, lo);
  seq = lo;
  const int64_t cc = slot - (rs.t0 / C + lo);
  c = (int)cc;
  return cc >= 0 && cc * C < rs.T;
}
template <int C, typename Args>
__device__ __forceinline__ bool slot_chunk(const Args& p, int64_t slot, RowSpan& rs, int& c) {
  int seq;
  return slot_chunk<C>(p, slot, rs, c, seq);
}

}  // namespace tiles
}  // namespace gdn
