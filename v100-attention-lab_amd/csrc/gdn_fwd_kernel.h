// Fused chunked Gated DeltaNet forward for MI355X (gfx950 / CDNA4).
//
// One workgroup (4 waves of 64) owns one (batch b, head h, V-slice of BV
// columns) and scans the chunks of the sequence in order, keeping its
// K x BV slice of the fp32 state S = h^T resident in the MFMA accumulator
// registers of its "scan" waves for the whole sequence.  Nothing but the
// final state leaves the chip, so memory stays O(B*H*K*V).
//
// Per chunk of C steps (b = cumsum(g) inside the chunk; the math is the
// chunked UT form of the reference, gdn_ref.py:51-58, gdn_triton.py:54-106):
//   P0  q, k [C,K], v [C,BV], g, beta [C] -> LDS (16-byte global loads;
//       k is also stored transposed; bf16 inputs become fp16 operands).
//   P1  b, e^{b}, e^{bC-b} (wave 0, in registers -> LDS).
//   P2  MFMA: G = K K^T -> A[t,j] = beta_t e^{b_t-b_j} G[t,j]   (t > j)
//             Q K^T     -> P[t,j] = e^{b_t-b_j} (q_t.k_j)       (t >= j)
//       masks are applied before the exponential.
//   P3  VALU forward substitution T = (I+A)^{-1}, one lane per column,
//       rows of A broadcast from LDS; then Tw = -T diag(beta e^b) and
//       Tu = T diag(beta) as MFMA operands.
//   P4  MFMA: W'^T = K^T Tw^T  (W' = -W, W = (I+A)^{-1} diag(beta e^b) K).
//   P5  scan waves (16 state columns each), MFMA:
//         u   = Tu V + W' S                    (U - W h^T)
//         o   = scale (P u + diag(e^b) Q S)
//         S  <- e^{bC} S + K^T diag(e^{bC-b}) u
//       The last line is the reference's update h(e^{bC}I - Wbar^T K) +
//       Ubar^T K (gdn_ref.py:93-98) reassociated: Ubar - Wbar h^T =
//       diag(e^{bC-b}) (U - W h^T), which avoids the K x K temporary.
//
// MFMA operand layout.  v_mfma_f32_16x16x32_{f16} takes, per lane l, row
// (A) / column (B) l%16 and eight reduction slots owned by lane group
// g = l/16.  The accumulator D holds column l%16 and rows 4g..4g+3.  Since
// the reduction is a plain sum, any bijection between (g, slot) and the
// reduction index works as long as A and B agree.  This file uses
//     pi(g, s) = s < 4 ? 4g + s : 16 + 4g + (s - 4)     (within a 32-block)
// because then the two accumulator tiles covering rows [32c, 32c+32) of a
// product P are, lane for lane, exactly the B operand of P (reduction over
// P's rows) and the A operand of P^T.  The state S (K x BV) therefore feeds
// the next chunk's "x S" products straight from its accumulators, and u
// feeds "P u" and "K^T u" straight from its accumulators: no LDS round trip
// and no cross-lane shuffle on the serial path.  fp32 inputs use
// v_mfma_f32_16x16x4_f32 eight times per 32-block (slot s = one MFMA).

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "gdn_mi355x.h"

namespace gdn {

typedef _Float16 f16;
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

struct bf16_t {
  uint16_t bits;
};

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsLimit = 160 * 1024;

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

// float -> bf16 bits, round to nearest even (NaN stays NaN): gfx950's
// v_cvt_pk_bf16_f32, one instruction per pair where two are packed.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float load_scalar(const void* base, int64_t off,
                                             int dtype) {
  if (dtype == GDN_DTYPE_F32) return static_cast<const float*>(base)[off];
  if (dtype == GDN_DTYPE_F16) return (float)static_cast<const f16*>(base)[off];
  return bf16_bits_to_float(static_cast<const uint16_t*>(base)[off]);
}

__device__ __forceinline__ void store_scalar(void* base, int64_t off, int dtype,
                                             float x) {
  if (dtype == GDN_DTYPE_F32) {
    static_cast<float*>(base)[off] = x;
  } else if (dtype == GDN_DTYPE_F16) {
    static_cast<f16*>(base)[off] = (f16)x;
  } else {
    static_cast<uint16_t*>(base)[off] = float_to_bf16_bits(x);
  }
}

// ---------------------------------------------------------------------------
// input element type -> MFMA operand type, 16 bytes at a time
// ---------------------------------------------------------------------------

template <typename TIn>
struct InTraits;

template <>
struct InTraits<f16> {
  static constexpr int kVec = 8;  // elements per 16-byte load
  __device__ static __forceinline__ void to_op(const uint4& r, f16* out) {
    const f16* p = reinterpret_cast<const f16*>(&r);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = p[e];
  }
};

template <>
struct InTraits<bf16_t> {
  static constexpr int kVec = 8;
  // bf16 -> fp16 is exact for |x| in fp16's normal range; smaller values
  // keep fp16's subnormal precision (absolute 2^-24).
  __device__ static __forceinline__ void to_op(const uint4& r, f16* out) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[2 * e] = (f16)bf16_bits_to_float(w[e] & 0xffffu);
      out[2 * e + 1] = (f16)bf16_bits_to_float(w[e] >> 16);
    }
  }
  // times sc (a power of two: exact) before the conversion
  __device__ static __forceinline__ void to_op_sc(const uint4& r, f16* out, float sc) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[2 * e] = (f16)(bf16_bits_to_float(w[e] & 0xffffu) * sc);
      out[2 * e + 1] = (f16)(bf16_bits_to_float(w[e] >> 16) * sc);
    }
  }
};

template <>
struct InTraits<float> {
  static constexpr int kVec = 4;
  __device__ static __forceinline__ void to_op(const uint4& r, float* out) {
    out[0] = __uint_as_float(r.x);
    out[1] = __uint_as_float(r.y);
    out[2] = __uint_as_float(r.z);
    out[3] = __uint_as_float(r.w);
  }
};

// ---------------------------------------------------------------------------
// Range of bf16 inputs.  bf16 q, k, v reach the matrix cores as fp16
// operands, and so do quantities derived from v (u, the state): fp16 holds
// |x| <= 65504 and is subnormal below 2^-14, far less than bf16.  o and the
// state are jointly linear in (v, h0), and each column of the state evolves
// on its own, so a workgroup that owns a slice of V columns runs on v and h0
// scaled by a power of two 2^s chosen from the slice's largest magnitude and
// scales o and final_state by 2^-s.  Powers of two are exact in fp32 and
// carry over fp16 rounding unchanged, and s = 0 (nothing changes) whenever
// that magnitude lies in [2^-6, 2^10].  (q and k are not rescaled: the delta
// rule needs |k| of order one, and q is normalised in every caller here.)
// ---------------------------------------------------------------------------

// Largest |x| of a pair of bf16 values as an fp32 bit pattern (patterns of
// non-negative floats order like their values; NaN patterns lie above inf).
__device__ __forceinline__ uint32_t bf16x2_absmax_bits(uint32_t w) {
  return max((w & 0x7fffu) << 16, w & 0x7fff0000u);
}
__device__ __forceinline__ uint32_t bf16x8_absmax_bits(const uint4& x) {
  return max(max(bf16x2_absmax_bits(x.x), bf16x2_absmax_bits(x.y)),
             max(bf16x2_absmax_bits(x.z), bf16x2_absmax_bits(x.w)));
}

// This thread's part of the largest magnitude of h0[K x cols] (fp32,
// element strides sk and sc; nullable), as float bits.
__device__ __forceinline__ uint32_t state_absmax_bits(const float* h0, int64_t sk, int64_t sc, int K, int cols) {
  uint32_t m = 0;
  if (h0 != nullptr) {
    const int64_t nh = (int64_t)K * cols;
    for (int64_t i = threadIdx.x; i < nh; i += blockDim.x) {
      const int64_t kk = i / cols;
      const int c = (int)(i - kk * cols);
      m = max(m, __float_as_uint(h0[kk * sk + c * sc]) & 0x7fffffffu);
    }
  }
  return m;
}

// Maximum of m over the workgroup (every thread calls it; one barrier;
// red holds a value per wave).
__device__ __forceinline__ uint32_t block_max_bits(uint32_t m, uint32_t* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = 0;
  for (int w = 0; w < (int)(blockDim.x + 63) / 64; ++w) m = max(m, red[w]);
  return m;
}

// Largest magnitude of v[rows x cols] (bf16, rows `rstride` bytes apart,
// cols a multiple of 8, 16-byte aligned rows) and of h0[K x cols] (fp32,
// element strides sk and sc; nullable), over the whole workgroup: every
// thread of the workgroup calls it (one barrier).  NaN if either holds one.
__device__ __forceinline__ float slice_absmax_bf16(const char* v, int64_t rstride, int rows, int cols,
                                                   const float* h0, int64_t sk, int64_t sc, int K) {
  __shared__ uint32_t red[16];
  const int tid = threadIdx.x, nthr = blockDim.x;
  uint32_t m = 0;
  const int pieces = cols >> 3;
  auto piece_max = [](const uint4& x) { return bf16x8_absmax_bits(x); };
  if (nthr % pieces == 0) {
    // a fixed 16-byte column piece per thread, rows nthr / pieces apart,
    // eight loads in flight
    const int rstep = nthr / pieces;
    const char* const vc = v + (tid % pieces) * 16;
    int r = tid / pieces;
    for (; r + 7 * rstep < rows; r += 8 * rstep) {
      uint4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const uint4*>(vc + (int64_t)(r + u * rstep) * rstride);
#pragma unroll
      for (int u = 0; u < 8; ++u) m = max(m, piece_max(x[u]));
    }
    for (; r < rows; r += rstep) m = max(m, piece_max(*reinterpret_cast<const uint4*>(vc + (int64_t)r * rstride)));
  } else {
    const int64_t nv = (int64_t)rows * pieces;
    for (int64_t i = tid; i < nv; i += nthr) {
      const int64_t r = i / pieces;
      const int c = (int)(i - r * pieces);
      m = max(m, piece_max(*reinterpret_cast<const uint4*>(v + r * rstride + c * 16)));
    }
  }
  return __uint_as_float(block_max_bits(max(m, state_absmax_bits(h0, sk, sc, K, cols)), red));
}

// The shift s for a slice whose largest magnitude is m: 0 when m is zero,
// not finite or in [2^-6, 2^10]; else m 2^s lies in [1, 2).
__device__ __forceinline__ int range_shift(float m) {
  if (!(m > 0.f) || !(m < __builtin_inff())) return 0;
  if (m >= 0x1p-6f && m <= 0x1p10f) return 0;
  int e;
  (void)frexpf(m, &e);  // m = f 2^e, f in [0.5, 1)
  return min(max(1 - e, -126), 126);
}

// Scale factors of a slice: v and h0 by 2^s, o (with the caller's scale)
// and final_state by 2^-s.
struct RangeScale {
  float v = 1.f, o = 1.f, fs = 1.f;
};

// The scale factors for a slice whose largest magnitude is m (v and h0
// taken together).
__device__ __forceinline__ RangeScale range_scale_of(float m, float scale) {
  RangeScale r;
  const int sh = range_shift(m);
  r.v = ldexpf(1.f, sh);
  r.fs = ldexpf(1.f, -sh);
  r.o = scale * r.fs;
  return r;
}

template <typename TIn>
__device__ __forceinline__ RangeScale slice_range_scale(const char* v, int64_t rstride, int rows, int cols,
                                                        const float* h0, int64_t sk, int64_t sc, int K,
                                                        float scale) {
  RangeScale r;
  r.o = scale;
  if constexpr (std::is_same<TIn, bf16_t>::value) {
    const int sh = range_shift(slice_absmax_bf16(v, rstride, rows, cols, h0, sk, sc, K));
    r.v = ldexpf(1.f, sh);
    r.fs = ldexpf(1.f, -sh);
    r.o = scale * r.fs;
  }
  return r;
}

template <typename TIn>
struct OpOf {
  using type = f16;
};
template <>
struct OpOf<float> {
  using type = float;
};

// ---------------------------------------------------------------------------
// MFMA operand traits
// ---------------------------------------------------------------------------

template <typename TOp>
struct Mma;

template <>
struct Mma<f16> {
  using frag = f16x8;
  __device__ static __forceinline__ f32x4 mma(const frag& a, const frag& b,
                                              f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // Slots 0..7 <- blk[8g .. 8g+8)   (plain layout, used when both operands
  // come from LDS rows).
  __device__ static __forceinline__ frag load_contig(const f16* blk, int g) {
    return *reinterpret_cast<const f16x8*>(blk + 8 * g);
  }
  // Slots 0..7 <- blk[pi(g, 0..7)].
  __device__ static __forceinline__ frag load_pi(const f16* blk, int g) {
    const f16x4 lo = *reinterpret_cast<const f16x4*>(blk + 4 * g);
    const f16x4 hi = *reinterpret_cast<const f16x4*>(blk + 16 + 4 * g);
    return frag{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  // Accumulator tiles (rows [0,16) and [16,32) of a 32-block) -> operand.
  __device__ static __forceinline__ frag from_acc(const f32x4& lo,
                                                  const f32x4& hi) {
    return frag{(f16)lo[0], (f16)lo[1], (f16)lo[2], (f16)lo[3],
                (f16)hi[0], (f16)hi[1], (f16)hi[2], (f16)hi[3]};
  }
  __device__ static __forceinline__ void store4(f16* dst, const f32x4& x) {
    *reinterpret_cast<f16x4*>(dst) =
        f16x4{(f16)x[0], (f16)x[1], (f16)x[2], (f16)x[3]};
  }
};

template <>
struct Mma<float> {
  using frag = f32x8;
  __device__ static __forceinline__ f32x4 mma(const frag& a, const frag& b,
                                              f32x4 c) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
    }
    return c;
  }
  __device__ static __forceinline__ frag load_contig(const float* blk, int g) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(blk + 8 * g);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(blk + 8 * g + 4);
    return frag{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  __device__ static __forceinline__ frag load_pi(const float* blk, int g) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(blk + 4 * g);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(blk + 16 + 4 * g);
    return frag{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  __device__ static __forceinline__ frag from_acc(const f32x4& lo,
                                                  const f32x4& hi) {
    return frag{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  __device__ static __forceinline__ void store4(float* dst, const f32x4& x) {
    *reinterpret_cast<f32x4*>(dst) = x;
  }
};

// The value of x as one fp32 register: every later use (an fp16 rounding
// and the residual against it) sees the same rounded value.  Without it the
// compiler may fuse the product that made x into each use separately (an
// fp16 conversion of the exact product in one, of the rounded one in the
// other), and hi + lo then misses x by half an fp16 ulp.
__device__ __forceinline__ float pin(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// The fp16 rounding residual of two accumulator tiles, as an operand:
// x - (float)hi, so that hi + lo carries x to about 2^-22 relative.
__device__ __forceinline__ f16x8 split_lo(const f32x4& lo, const f32x4& hi, const f16x8& h) {
  return f16x8{(f16)(lo[0] - (float)h[0]), (f16)(lo[1] - (float)h[1]),
               (f16)(lo[2] - (float)h[2]), (f16)(lo[3] - (float)h[3]),
               (f16)(hi[0] - (float)h[4]), (f16)(hi[1] - (float)h[5]),
               (f16)(hi[2] - (float)h[6]), (f16)(hi[3] - (float)h[7])};
}

// ---------------------------------------------------------------------------
// LDS layout of one workgroup
// ---------------------------------------------------------------------------

template <typename TOp, int K, int C, int BV>
struct alignas(16) Smem {
  static constexpr int kPad = 16 / (int)sizeof(TOp);
  static constexpr int SK = K + kPad;  // row stride of [C][K] tiles
  static constexpr int SC = C + kPad;  // row stride of [*][C] tiles
  TOp q[C * SK];      // q rows
  TOp k[C * SK];      // k rows
  TOp w[C * SK];      // W' = -W rows
  TOp kt[K * SC];     // k transposed: kt[kk][t]
  TOp vt[BV * SC];    // v slice transposed: vt[vc][t]
  TOp p[C * SC];      // P[t][j] = e^{b_t-b_j} q_t.k_j, j <= t (else 0)
  TOp plo[C * SC];    // fp16 residual P - (float)P (fp16 operands only)
  TOp tw[C * SC];     // Tw = -T diag(beta e^b)
  TOp tu[C * SC];     // Tu = T diag(beta)
  float a[C * C];     // A (strictly lower) for the substitution
  float gate[C];
  float beta[C];
  float b[C];         // cumsum(g) inside the chunk
  float eb[C];        // e^{b_t}
  float ec[C];        // e^{b_C - b_t}
};

template <typename TOp, int K, int C, int BV>
constexpr int smem_bytes() {
  return (int)sizeof(Smem<TOp, K, C, BV>);
}

struct KArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;
  void* o;
  float* fs;
  int64_t sq[3], sk[3], sv[3], sg[3], sb[3], so[3];
  int64_t sh0[4], sfs[4];
  int B, T, H, V, nv;
  float scale;
  int g_dtype, beta_dtype, o_dtype;
  int xcd_remap;
  const int64_t* cu;  // nullable: B + 1 row offsets of packed sequences
};

// Rows of work unit bi.  Without cu: rows [0, T) of batch bi.  With cu
// (sequences packed along t of batch 0): rows [cu[bi], cu[bi + 1]) of batch
// 0, clamped to [0, T] so that malformed offsets never address memory
// outside the tensors.
struct RowSpan {
  int64_t b;   // batch index
  int64_t t0;  // first row
  int T;       // number of rows
};

__device__ __forceinline__ RowSpan row_span(const int64_t* cu, int T, int bi) {
  if (cu == nullptr) return RowSpan{bi, 0, T};
  int64_t lo = cu[bi], hi = cu[bi + 1];
  lo = lo < 0 ? 0 : (lo > T ? T : lo);
  hi = hi < lo ? lo : (hi > T ? T : hi);
  return RowSpan{0, lo, (int)(hi - lo)};
}

__device__ __forceinline__ RowSpan row_span(const KArgs& p, int bi) { return row_span(p.cu, p.T, bi); }

// Element offset of the first row of head h in a [B, T, H, *] tensor with
// (b, t, h) strides s.
__device__ __forceinline__ int64_t head_base(const RowSpan& r, int h, const int64_t* s) {
  return r.b * s[0] + r.t0 * s[1] + h * s[2];
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------

template <typename TIn, int K, int C, int BV>
__global__ __launch_bounds__(kThreads) void gdn_fwd_kernel(const KArgs p) {
  using TOp = typename OpOf<TIn>::type;
  using M = Mma<TOp>;
  using frag = typename M::frag;
  using S = Smem<TOp, K, C, BV>;
  constexpr int SK = S::SK, SC = S::SC;
  constexpr int NSW = BV / 16;   // scan waves, 16 state columns each
  constexpr int KB = K / 32, CB = C / 32, KT = K / 16, CT = C / 16;
  constexpr int VEC = InTraits<TIn>::kVec;
  static_assert(NSW >= 1 && NSW <= kWaves, "BV must be 16..64");
  static_assert(K % 32 == 0 && C % 32 == 0 && BV % VEC == 0, "tile shape");

  __shared__ S s;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;   // A row / B column / D column of this lane
  const int gq = lane >> 4;  // lane group: reduction slots / D rows

  // Work unit.  With xcd_remap, units u = x*(N/8) .. are dispatched to XCD x
  // (workgroups go round-robin over the 8 XCDs), so the V-slices of one
  // (b, h) share an L2 and fetch q/k from HBM once.
  int unit = blockIdx.x;
  if (p.xcd_remap) unit = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int vs = unit % p.nv;
  const int bh = unit / p.nv;
  const int bi = bh / p.H;
  const int hi = bh % p.H;
  const int v0 = vs * BV;
  const RowSpan rs = row_span(p, bi);
  const int T = rs.T;

  const TIn* qg = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq);
  const TIn* kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* vg = static_cast<const TIn*>(p.v) + head_base(rs, hi, p.sv) + v0;
  const int64_t g_base = head_base(rs, hi, p.sg);
  const int64_t b_base = head_base(rs, hi, p.sb);
  // bf16: this slice's v and h0 scaled into fp16's range, o and the final
  // state scaled back (identity for fp16 and fp32)
  const RangeScale rsc = slice_range_scale<TIn>(
      reinterpret_cast<const char*>(vg), p.sv[1] * (int64_t)sizeof(TIn), T, BV,
      p.h0 ? p.h0 + bi * p.sh0[0] + hi * p.sh0[1] + v0 * p.sh0[3] : nullptr, p.sh0[2], p.sh0[3], K, p.scale);

  // State slice S[:, v0 + 16*wave + n] in D layout: tile r holds rows
  // 16r + 4gq + i.
  f32x4 st[KT];
  const int vcol = 16 * wave + n;  // column inside this workgroup's slice
#pragma unroll
  for (int r = 0; r < KT; ++r) st[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (wave < NSW && p.h0 != nullptr) {
    const float* h0 = p.h0 + bi * p.sh0[0] + hi * p.sh0[1] + (v0 + vcol) * p.sh0[3];
#pragma unroll
    for (int r = 0; r < KT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) st[r][i] = h0[(16 * r + 4 * gq + i) * p.sh0[2]] * rsc.v;
  }

  for (int t0 = 0; t0 < T; t0 += C) {
    // ---------------- P0: chunk tiles -> LDS ----------------
    {
      constexpr int RV = K / VEC;  // 16-byte vectors per q/k row
#pragma unroll 2
      for (int idx = tid; idx < C * RV; idx += kThreads) {
        const int t = idx / RV;
        const int c = (idx % RV) * VEC;
        uint4 rq = {0u, 0u, 0u, 0u}, rk = {0u, 0u, 0u, 0u};
        if (t0 + t < T) {
          rq = *reinterpret_cast<const uint4*>(qg + (int64_t)(t0 + t) * p.sq[1] + c);
          rk = *reinterpret_cast<const uint4*>(kg + (int64_t)(t0 + t) * p.sk[1] + c);
        }
        TOp xq[VEC], xk[VEC];
        InTraits<TIn>::to_op(rq, xq);
        InTraits<TIn>::to_op(rk, xk);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          s.q[t * SK + c + e] = xq[e];
          s.k[t * SK + c + e] = xk[e];
          s.kt[(c + e) * SC + t] = xk[e];
        }
      }
      constexpr int RVV = BV / VEC;
      for (int idx = tid; idx < C * RVV; idx += kThreads) {
        const int t = idx / RVV;
        const int c = (idx % RVV) * VEC;
        uint4 rv = {0u, 0u, 0u, 0u};
        if (t0 + t < T) rv = *reinterpret_cast<const uint4*>(vg + (int64_t)(t0 + t) * p.sv[1] + c);
        TOp xv[VEC];
        if constexpr (std::is_same<TIn, bf16_t>::value)
          InTraits<TIn>::to_op_sc(rv, xv, rsc.v);
        else
          InTraits<TIn>::to_op(rv, xv);
#pragma unroll
        for (int e = 0; e < VEC; ++e) s.vt[(c + e) * SC + t] = xv[e];
      }
      if (tid < C) {
        const bool ok = t0 + tid < T;
        s.gate[tid] = ok ? load_scalar(p.g, g_base + (int64_t)(t0 + tid) * p.sg[1], p.g_dtype) : 0.f;
        s.beta[tid] = ok ? load_scalar(p.beta, b_base + (int64_t)(t0 + tid) * p.sb[1], p.beta_dtype) : 0.f;
      }
    }
    __syncthreads();

    // ---------------- P1: gate cumsum and decays ----------------
    if (wave == 0) {
      // Sequential prefix sum in each lane (same association order as a
      // sequential cumsum).
      float bt = 0.f;
      for (int j = 0; j < C; ++j) {
        const float gj = s.gate[j];
        if (j <= lane) bt += gj;
      }
      const float bC = __shfl(bt, C - 1, 64);
      if (lane < C) {
        s.b[lane] = bt;
        s.eb[lane] = expf(bt);
        s.ec[lane] = expf(bC - bt);
      }
    }
    __syncthreads();

    // ---------------- P2: K K^T -> A,  Q K^T -> P ----------------
    {
      constexpr int NJ = 2 * CT * CT;
      for (int job = wave; job < NJ; job += kWaves) {
        const int mat = job / (CT * CT);
        const int mt = (job / CT) % CT;
        const int nt = job % CT;
        const int j = 16 * nt + n;
        if (nt > mt) {  // tile above the diagonal
          if (mat == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              s.p[(16 * mt + 4 * gq + i) * SC + j] = (TOp)0.f;
              s.plo[(16 * mt + 4 * gq + i) * SC + j] = (TOp)0.f;
            }
          }
          continue;
        }
        const TOp* arow = (mat == 0 ? s.k : s.q) + (16 * mt + n) * SK;
        const TOp* brow = s.k + (16 * nt + n) * SK;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          acc = M::mma(M::load_contig(arow + 32 * kb, gq), M::load_contig(brow + 32 * kb, gq), acc);
        }
        const float bj = s.b[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * mt + 4 * gq + i;
          if (mat == 0) {
            s.a[t * C + j] = (t > j) ? acc[i] * expf(s.b[t] - bj) * s.beta[t] : 0.f;
          } else {
            const float pv = pin((t >= j) ? acc[i] * expf(s.b[t] - bj) : 0.f);
            s.p[t * SC + j] = (TOp)pv;
            s.plo[t * SC + j] = (TOp)(pv - (float)(TOp)pv);
          }
        }
      }
    }
    __syncthreads();

    // ---------------- P3: T = (I + A)^{-1} by forward substitution ----------
    if constexpr (C == 64) {
      // Block forward substitution on the VALU, T = [[T11, 0], [T21, T22]]:
      // T11 = (I + A11)^{-1} and T22 = (I + A22)^{-1} by substitution at the
      // same time (waves 0 and 1, lane c owns column c of its block, written
      // over A11 / A22); then the second block row, (I + A22) T21 = -A21 T11,
      // as X = A21 T11 (into the unused upper-right block) and T21 = -T22 X
      // (over A21), dot products over LDS rows by every thread.
      constexpr int H2 = 32;
      if (wave < 2 && lane < H2) {
        const int o = H2 * wave;
        float tc[H2];
#pragma unroll
        for (int i = 0; i < H2; ++i) {
          float acc = (lane == i) ? 1.f : 0.f;
#pragma unroll
          for (int j4 = 0; j4 < i; j4 += 4) {
            const f32x4 a4 = *reinterpret_cast<const f32x4*>(&s.a[(o + i) * C + o + j4]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (j4 + e < i) acc = fmaf(-a4[e], tc[j4 + e], acc);
          }
          tc[i] = acc;
        }
        // the block's A entries are no longer read: overwrite them with T
#pragma unroll
        for (int i = 0; i < H2; ++i) s.a[(o + i) * C + o + lane] = tc[i];
      }
      __syncthreads();
      // X = A21 T11 -> upper-right block (T11's zeros above its diagonal are
      // exact)
      for (int e = tid; e < H2 * H2; e += kThreads) {
        const int m = e / H2, nn = e % H2;
        float acc = 0.f;
#pragma unroll 8
        for (int kk = 0; kk < H2; ++kk) acc = fmaf(s.a[(H2 + m) * C + kk], s.a[kk * C + nn], acc);
        s.a[m * C + H2 + nn] = acc;
      }
      __syncthreads();
      // T21 = -T22 X -> lower-left block (A21 is no longer needed)
      for (int e = tid; e < H2 * H2; e += kThreads) {
        const int m = e / H2, nn = e % H2;
        float acc = 0.f;
#pragma unroll 8
        for (int kk = 0; kk < H2; ++kk) acc = fmaf(s.a[(H2 + m) * C + H2 + kk], s.a[kk * C + H2 + nn], acc);
        s.a[(H2 + m) * C + nn] = -acc;
      }
      __syncthreads();
      for (int e = tid; e < C * C; e += kThreads) {
        const int i = e / C, c = e % C;
        const float t = c <= i ? s.a[i * C + c] : 0.f;
        const float ru = s.beta[c];
        s.tw[i * SC + c] = (TOp)(t * (-ru * s.eb[c]));
        s.tu[i * SC + c] = (TOp)(t * ru);
      }
    } else if (wave == 0) {
      // Lane c owns column c of T: T[i][c] = [i == c] - sum_{j<i} A[i][j] T[j][c].
      float tc[C];
#pragma unroll
      for (int i = 0; i < C; ++i) {
        float acc = (lane == i) ? 1.f : 0.f;
#pragma unroll
        for (int j4 = 0; j4 < i; j4 += 4) {
          const f32x4 a4 = *reinterpret_cast<const f32x4*>(&s.a[i * C + j4]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j4 + e < i) acc = fmaf(-a4[e], tc[j4 + e], acc);
        }
        tc[i] = acc;
      }
      if (lane < C) {
        const float ru = s.beta[lane];
        const float rw = -ru * s.eb[lane];
#pragma unroll
        for (int i = 0; i < C; ++i) {
          s.tw[i * SC + lane] = (TOp)(tc[i] * rw);
          s.tu[i * SC + lane] = (TOp)(tc[i] * ru);
        }
      }
    }
    __syncthreads();

    // ---------------- P4: W'^T = K^T Tw^T -> s.w (rows of W') ----------------
    {
      constexpr int NJ = KT * CT;
      for (int job = wave; job < NJ; job += kWaves) {
        const int mt = job / CT;  // K tile
        const int nt = job % CT;  // t tile
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          acc = M::mma(M::load_pi(s.kt + (16 * mt + n) * SC + 32 * cb, gq),
                       M::load_pi(s.tw + (16 * nt + n) * SC + 32 * cb, gq), acc);
        }
        M::store4(s.w + (16 * nt + n) * SK + 16 * mt + 4 * gq, acc);
      }
    }
    __syncthreads();

    // ---------------- P5: state-dependent part (scan waves) ----------------
    if (wave < NSW) {
      frag sB[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sB[kb] = M::from_acc(st[2 * kb], st[2 * kb + 1]);

      f32x4 u[CT], oq[CT];
#pragma unroll
      for (int mt = 0; mt < CT; ++mt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          acc = M::mma(M::load_pi(s.tu + (16 * mt + n) * SC + 32 * cb, gq),
                       M::load_pi(s.vt + vcol * SC + 32 * cb, gq), acc);
        f32x4 accq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          acc = M::mma(M::load_pi(s.w + (16 * mt + n) * SK + 32 * kb, gq), sB[kb], acc);
          accq = M::mma(M::load_pi(s.q + (16 * mt + n) * SK + 32 * kb, gq), sB[kb], accq);
        }
        u[mt] = acc;
        oq[mt] = accq;
      }

      frag uB[CB], uL[CB], utB[CB];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const f32x4 lo = u[2 * cb], hi = u[2 * cb + 1];
        uB[cb] = M::from_acc(lo, hi);
        if constexpr (std::is_same<TOp, f16>::value) uL[cb] = split_lo(lo, hi, uB[cb]);
        f32x4 lo2, hi2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo2[i] = lo[i] * s.ec[32 * cb + 4 * gq + i];
          hi2[i] = hi[i] * s.ec[32 * cb + 16 + 4 * gq + i];
        }
        utB[cb] = M::from_acc(lo2, hi2);
      }

      const int64_t o_col = head_base(rs, hi, p.so) + v0 + vcol;
#pragma unroll
      for (int mt = 0; mt < CT; ++mt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const frag pA = M::load_pi(s.p + (16 * mt + n) * SC + 32 * cb, gq);
          if constexpr (std::is_same<TOp, f16>::value) {
            // P u as P_hi u_hi + P_hi u_lo + P_lo u_hi
            acc = M::mma(pA, uL[cb], acc);
            acc = M::mma(M::load_pi(s.plo + (16 * mt + n) * SC + 32 * cb, gq), uB[cb], acc);
          }
          acc = M::mma(pA, uB[cb], acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * mt + 4 * gq + i;
          if (t0 + t < T) {
            const float val = rsc.o * (acc[i] + s.eb[t] * oq[mt][i]);
            store_scalar(p.o, o_col + (int64_t)(t0 + t) * p.so[1], p.o_dtype, val);
          }
        }
      }

      const float ebC = s.eb[C - 1];
#pragma unroll
      for (int r = 0; r < KT; ++r) {
        f32x4 acc = st[r] * ebC;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          acc = M::mma(M::load_pi(s.kt + (16 * r + n) * SC + 32 * cb, gq), utB[cb], acc);
        st[r] = acc;
      }
    }
    __syncthreads();
  }

  if (wave < NSW) {
    float* fs = p.fs + bi * p.sfs[0] + hi * p.sfs[1] + (v0 + vcol) * p.sfs[3];
#pragma unroll
    for (int r = 0; r < KT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) fs[(16 * r + 4 * gq + i) * p.sfs[2]] = st[r][i] * rsc.fs;
  }
}

// ---------------------------------------------------------------------------
// dispatch over compile-time shapes
// ---------------------------------------------------------------------------

inline int elem_bytes(int dtype) { return dtype == GDN_DTYPE_F32 ? 4 : 2; }

inline bool valid_dtype(int d) {
  return d == GDN_DTYPE_F32 || d == GDN_DTYPE_F16 || d == GDN_DTYPE_BF16;
}

template <typename TIn, int K, int C, int BV>
constexpr bool fits() {
  return smem_bytes<typename OpOf<TIn>::type, K, C, BV>() <= kLdsLimit;
}

template <typename TIn, int K, int C, int BV>
int launch_one(const KArgs& a, int grid, hipStream_t stream) {
  if constexpr (fits<TIn, K, C, BV>()) {
    hipLaunchKernelGGL((gdn_fwd_kernel<TIn, K, C, BV>), dim3(grid), dim3(kThreads), 0,
                       stream, a);
    return (int)hipGetLastError();
  } else {
    return GDN_ERR_UNSUPPORTED;
  }
}

template <typename TIn, int K, int C>
int launch_bv(const KArgs& a, int bv, int grid, hipStream_t s) {
  switch (bv) {
    case 16: return launch_one<TIn, K, C, 16>(a, grid, s);
    case 32: return launch_one<TIn, K, C, 32>(a, grid, s);
    case 64: return launch_one<TIn, K, C, 64>(a, grid, s);
    default: return GDN_ERR_UNSUPPORTED;
  }
}

template <typename TIn, int K>
int launch_c(const KArgs& a, int c, int bv, int grid, hipStream_t s) {
  switch (c) {
    case 32: return launch_bv<TIn, K, 32>(a, bv, grid, s);
    case 64: return launch_bv<TIn, K, 64>(a, bv, grid, s);
    default: return GDN_ERR_UNSUPPORTED;
  }
}

template <typename TIn>
int launch_k(const KArgs& a, int kdim, int c, int bv, int grid, hipStream_t s) {
  switch (kdim) {
    case 32: return launch_c<TIn, 32>(a, c, bv, grid, s);
    case 64: return launch_c<TIn, 64>(a, c, bv, grid, s);
    case 128: return launch_c<TIn, 128>(a, c, bv, grid, s);
    case 256: return launch_c<TIn, 256>(a, c, bv, grid, s);
    default: return GDN_ERR_UNSUPPORTED;
  }
}

// Whether (dtype, K, C, BV) has an instantiated kernel.
inline bool supported(int dtype, int K, int C, int BV) {
  auto f = [&](auto tag) -> bool {
    using TIn = decltype(tag);
    auto byk = [&](auto kc) -> bool {
      constexpr int KK = decltype(kc)::value;
      auto byc = [&](auto cc) -> bool {
        constexpr int CC = decltype(cc)::value;
        switch (BV) {
          case 16: return fits<TIn, KK, CC, 16>();
          case 32: return fits<TIn, KK, CC, 32>();
          case 64: return fits<TIn, KK, CC, 64>();
          default: return false;
        }
      };
      if (C == 32) return byc(std::integral_constant<int, 32>{});
      if (C == 64) return byc(std::integral_constant<int, 64>{});
      return false;
    };
    switch (K) {
      case 32: return byk(std::integral_constant<int, 32>{});
      case 64: return byk(std::integral_constant<int, 64>{});
      case 128: return byk(std::integral_constant<int, 128>{});
      case 256: return byk(std::integral_constant<int, 256>{});
      default: return false;
    }
  };
  if (dtype == GDN_DTYPE_F32) return f(float{});
  if (dtype == GDN_DTYPE_F16) return f(f16{});
  if (dtype == GDN_DTYPE_BF16) return f(bf16_t{});
  return false;
}

// Per-dtype launchers, each defined in its own translation unit
// (gdn_fwd_f16.hip, gdn_fwd_bf16.hip, gdn_fwd_f32.hip) so they compile in
// parallel.
int launch_f16(const KArgs& a, int K, int C, int bv, int grid, hipStream_t s);
int launch_bf16(const KArgs& a, int K, int C, int bv, int grid, hipStream_t s);
int launch_f32(const KArgs& a, int K, int C, int bv, int grid, hipStream_t s);
// The pipelined kernel (gdn_fwd_pipe.h) covers fp16/bf16 inputs, C = 32,
// K in {64, 128}, BV in {16, 32}; everything else runs the phased kernel.
inline bool pipe_supported(int dtype, int K, int C, int BV) {
  return (dtype == GDN_DTYPE_F16 || dtype == GDN_DTYPE_BF16) && C == 32 && (K == 64 || K == 128) &&
         (BV == 16 || BV == 32);
}
int launch_pipe_f16(const KArgs& a, int K, int bv, int grid, hipStream_t s);
int launch_pipe_bf16(const KArgs& a, int K, int bv, int grid, hipStream_t s);
// 64-row chunks with K in {32, 64, 128} run as two launches (gdn_fwd_c64.hip)
// over a caller-owned workspace of per-chunk records.
bool c64_supported(int K, int C, int V);
// 64-row chunks: chunks per (sequence, head) whose records the default
// workspace holds; longer sequences run in segments of this many chunks.
constexpr int64_t kSegC64 = 64;
int64_t c64_record_bytes(int K, int qkv_dtype);
int64_t c64_workspace_size(int B, int T, int H, int K, int n_seq, int qkv_dtype);
int c64_launch(const GdnFwdParams& P, int seg_chunks, hipStream_t stream);
// 32-row chunks, fp16 or bf16 (V / 16 <= 156), K in {64, 128}, BV in {16, 32}: per-chunk records
// then the scan (gdn_fwd_scan32.hip), in segments of at most seg_chunks
// chunks per sequence whose records fit the caller's workspace.
bool scan32_supported(int dtype, int K, int C, int BV, int V);
int64_t scan32_record_bytes(int dtype, int K);  // per (chunk, head)
int scan32_launch(const GdnFwdParams& P, int bv, int seg_chunks, hipStream_t stream);

}  // namespace gdn
